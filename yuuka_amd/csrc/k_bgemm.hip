// k_bgemm.hip — verify GEMM for many rows (batched requests, 9..512 rows):
//
//   out_s[m, n] = epi( sum_k y[m, k] * dequant(W_s)[n, k] )
//
// with the prologues and epilogues of the fused verify GEMM (fgemm.h:
// RMSNorm or gated head norm of x, store / residual / SwiGLU, output maps).
// At a few rows the fused streaming kernel reads every weight once per
// launch; a batch of B requests x (k+1) rows would read them once per 8-row
// block. Here each weight super-block is read once per 64 rows:
//
//  * prologue (one workgroup per row): y = prologue(x) computed as the
//    reference computes it (forward.go:460-482 rmsNorm, recurrent.go:39-50
//    gated norm), then quantized per 256-element super-block into an int16
//    split into two int8 planes (q = 256 h + l, |q| <= 32639), one scale per
//    (row, super-block) and the exact int32 sums of every 32-element
//    sub-block (Q4_K min term) — a workspace of rows * (2K + K/8 + K/64) B.
//  * GEMM (workgroup = 64 rows x 8 tiles of 16 output channels, one tile per
//    wave): per super-block the workgroup stages the 64 rows' planes in LDS
//    in MFMA operand order; each wave decodes its tile's weights straight
//    from HBM into MFMA B operands (Q4_K: one v_mfma_i32_16x16x32_i8 per
//    32-element sub-block; Q6_K: two, one per 16-element scale group) while
//    the next super-block's weights are in flight, and multiplies them with
//    the eight 8-row A tiles (high planes in MFMA rows 0..7, low planes in
//    8..15). Sub-block scales are applied in int32 (exact), d / dmin and the
//    activation scale per super-block in FP32.
//
// Replaces, for batched verify shapes, the reference's per-matrix GEMV
// launches over all rows (kernels/hip/gemm/lm_head.hip:61-173 with MaxRows 16,
// engine/gpu/plan.go); no reference kernel serves more than 16 rows.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "fgemm.h"
#include "refmath.h"

namespace yk {
namespace {

typedef __attribute__((ext_vector_type(4))) int i32x4;

constexpr int kQ4K = YUUKA_DTYPE_Q4_K;
constexpr int kQ6K = YUUKA_DTYPE_Q6_K;
constexpr int kQMax = 32639;
constexpr int kBgWaves = 8;
constexpr int kBgThreads = 64 * kBgWaves;
constexpr int kBgRows = 64;  // rows per workgroup: 8 A tiles of 8 rows
// LDS of the GEMM, per stage: A planes [8 t][8 j][4 g][16 r][8 B] + sums
// [8 t][8 j][8] int32 + scales [8 t][8] float; two stages. The SwiGLU
// epilogue reuses the first.
constexpr uint32_t kBgLdsA = 8 * 8 * 4 * 16 * 8;
constexpr uint32_t kBgStage = kBgLdsA + 8 * 8 * 8 * 4 + 8 * 8 * 4;  // one stage (double-buffered)
constexpr uint32_t kBgLds = 2 * kBgStage;

struct BgQuant {
    int8_t *planes;  // [rows][K/32][2: high, low][32 B]
    int32_t *sums;   // [rows][K/32]
    float *scales;   // [rows][K/256]
};

__host__ __device__ inline BgQuant bg_view(void *ws, int rows, int K) {
    uint8_t *p = static_cast<uint8_t *>(ws);
    BgQuant q;
    q.planes = reinterpret_cast<int8_t *>(p);
    q.sums = reinterpret_cast<int32_t *>(p + (uint64_t)rows * K * 2);
    q.scales = reinterpret_cast<float *>(p + (uint64_t)rows * K * 2 + (uint64_t)rows * (K / 32) * 4);
    return q;
}

__device__ __forceinline__ double wave_sum_d(double v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// ---------------------------------------------------------------- prologue
__global__ __launch_bounds__(256) void bg_prologue_kernel(const FusedGemmArgs A, BgQuant q) {
    extern __shared__ float ys[];  // [K]
    __shared__ double red[4];
    const int row = blockIdx.x, K = A.K;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const float *x = A.x + (uint64_t)row * K;
    if (A.gate) {
        // gated head norm over heads of 128: x * (scale * w) * gate
        const float *z = A.gate + (uint64_t)row * K;
        for (int h = wave; h < K / 128; h += 4) {
            const float a0 = x[h * 128 + lane], a1 = x[h * 128 + 64 + lane];
            double ss = (double)a0 * (double)a0 + (double)a1 * (double)a1;
            ss = wave_sum_d(ss);
            const float mean = (float)(ss / 128.0);
            const float scale = (float)(1.0 / sqrt((double)(mean + A.eps)));
            ys[h * 128 + lane] = __fmul_rn(__fmul_rn(a0, __fmul_rn(scale, A.head_norm[lane])), z[h * 128 + lane]);
            ys[h * 128 + 64 + lane] =
                __fmul_rn(__fmul_rn(a1, __fmul_rn(scale, A.head_norm[64 + lane])), z[h * 128 + 64 + lane]);
        }
    } else if (A.norm) {
        // forward.go:460-470 rmsNorm: float64 sum of squares, x * scale * w
        double s = 0.0;
        for (int c = t; c < K; c += 256) s += (double)x[c] * (double)x[c];
        s = wave_sum_d(s);
        if (lane == 0) red[wave] = s;
        __syncthreads();
        s = red[0] + red[1] + red[2] + red[3];
        const float mean = (float)(s / (double)K);
        const float scale = (float)(1.0 / sqrt((double)(mean + A.eps)));
        for (int c = t; c < K; c += 256) ys[c] = __fmul_rn(__fmul_rn(x[c], scale), A.norm[c]);
    } else {
        for (int c = t; c < K; c += 256) ys[c] = x[c];
    }
    __syncthreads();
    const int nsb = K / 256;
    for (int sb = wave; sb < nsb; sb += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(ys + sb * 256 + 4 * lane);
        float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
        const float inv = m > 0.f ? (float)kQMax / m : 0.f;
        const int qv[4] = {(int)rintf(v.x * inv), (int)rintf(v.y * inv), (int)rintf(v.z * inv),
                           (int)rintf(v.w * inv)};
        uint32_t hp = 0, lp = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int h = (qv[i] + 128) >> 8;
            const int l = qv[i] - 256 * h;
            hp |= (uint32_t)(h & 0xff) << (8 * i);
            lp |= (uint32_t)(l & 0xff) << (8 * i);
        }
        const int j = lane >> 3, o = 4 * (lane & 7);
        int8_t *dst = q.planes + (uint64_t)row * K * 2 + (uint64_t)(sb * 8 + j) * 64 + o;
        *reinterpret_cast<uint32_t *>(dst) = hp;
        *reinterpret_cast<uint32_t *>(dst + 32) = lp;
        int sum = qv[0] + qv[1] + qv[2] + qv[3];
        sum += __shfl_xor(sum, 1);
        sum += __shfl_xor(sum, 2);
        sum += __shfl_xor(sum, 4);
        if ((lane & 7) == 0) q.sums[(uint64_t)row * (K / 32) + sb * 8 + j] = sum;
        if (lane == 0) q.scales[(uint64_t)row * nsb + sb] = m > 0.f ? m / (float)kQMax : 0.f;
    }
}

// ---------------------------------------------------------------- GEMM
struct BgArgs {
    FusedGemmArgs f;
    BgQuant q;
    int tiles[kFusedMaxSeg + 1];  // prefix counts of workgroups (8 tiles of 16 channels) per segment
    int cols[kFusedMaxSeg + 1];   // prefix counts of output channels per segment
    int swiglu;
    int splits;                   // K split over grid z; > 1: partial sums to `part`, then bg_reduce_kernel
    float *part;                  // [splits][rows][cols[nseg]]
};

// 24-bit multiply-add (full rate; a 32-bit multiply is quarter rate). Every
// product here fits: MFMA sub-block results |r| < 2^17, scales <= 63,
// sub-block sums |S| < 2^21.
__device__ __forceinline__ int mad24(int a, int b, int c) { return __mul24(a, b) + c; }

__device__ __forceinline__ i32x4 mfma_i8(int64_t a, int64_t b) {
    const i32x4 zero = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, zero, 0, 0, 0);
}

// 8 bytes at an even byte address (Q6_K blocks are 210 B): two dword-aligned
// loads and a byte shift.
__device__ __forceinline__ uint64_t load8_even(const uint8_t *p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t *w = reinterpret_cast<const uint32_t *>(a & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(a & 3);
    const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
    const uint32_t lo = __builtin_amdgcn_alignbyte(w1, w0, sh);
    const uint32_t hi = __builtin_amdgcn_alignbyte(w2, w1, sh);
    return (uint64_t)lo | ((uint64_t)hi << 32);
}

// Signed q - 32 for eight packed unsigned 6-bit values (one per byte).
__device__ __forceinline__ uint64_t q6_to_i8(uint64_t q6) {
    const uint64_t t = q6 ^ 0x2020202020202020ull;
    const uint64_t s = t & 0x2020202020202020ull;
    return t | (s << 1) | (s << 2);
}

// One super-block of one channel, as lane (c, g) needs it.
struct WQ4 {
    uint4 hdr;       // d, dmin, 12 scale bytes
    uint64_t q[4];   // bytes [32 p + 8 g, +8) of the 128 quant bytes
};
struct WQ6 {
    uint64_t ql[4];  // ql bytes [64 half + 32 p + 8 g, +8), index 2 half + p
    uint64_t qh[2];  // qh bytes [32 half + 8 g, +8)
    uint4 sc;        // 16 int8 scales
    uint32_t d;      // fp16 d in the low half
};

__device__ __forceinline__ void load_q4(WQ4 &w, const uint8_t *blk, int g) {
    w.hdr = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
    for (int p = 0; p < 4; p++) w.q[p] = *reinterpret_cast<const uint64_t *>(blk + 16 + 32 * p + 8 * g);
}

__device__ __forceinline__ void load_q6(WQ6 &w, const uint8_t *blk, int g) {
#pragma unroll
    for (int i = 0; i < 4; i++) w.ql[i] = load8_even(blk + 64 * (i >> 1) + 32 * (i & 1) + 8 * g);
#pragma unroll
    for (int h = 0; h < 2; h++) w.qh[h] = load8_even(blk + 128 + 32 * h + 8 * g);
    // the block's last 18 bytes by 2-byte loads: nothing past byte 210 is read
    const uint64_t s01 = load8_even(blk + 192);
    const uint16_t *t = reinterpret_cast<const uint16_t *>(blk + 200);
    w.sc.x = (uint32_t)s01;
    w.sc.y = (uint32_t)(s01 >> 32);
    w.sc.z = (uint32_t)t[0] | ((uint32_t)t[1] << 16);
    w.sc.w = (uint32_t)t[2] | ((uint32_t)t[3] << 16);
    w.d = t[4];
}

__device__ __forceinline__ int sbyte(const uint4 &v, int i) {
    const uint32_t w = i < 4 ? v.x : (i < 8 ? v.y : (i < 12 ? v.z : v.w));
    return (int)(int8_t)((w >> (8 * (i & 3))) & 0xff);
}

// tensor/quant.go:96-103 getScaleMinK4 for sub-block j (scale bytes in
// words s1, s2, s3 = block bytes 4..15).
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s1, uint32_t s2, uint32_t s3, int *sc, int *mn) {
    if (j < 4) {
        *sc = (s1 >> (8 * j)) & 63;
        *mn = (s2 >> (8 * j)) & 63;
    } else {
        const int k = j - 4;
        const uint32_t a = (s1 >> (8 * k)) & 0xff, b = (s2 >> (8 * k)) & 0xff, cc = (s3 >> (8 * k)) & 0xff;
        *sc = (int)((cc & 0xF) | ((a >> 6) << 4));
        *mn = (int)((cc >> 4) | ((b >> 6) << 4));
    }
}

__device__ __forceinline__ int seg_of(const BgArgs &A, int tile) {
    int s = 0;
#pragma unroll
    for (int i = 1; i < kFusedMaxSeg; i++)
        if (i < A.f.nseg && tile >= A.tiles[i]) s = i;
    return s;
}

__device__ __forceinline__ float out_map(const FusedSeg &S, int n, float v) {
    switch (S.act) {
    case 1: return silu_ref(v);
    case 2: return sigmoid_ref(v);
    case 3: return (float)exp((double)__fmul_rn(softplus_ref(__fadd_rn(v, S.p0[n])), S.p1[n]));
    default: return v;
    }
}

// Super-block sb of the workgroup's rows (planes, sums, scales): loaded by
// every thread into registers, then written to one of two LDS buffers.
struct Staged {
    uint4 v[4];
    int32_t sum;
    float xs;
};

__device__ __forceinline__ void stage_load(const BgArgs &A, Staged &st, int m0, int mrows, int sb) {
    const int K = A.f.K, nsb = K / 256, nsub = K / 32;
#pragma unroll
    for (int u = 0; u < 4; u++) {  // piece = (row, sub-block, plane, 16-byte half)
        const int idx = threadIdx.x + u * kBgThreads;
        const int r = idx >> 5, j = (idx >> 2) & 7, p = (idx >> 1) & 1, half = idx & 1;
        st.v[u] = r < mrows ? *reinterpret_cast<const uint4 *>(A.q.planes + (uint64_t)(m0 + r) * K * 2 +
                                                               (uint64_t)(sb * 8 + j) * 64 + 32 * p + 16 * half)
                            : make_uint4(0u, 0u, 0u, 0u);
    }
    {
        const int r = threadIdx.x >> 3, j = threadIdx.x & 7;
        st.sum = r < mrows ? A.q.sums[(uint64_t)(m0 + r) * nsub + sb * 8 + j] : 0;
    }
    st.xs = threadIdx.x < mrows ? A.q.scales[(uint64_t)(m0 + threadIdx.x) * nsb + sb] : 0.f;
}

// LDS byte offset of the 8 A bytes of tile t (8 rows, two planes), sub-block
// j, lane group gg, MFMA row rr: sub-blocks 2 jp and 2 jp + 1 sit side by side,
// so one 16-byte read gives a lane both halves of a K = 64 operand.
__device__ __forceinline__ uint32_t la_off(int t, int j, int gg, int rr) {
    return ((uint32_t)(((t * 4 + (j >> 1)) * 4 + gg) * 16 + rr) * 2 + (j & 1)) * 8;
}

__device__ __forceinline__ void stage_store(const Staged &st, uint8_t *la, int32_t *lsum, float *lxs) {
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int idx = threadIdx.x + u * kBgThreads;
        const int r = idx >> 5, j = (idx >> 2) & 7, p = (idx >> 1) & 1, half = idx & 1;
        const int t = r >> 3, rr = (r & 7) + 8 * p;
        uint8_t *d0 = la + la_off(t, j, 2 * half, rr);
        *reinterpret_cast<uint2 *>(d0) = make_uint2(st.v[u].x, st.v[u].y);
        *reinterpret_cast<uint2 *>(d0 + 256) = make_uint2(st.v[u].z, st.v[u].w);
    }
    {
        const int r = threadIdx.x >> 3, j = threadIdx.x & 7;
        lsum[((r >> 3) * 8 + j) * 8 + (r & 7)] = st.sum;
    }
    if (threadIdx.x < kBgRows) lxs[threadIdx.x] = st.xs;
}

// The main loop of one wave over the super-blocks (weights of dtype DT).
// LDS holds two stages; stage sb + 1 is loaded while sb is multiplied.
template <int DT>
__device__ __forceinline__ void bg_main(const BgArgs &A, uint8_t *lds, int m0, int mrows, bool live,
                                        const uint8_t *wrow, float (&y)[8][4]) {
    const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
    // this split's super-blocks [sb_lo, nsb)
    const int nsb_all = A.f.K / 256;
    const int sb_lo = (int)((int64_t)nsb_all * blockIdx.z / A.splits);
    const int nsb = (int)((int64_t)nsb_all * (blockIdx.z + 1) / A.splits);
    wrow += (uint64_t)sb_lo * (DT == kQ4K ? 144 : 210);
    const int rb = 4 * (g & 1);
    typedef typename std::conditional<DT == kQ4K, WQ4, WQ6>::type W;
    constexpr int blk = DT == kQ4K ? 144 : 210;
    W w{};
    if (live) {
        if constexpr (DT == kQ4K) load_q4(w, wrow, g);
        else load_q6(w, wrow, g);
    }
    Staged st;
    stage_load(A, st, m0, mrows, sb_lo);
    stage_store(st, lds, reinterpret_cast<int32_t *>(lds + kBgLdsA), reinterpret_cast<float *>(lds + kBgLdsA + 2048));
    __syncthreads();
    for (int sb = sb_lo; sb < nsb; sb++) {
        uint8_t *cur_l = lds + (uint32_t)((sb - sb_lo) & 1) * kBgStage;
        uint8_t *nxt_l = lds + (uint32_t)((sb - sb_lo + 1) & 1) * kBgStage;
        const uint8_t *la = cur_l;
        const int32_t *lsum = reinterpret_cast<const int32_t *>(cur_l + kBgLdsA);
        const float *lxs = reinterpret_cast<const float *>(cur_l + kBgLdsA + 2048);
        const bool more = sb + 1 < nsb;
        if (more) stage_load(A, st, m0, mrows, sb + 1);
        const W cur = w;  // this super-block; the next one's loads go out now
        if (live && more) {
            if constexpr (DT == kQ4K) load_q4(w, wrow + (uint64_t)(sb + 1 - sb_lo) * blk, g);
            else load_q6(w, wrow + (uint64_t)(sb + 1 - sb_lo) * blk, g);
        }
        if (live) {
            if constexpr (DT == kQ4K) {
                // Scale and min term on the MFMA accumulators: with sc = 8 sc_hi
                // + sc_lo (3-bit digits), q * sc_lo and q * sc_hi (<= 105) are
                // exact int8 B operands, and the sub-block min m (<= 63)
                // broadcast over the sub-block gives the min term directly. A
                // K = 64 MFMA covers sub-blocks 2 jp and 2 jp + 1 (low and high
                // nibbles of the same quant bytes): three chained MFMAs per
                // sub-block pair and 8-row tile, no VALU multiply-adds. Two
                // passes of four A tiles bound the registers.
                const float d = h2f((uint16_t)(cur.hdr.x & 0xffffu)), dmin = h2f((uint16_t)(cur.hdr.x >> 16));
#pragma unroll
                for (int th = 0; th < 2; th++) {
                    i32x4 alo[4], ahi[4], amn[4];
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        alo[u] = i32x4{0, 0, 0, 0};
                        ahi[u] = i32x4{0, 0, 0, 0};
                        amn[u] = i32x4{0, 0, 0, 0};
                    }
#pragma unroll
                    for (int jp = 0; jp < 4; jp++) {
                        const uint64_t raw = cur.q[jp];
                        const uint64_t qe = raw & 0x0F0F0F0F0F0F0F0Full, qo = (raw >> 4) & 0x0F0F0F0F0F0F0F0Full;
                        int sce, mne, sco, mno;
                        scale_min_k4(2 * jp, cur.hdr.y, cur.hdr.z, cur.hdr.w, &sce, &mne);
                        scale_min_k4(2 * jp + 1, cur.hdr.y, cur.hdr.z, cur.hdr.w, &sco, &mno);
                        // per-byte products stay below 256: no carries between bytes
                        const uint32_t q[4] = {(uint32_t)qe, (uint32_t)(qe >> 32), (uint32_t)qo, (uint32_t)(qo >> 32)};
                        const uint32_t lo[2] = {(uint32_t)(sce & 7), (uint32_t)(sco & 7)};
                        const uint32_t hi[2] = {(uint32_t)(sce >> 3), (uint32_t)(sco >> 3)};
                        const i32x4 b_lo = {(int)(q[0] * lo[0]), (int)(q[1] * lo[0]), (int)(q[2] * lo[1]), (int)(q[3] * lo[1])};
                        const i32x4 b_hi = {(int)(q[0] * hi[0]), (int)(q[1] * hi[0]), (int)(q[2] * hi[1]), (int)(q[3] * hi[1])};
                        const int me = (int)((uint32_t)mne * 0x01010101u), mo = (int)((uint32_t)mno * 0x01010101u);
                        const i32x4 b_mn = {me, me, mo, mo};
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            const int t = 4 * th + u;
                            const i32x4 av = *reinterpret_cast<const i32x4 *>(la + la_off(t, 2 * jp, g, c));
                            alo[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b_lo, alo[u], 0, 0, 0);
                            ahi[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b_hi, ahi[u], 0, 0, 0);
                            amn[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b_mn, amn[u], 0, 0, 0);
                        }
                    }
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int t = 4 * th + u;
                        const float4 xs = *reinterpret_cast<const float4 *>(lxs + t * 8 + rb);
                        const float xsv[4] = {xs.x, xs.y, xs.z, xs.w};
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            // this lane's plane (rows 0..7 high, 8..15 low), then both
                            const float v = d * (float)(alo[u][i] + 8 * ahi[u][i]) - dmin * (float)amn[u][i];
                            const float other = __shfl_xor(v, 32);
                            y[t][i] += xsv[i] * (256.f * v + other);
                        }
                    }
                }
            } else {
                const float d = h2f((uint16_t)cur.d);
                int64_t bq[8];
                int sc2[8];  // scales of elements 0..15 (low half) and 16..31 (high half) of sub-block j
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int half = j >> 2, qd = j & 3;
                    const uint64_t lo4 = (cur.ql[2 * half + (qd & 1)] >> (4 * (qd >> 1))) & 0x0F0F0F0F0F0F0F0Full;
                    const uint64_t hi2 = ((cur.qh[half] >> (2 * qd)) & 0x0303030303030303ull) << 4;
                    bq[j] = (int64_t)q6_to_i8(lo4 | hi2);
                    sc2[j] = (sbyte(cur.sc, 8 * half + 2 * qd) & 0xffff) | (sbyte(cur.sc, 8 * half + 2 * qd + 1) << 16);
                }
#pragma unroll
                for (int t = 0; t < 8; t++) {  // all 8 tiles: rows past the end are zero in LDS
                    int acc[4] = {0, 0, 0, 0};
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const int64_t a = *reinterpret_cast<const int64_t *>(la + la_off(t, j, g, c));
                        // lanes g < 2 hold elements 0..15 (first scale group)
                        const i32x4 r0 = mfma_i8(a, g < 2 ? bq[j] : 0);
                        const i32x4 r1 = mfma_i8(a, g < 2 ? 0 : bq[j]);
                        const int s0 = (int)(int16_t)(sc2[j] & 0xffff), s1 = sc2[j] >> 16;
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[i] = mad24(r1[i], s1, mad24(r0[i], s0, acc[i]));
                    }
                    const float4 xs = *reinterpret_cast<const float4 *>(lxs + t * 8 + rb);
                    const float xsv[4] = {xs.x, xs.y, xs.z, xs.w};
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int lo = __shfl_xor(acc[i], 32);
                        y[t][i] += xsv[i] * (d * (256.f * (float)acc[i] + (float)lo));
                    }
                    __builtin_amdgcn_sched_barrier(0);  // one A tile at a time (register pressure)
                }
            }
        }
        if (more)
            stage_store(st, nxt_l, reinterpret_cast<int32_t *>(nxt_l + kBgLdsA),
                        reinterpret_cast<float *>(nxt_l + kBgLdsA + 2048));
        __syncthreads();  // stage sb + 1 written; stage sb read by every wave
    }
}

__global__ __launch_bounds__(kBgThreads) void bg_gemm_kernel(const BgArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const FusedGemmArgs &F = A.f;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.y * kBgRows;
    const int mrows = min(kBgRows, F.rows - m0);

    // this wave's tile: the workgroup's segment (segments start on whole
    // workgroups, so a workgroup has one weight type) and tile 8 w + wave, or
    // (SwiGLU) waves 0..3 gate tiles and 4..7 the same up tiles
    int tile, seg;
    if (A.swiglu) {
        tile = blockIdx.x * 4 + (wave & 3);
        seg = wave >> 2;
    } else {
        seg = seg_of(A, blockIdx.x);
        tile = (blockIdx.x - A.tiles[seg]) * kBgWaves + wave;
    }
    const FusedSeg &S = F.seg[seg];
    const int n0 = tile * 16;
    const bool live = n0 < S.n;
    const int n = min(n0 + c, S.n - 1);  // clamped channel for the loads
    const uint8_t *wrow = static_cast<const uint8_t *>(S.w) + (uint64_t)n * S.row_bytes;

    float y[8][4];
#pragma unroll
    for (int t = 0; t < 8; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) y[t][i] = 0.f;
    if (S.dtype == kQ6K)
        bg_main<kQ6K>(A, lds, m0, mrows, live, wrow, y);
    else
        bg_main<kQ4K>(A, lds, m0, mrows, live, wrow, y);

    // epilogue: lanes g < 2 hold rows 8 t + 4 g + i of channel n0 + c
    if (A.splits > 1) {  // partial sums of this split; bg_reduce_kernel finishes
        if (!live || g >= 2 || n0 + c >= S.n) return;
        const int ncol = A.cols[F.nseg];
        float *pp = A.part + (uint64_t)blockIdx.z * F.rows * ncol + A.cols[seg] + n0 + c;
#pragma unroll
        for (int t = 0; t < 8; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = 8 * t + 4 * g + i;
                if (r < mrows) pp[(uint64_t)(m0 + r) * ncol] = y[t][i];
            }
        return;
    }
    if (A.swiglu) {
        __syncthreads();
        float *up = reinterpret_cast<float *>(lds);  // [4 tiles][64 rows][16]
        if (wave >= 4 && g < 2) {
#pragma unroll
            for (int t = 0; t < 8; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) up[((wave - 4) * kBgRows + 8 * t + 4 * g + i) * 16 + c] = y[t][i];
        }
        __syncthreads();
        if (wave < 4 && g < 2 && live && n0 + c < S.n) {
#pragma unroll
            for (int t = 0; t < 8; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 8 * t + 4 * g + i;
                    if (r >= mrows) continue;
                    const float u = up[(wave * kBgRows + r) * 16 + c];
                    S.out[(uint64_t)(m0 + r) * S.n + n0 + c] = __fmul_rn(silu_ref(y[t][i]), u);
                }
        }
        return;
    }
    if (!live || g >= 2 || n0 + c >= S.n) return;
#pragma unroll
    for (int t = 0; t < 8; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 8 * t + 4 * g + i;
            if (r >= mrows) continue;
            const uint64_t o = (uint64_t)(m0 + r) * S.n + n0 + c;
            float v = y[t][i];
            if (F.epilogue == kEpiResidual) v = __fadd_rn(v, S.res[o]);
            else v = out_map(S, n0 + c, v);
            S.out[o] = v;
        }
}

// Sum of the splits in split order, then the epilogue (one thread per output).
__global__ __launch_bounds__(256) void bg_reduce_kernel(const BgArgs A) {
    const FusedGemmArgs &F = A.f;
    const int ncol = A.cols[F.nseg];
    const int nout = A.swiglu ? F.seg[0].n : ncol;
    const uint64_t idx = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (uint64_t)F.rows * nout) return;
    const int m = (int)(idx / nout), col = (int)(idx % nout);
    auto sum = [&](int cc) {
        float v = 0.f;
        for (int sp = 0; sp < A.splits; sp++) v += A.part[((uint64_t)sp * F.rows + m) * ncol + cc];
        return v;
    };
    if (A.swiglu) {
        const float gsum = sum(col), usum = sum(A.cols[1] + col);
        F.seg[0].out[(uint64_t)m * F.seg[0].n + col] = __fmul_rn(silu_ref(gsum), usum);
        return;
    }
    int seg = 0;
    for (int i = 1; i < F.nseg; i++)
        if (col >= A.cols[i]) seg = i;
    const FusedSeg &S = F.seg[seg];
    const int n = col - A.cols[seg];
    const uint64_t o = (uint64_t)m * S.n + n;
    float v = sum(col);
    if (F.epilogue == kEpiResidual) v = __fadd_rn(v, S.res[o]);
    else v = out_map(S, n, v);
    S.out[o] = v;
}

// K splits that bring a small launch near two workgroups per CU.
int bg_splits(int wgs, int nsb) {
    int sp = (512 + wgs - 1) / wgs;
    sp = std::min(sp, std::max(1, nsb / 2));
    return std::max(1, std::min(sp, 16));
}

uint64_t bg_quant_bytes(int rows, int K) {
    return (uint64_t)rows * K * 2 + (uint64_t)rows * (K / 32) * 4 + (uint64_t)rows * (K / 256) * 4;
}

}  // namespace

// Grid of one launch: x workgroups of 8 tiles (SwiGLU: 4 channel tiles of
// both matrices), y row blocks, z K splits.
static void bg_grid(const int *n, int nseg, bool swiglu, int rows, int K, unsigned *gx, unsigned *gy, int *splits) {
    unsigned x = 0;
    if (swiglu)
        x = (unsigned)((n[0] + 63) / 64);
    else
        for (int i = 0; i < nseg; i++) x += (unsigned)((n[i] + 16 * kBgWaves - 1) / (16 * kBgWaves));
    *gx = x;
    *gy = (unsigned)((rows + kBgRows - 1) / kBgRows);
    *splits = getenv("YUUKA_BG_NOSPLIT") ? 1 : bg_splits((int)(x * *gy), K / 256);
}

uint64_t fused_gemm_rows_ws(int rows, int K, const int *n, int nseg, bool swiglu) {
    unsigned gx, gy;
    int splits;
    bg_grid(n, nseg, swiglu, rows, K, &gx, &gy, &splits);
    int ncol = 0;
    for (int i = 0; i < nseg; i++) ncol += n[i];
    const uint64_t part = splits > 1 ? (uint64_t)splits * rows * ncol * 4 : 0;
    return ((bg_quant_bytes(rows, K) + 255) & ~255ull) + part + 256;
}

hipError_t launch_fused_gemm_rows(const FusedGemmArgs &a, void *ws, hipStream_t s) {
    BgArgs A{};
    A.f = a;
    A.q = bg_view(ws, a.rows, a.K);
    A.swiglu = a.epilogue == kEpiSwiglu ? 1 : 0;
    // segment prefix in workgroups of 8 tiles (a workgroup never straddles two segments)
    A.tiles[0] = 0;
    for (int i = 0; i < a.nseg; i++) A.tiles[i + 1] = A.tiles[i] + (a.seg[i].n + 16 * kBgWaves - 1) / (16 * kBgWaves);
    for (int i = a.nseg + 1; i <= kFusedMaxSeg; i++) A.tiles[i] = A.tiles[a.nseg];
    const uint32_t plds = (uint32_t)a.K * 4;
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(bg_prologue_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 64 * 1024);
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(bg_gemm_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)kBgLds);
        attr = true;
    }
    bg_prologue_kernel<<<(unsigned)a.rows, 256, plds, s>>>(a, A.q);
    int nn[kFusedMaxSeg];
    for (int i = 0; i < a.nseg; i++) nn[i] = a.seg[i].n;
    unsigned gx, gy;
    bg_grid(nn, a.nseg, A.swiglu != 0, a.rows, a.K, &gx, &gy, &A.splits);
    A.cols[0] = 0;
    for (int i = 0; i < a.nseg; i++) A.cols[i + 1] = A.cols[i] + a.seg[i].n;
    for (int i = a.nseg + 1; i <= kFusedMaxSeg; i++) A.cols[i] = A.cols[a.nseg];
    A.part = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) + ((bg_quant_bytes(a.rows, a.K) + 255) & ~255ull));
    bg_gemm_kernel<<<dim3(gx, gy, (unsigned)A.splits), kBgThreads, kBgLds, s>>>(A);
    if (A.splits > 1) {
        const uint64_t nout = (uint64_t)a.rows * (A.swiglu ? a.seg[0].n : A.cols[a.nseg]);
        bg_reduce_kernel<<<(unsigned)((nout + 255) / 256), 256, 0, s>>>(A);
    }
    return hipGetLastError();
}

}  // namespace yk
