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
//    split into two int8 planes (q = 256 h + l, |q| <= 32639) and one scale
//    per (row, super-block) — a workspace of rows * (2K + K/64) B.
//  * GEMM (workgroup = 64 rows x 8 tiles of 16 output channels, one tile per
//    wave): per super-block the workgroup stages the 64 rows' planes in LDS
//    in MFMA operand order; each wave decodes its tile's weights straight
//    from HBM into MFMA B operands while the next super-block's weights are
//    in flight, and multiplies them with the eight 8-row A tiles (high planes
//    in MFMA rows 0..7, low planes in 8..15). Q4_K: the 6-bit sub-block scale
//    and min ride in the B operands (three v_mfma_i32_16x16x64_i8 per pair of
//    sub-blocks); Q6_K: two v_mfma_i32_16x16x32_i8 per sub-block (one per
//    16-element scale group), scales applied in int32. Everything up to the
//    super-block is exact integer; d / dmin and the activation scale are
//    applied per super-block in FP32.
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
// LDS of the GEMM, per stage: A planes [8 t][4 jp][4 g][16 r][2][8 B] +
// scales [8 t][8] float; two stages. The SwiGLU epilogue reuses the first.
constexpr uint32_t kBgLdsA = 8 * 8 * 4 * 16 * 8;
constexpr uint32_t kBgStage = kBgLdsA + 8 * 8 * 4;  // one stage (double-buffered)
constexpr uint32_t kBgLds = 2 * kBgStage;

struct BgQuant {
    int8_t *planes;  // [rows][K/32][2: high, low][32 B]
    float *scales;   // [rows][K/256]
};

__host__ __device__ inline BgQuant bg_view(void *ws, int rows, int K) {
    uint8_t *p = static_cast<uint8_t *>(ws);
    BgQuant q;
    q.planes = reinterpret_cast<int8_t *>(p);
    q.scales = reinterpret_cast<float *>(p + (uint64_t)rows * K * 2);
    return q;
}

// Reductions on the DPP path (a __shfl_xor is an LDS permute): within each
// 16-lane row (lane pairs, quads, half rows, rows), then the rows' results
// through readlane.
template <int C>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, C, 0xf, 0xf, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), C, 0xf, 0xf, true);
    return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}
__device__ __forceinline__ double rl_d(double v, int l) {
    const uint64_t b = __double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double row16_sum_d(double v) {  // every lane: its 16-lane row's sum
    v += dpp_d<0xb1>(v);
    v += dpp_d<0x4e>(v);
    v += dpp_d<0x141>(v);
    return v + dpp_d<0x140>(v);
}
__device__ __forceinline__ double wave_sum_d(double v) {
    v = row16_sum_d(v);
    return (rl_d(v, 0) + rl_d(v, 16)) + (rl_d(v, 32) + rl_d(v, 48));
}
// Maximum of non-negative values over the wave.
__device__ __forceinline__ float wave_max_nonneg(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, true)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, true)));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// ---------------------------------------------------------------- prologue
constexpr int kPrThreads = 512;

__global__ __launch_bounds__(kPrThreads) void bg_prologue_kernel(const FusedGemmArgs A, BgQuant q) {
    extern __shared__ float ys[];  // [K]: x, then y
    __shared__ double red[kPrThreads / 64];
    const int row = blockIdx.x, K = A.K;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    // x into LDS with independent 16-byte loads (the float64 sum of squares
    // for RMSNorm on the way)
    const float4 *x4 = reinterpret_cast<const float4 *>(A.x + (uint64_t)row * K);
    double ss = 0.0;
#pragma unroll 4
    for (int c = t; c < K / 4; c += kPrThreads) {
        const float4 v = x4[c];
        *reinterpret_cast<float4 *>(ys + 4 * c) = v;
        ss += (double)v.x * (double)v.x + (double)v.y * (double)v.y + (double)v.z * (double)v.z +
              (double)v.w * (double)v.w;
    }
    float nscale = 1.f;
    if (A.norm) {
        // forward.go:460-470 rmsNorm: float64 sum of squares, x * scale * w
        ss = wave_sum_d(ss);
        if (lane == 0) red[wave] = ss;
    }
    __syncthreads();
    if (A.norm) {
        double s = 0.0;
#pragma unroll
        for (int w = 0; w < kPrThreads / 64; w++) s += red[w];
        const float mean = (float)(s / (double)K);
        nscale = (float)(1.0 / sqrt((double)(mean + A.eps)));
    }
    const int nsb = K / 256;
#pragma unroll 2
    for (int sb = wave; sb < nsb; sb += kPrThreads / 64) {
        const int e = sb * 256 + 4 * lane;
        float4 v = *reinterpret_cast<const float4 *>(ys + e);
        if (A.gate) {
            // recurrent.go:39-50 gated head norm over heads of 128 (lanes 0..31
            // and 32..63 hold one head each): x * (scale * w) * gate
            const float4 z = *reinterpret_cast<const float4 *>(A.gate + (uint64_t)row * K + e);
            const float4 w = *reinterpret_cast<const float4 *>(A.head_norm + (e & 127));
            double hs = (double)v.x * (double)v.x + (double)v.y * (double)v.y + (double)v.z * (double)v.z +
                        (double)v.w * (double)v.w;
            hs = row16_sum_d(hs);  // each 128-element head is two 16-lane rows
            hs = lane < 32 ? rl_d(hs, 0) + rl_d(hs, 16) : rl_d(hs, 32) + rl_d(hs, 48);
            const float mean = (float)(hs / 128.0);
            const float hsc = (float)(1.0 / sqrt((double)(mean + A.eps)));
            v.x = __fmul_rn(__fmul_rn(v.x, __fmul_rn(hsc, w.x)), z.x);
            v.y = __fmul_rn(__fmul_rn(v.y, __fmul_rn(hsc, w.y)), z.y);
            v.z = __fmul_rn(__fmul_rn(v.z, __fmul_rn(hsc, w.z)), z.z);
            v.w = __fmul_rn(__fmul_rn(v.w, __fmul_rn(hsc, w.w)), z.w);
        } else if (A.norm) {
            const float4 w = *reinterpret_cast<const float4 *>(A.norm + e);
            v.x = __fmul_rn(__fmul_rn(v.x, nscale), w.x);
            v.y = __fmul_rn(__fmul_rn(v.y, nscale), w.y);
            v.z = __fmul_rn(__fmul_rn(v.z, nscale), w.z);
            v.w = __fmul_rn(__fmul_rn(v.w, nscale), w.w);
        }
        float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
        m = wave_max_nonneg(m);
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

// 24-bit multiply-add (full rate; a 32-bit multiply is quarter rate). Used
// for the Q6_K digit recombination 49 a2 + 7 a1 + a0, where |a| < 2^22.
__device__ __forceinline__ int mad24(int a, int b, int c) { return __mul24(a, b) + c; }

typedef __attribute__((ext_vector_type(2))) unsigned short u16x2;

// Every byte of q times k, for byte products below 256: one packed 16-bit
// multiply (b0 + 256 b1) k = b0 k + 256 b1 k per half, no carry between bytes.
__device__ __forceinline__ uint32_t bytes_times(uint32_t q, uint32_t k) {
    const u16x2 b = {(unsigned short)k, (unsigned short)k};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, q) * b);
}

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

// Super-block sb of the workgroup's rows (planes, scales): loaded by
// every thread into registers, then written to one of two LDS buffers.
struct Staged {
    uint4 v[4];
    float xs;
};

// LDS byte offset of the 8 A bytes of tile t (8 rows, two planes), sub-block
// j, lane group gg, MFMA row rr: sub-blocks 2 jp and 2 jp + 1 sit side by side,
// so one 16-byte read gives a lane both halves of a K = 64 operand.
__device__ __forceinline__ uint32_t la_off(int t, int j, int gg, int rr) {
    return ((uint32_t)(((t * 4 + (j >> 1)) * 4 + gg) * 16 + rr) * 2 + (j & 1)) * 8;
}

// Thread piece u = ((t * 8 + j) * 2 + half) * 16 + rr (four per thread):
// bytes [16 half, 16 half + 16) of plane rr >> 3 of row 8 t + (rr & 7),
// sub-block j: one 16-byte global load (a row's 128 bytes come from 8
// lanes) and two 8-byte LDS writes for lane groups 2 half and 2 half + 1
// that cover every bank.
__device__ __forceinline__ void stage_load(const BgArgs &A, Staged &st, int m0, int mrows, int sb) {
    const int K = A.f.K, nsb = K / 256;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int u = threadIdx.x + k * kBgThreads;
        const int rr = u & 15, half = (u >> 4) & 1, j = (u >> 5) & 7, t = u >> 8;
        const int r = 8 * t + (rr & 7);
        st.v[k] = r < mrows ? *reinterpret_cast<const uint4 *>(A.q.planes + (uint64_t)(m0 + r) * K * 2 +
                                                               (uint64_t)(sb * 8 + j) * 64 + 32 * (rr >> 3) + 16 * half)
                            : make_uint4(0u, 0u, 0u, 0u);
    }
    st.xs = threadIdx.x < mrows ? A.q.scales[(uint64_t)(m0 + threadIdx.x) * nsb + sb] : 0.f;
}

__device__ __forceinline__ void stage_store(const Staged &st, uint8_t *la, float *lxs) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int u = threadIdx.x + k * kBgThreads;
        const int rr = u & 15, half = (u >> 4) & 1, j = (u >> 5) & 7, t = u >> 8;
        uint8_t *d0 = la + la_off(t, j, 2 * half, rr);
        *reinterpret_cast<uint2 *>(d0) = make_uint2(st.v[k].x, st.v[k].y);
        *reinterpret_cast<uint2 *>(d0 + 256) = make_uint2(st.v[k].z, st.v[k].w);
    }
    if (threadIdx.x < kBgRows) lxs[threadIdx.x] = st.xs;
}

// The main loop of one wave over the super-blocks (weights of dtype DT).
// LDS holds two stages; stage sb + 1 is loaded while sb is multiplied.
template <int DT, int TH>
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
    stage_store(st, lds, reinterpret_cast<float *>(lds + kBgLdsA));
    __syncthreads();
    for (int sb = sb_lo; sb < nsb; sb++) {
        uint8_t *cur_l = lds + (uint32_t)((sb - sb_lo) & 1) * kBgStage;
        uint8_t *nxt_l = lds + (uint32_t)((sb - sb_lo + 1) & 1) * kBgStage;
        const uint8_t *la = cur_l;
        const float *lxs = reinterpret_cast<const float *>(cur_l + kBgLdsA);
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
                for (int th = 0; th < TH; th++) {  // TH = 1: rows in tiles 0..3 only
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
                        const i32x4 b_lo = {(int)bytes_times(q[0], lo[0]), (int)bytes_times(q[1], lo[0]),
                                            (int)bytes_times(q[2], lo[1]), (int)bytes_times(q[3], lo[1])};
                        const i32x4 b_hi = {(int)bytes_times(q[0], hi[0]), (int)bytes_times(q[1], hi[0]),
                                            (int)bytes_times(q[2], hi[1]), (int)bytes_times(q[3], hi[1])};
                        // byte 0 in all four bytes (v_perm; a multiply by 0x01010101 is quarter rate)
                        const int me = (int)__builtin_amdgcn_perm((uint32_t)mne, (uint32_t)mne, 0u);
                        const int mo = (int)__builtin_amdgcn_perm((uint32_t)mno, (uint32_t)mno, 0u);
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
                            // this lane's plane (rows 0..7 high, 8..15 low)
                            const float v = d * (float)(alo[u][i] + 8 * ahi[u][i]) - dmin * (float)amn[u][i];
                            y[t][i] += xsv[i] * v;
                        }
                    }
                }
            } else {
                // Q6_K: q = ql | qh << 4 - 32 in [-32, 31] and a signed 8-bit
                // scale per 16 elements, written in balanced base 7
                // (s = e0 + 7 e1 + 49 e2, e in [-3, 3]): every q * e (|.| <= 96)
                // is an exact int8 B operand, so three K = 64 MFMAs per pair of
                // sub-blocks and 8-row tile replace the int32 scaling. A lane's
                // eight bytes of sub-block j lie in one 16-element scale group.
                const float d = h2f((uint16_t)cur.d);
                uint32_t qw[8][2];  // q + 32 (0..63) of sub-block j, bytes 0..3 and 4..7
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    const int half = j >> 2, qd = j & 3;
                    const uint64_t lo4 = (cur.ql[2 * half + (qd & 1)] >> (4 * (qd >> 1))) & 0x0F0F0F0F0F0F0F0Full;
                    const uint64_t hi2 = ((cur.qh[half] >> (2 * qd)) & 0x0303030303030303ull) << 4;
                    qw[j][0] = (uint32_t)(lo4 | hi2);
                    qw[j][1] = (uint32_t)((lo4 | hi2) >> 32);
                }
                // the three digits of this lane's scale for every sub-block,
                // each as (e, -32 e) in both 16-bit halves
                uint32_t dm[8][3], dc[8][3];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    uint32_t u = (uint32_t)(sbyte(cur.sc, 2 * j + (g >> 1)) + 171);  // 43..298
#pragma unroll
                    for (int k = 0; k < 3; k++) {
                        const uint32_t nq = k < 2 ? (u * 9363u) >> 16 : 0u;  // u / 7 for u < 13107
                        const int e = (int)(k < 2 ? u - 7 * nq : u) - 3;
                        // low 16 bits in both halves
                        dm[j][k] = __builtin_amdgcn_perm((uint32_t)e, (uint32_t)e, 0x01000100u);
                        dc[j][k] = __builtin_amdgcn_perm((uint32_t)(-32 * e), (uint32_t)(-32 * e), 0x01000100u);
                        u = nq;
                    }
                }
#pragma unroll
                for (int th = 0; th < TH; th++) {  // TH = 1: rows in tiles 0..3 only
                    i32x4 a0[4], a1[4], a2[4];
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        a0[u] = i32x4{0, 0, 0, 0};
                        a1[u] = i32x4{0, 0, 0, 0};
                        a2[u] = i32x4{0, 0, 0, 0};
                    }
#pragma unroll
                    for (int jp = 0; jp < 4; jp++) {
                        i32x4 bk[3];
#pragma unroll
                        for (int w = 0; w < 4; w++) {
                            const int j = 2 * jp + (w >> 1);
                            const uint32_t qv = qw[j][w & 1];
                            // bytes 0, 2 and 1, 3 in 16-bit halves: (q + 32) e - 32 e
                            const u16x2 ev = __builtin_bit_cast(u16x2, qv & 0x00FF00FFu);
                            const u16x2 ov = __builtin_bit_cast(u16x2, (qv >> 8) & 0x00FF00FFu);
#pragma unroll
                            for (int k = 0; k < 3; k++) {
                                const u16x2 m = __builtin_bit_cast(u16x2, dm[j][k]);
                                const u16x2 cc = __builtin_bit_cast(u16x2, dc[j][k]);
                                const uint32_t pe = __builtin_bit_cast(uint32_t, ev * m + cc);
                                const uint32_t po = __builtin_bit_cast(uint32_t, ov * m + cc);
                                bk[k][w] = (int)__builtin_amdgcn_perm(po, pe, 0x06020400u);
                            }
                        }
#pragma unroll
                        for (int u = 0; u < 4; u++) {
                            const int t = 4 * th + u;
                            const i32x4 av = *reinterpret_cast<const i32x4 *>(la + la_off(t, 2 * jp, g, c));
                            a0[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bk[0], a0[u], 0, 0, 0);
                            a1[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bk[1], a1[u], 0, 0, 0);
                            a2[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, bk[2], a2[u], 0, 0, 0);
                        }
                    }
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        const int t = 4 * th + u;
                        const float4 xs = *reinterpret_cast<const float4 *>(lxs + t * 8 + rb);
                        const float xsv[4] = {xs.x, xs.y, xs.z, xs.w};
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int acc = mad24(49, a2[u][i], mad24(7, a1[u][i], a0[u][i]));
                            y[t][i] += xsv[i] * (d * (float)acc);
                        }
                    }
                }
            }
        }
        if (more)
            stage_store(st, nxt_l, reinterpret_cast<float *>(nxt_l + kBgLdsA));
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
    // a block of at most 32 rows multiplies only the first four 8-row tiles
    if (S.dtype == kQ6K) {
        if (mrows > 32) bg_main<kQ6K, 2>(A, lds, m0, mrows, live, wrow, y);
        else bg_main<kQ6K, 1>(A, lds, m0, mrows, live, wrow, y);
    } else {
        if (mrows > 32) bg_main<kQ4K, 2>(A, lds, m0, mrows, live, wrow, y);
        else bg_main<kQ4K, 1>(A, lds, m0, mrows, live, wrow, y);
    }
    // y holds the plane sums: high on lanes g < 2, low on g >= 2 (same rows)
#pragma unroll
    for (int t = 0; t < 8; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) y[t][i] = fmaf(256.f, y[t][i], __shfl_xor(y[t][i], 32));

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
    const uint64_t sstride = (uint64_t)F.rows * ncol;
    auto sum = [&](int cc) {
        const float *p = A.part + (uint64_t)m * ncol + cc;
        float v = 0.f;
#pragma unroll 4
        for (int sp = 0; sp < A.splits; sp++) v += p[sp * sstride];  // split order
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

// K splits for a launch of `wgs` workgroups (one resident per CU: 8 waves
// of ~250 VGPRs): the split count with the fewest estimated super-block
// times, rounds of workgroups x (super-blocks per split + one for staging
// and the epilogue), plus a small cost per split for the reduction.
int bg_splits(int wgs, int nsb) {
    static int cus = 0;
    if (!cus) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cus = n;
        else
            cus = 256;
    }
    int best = 1;
    double best_t = 1e30;
    for (int sp = 1; sp <= std::min(16, std::max(1, nsb / 2)); sp++) {
        const double rounds = (double)((wgs * sp + cus - 1) / cus);
        const double t = rounds * ((nsb + sp - 1) / sp + 1) + (sp > 1 ? 0.25 * sp : 0.0);
        if (t < best_t - 1e-9) {
            best_t = t;
            best = sp;
        }
    }
    return best;
}

uint64_t bg_quant_bytes(int rows, int K) {
    return (uint64_t)rows * K * 2 + (uint64_t)rows * (K / 256) * 4;
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
    *splits = bg_splits((int)(x * *gy), K / 256);
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
    bg_prologue_kernel<<<(unsigned)a.rows, kPrThreads, plds, s>>>(a, A.q);
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
