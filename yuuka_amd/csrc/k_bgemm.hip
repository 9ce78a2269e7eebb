// k_bgemm.hip — verify GEMM for many rows (batched requests, 9..512 rows):
//
//   out_s[m, n] = epi( sum_k y[m, k] * dequant(W_s)[n, k] )
//
// with the prologues and epilogues of the fused verify GEMM (fgemm.h:
// RMSNorm or gated head norm of x, store / residual / SwiGLU, output maps).
// At a few rows the fused streaming kernel reads every weight once per
// launch; a batch of B requests x (k+1) rows would read them once per 8-row
// block. Here each weight super-block is read once per block of 48 rows (80
// for 49..80 rows), and the products run on v_mfma_f32_16x16x32_f16:
//
//  * prologue (one workgroup per row and group of 8 super-blocks): y =
//    prologue(x) computed as the reference computes it (recurrent.go:39-50
//    gated norm), or for the row RMSNorm (forward.go:460-482) y = x * w with
//    the group's float64 sum of squares stored, the GEMM scaling each row's
//    sums by its 1 / rms; then per 256-element super-block scaled into
//    [-256, 256] (one FP32 scale per row and super-block) and rounded to
//    FP16, with the FP32 sum of every 32-element sub-block of those FP16
//    values stored as an FP16 high part and its FP16 remainder — a workspace
//    of rows * (2 K + K / 8 + K / 64 + 64) B.
//  * GEMM (workgroup = a block of 16-row tiles x 8 tiles of 16 output
//    channels, one channel tile per wave): per super-block the block's FP16
//    values and sub-block sums are copied straight into LDS
//    (global_load_lds), double-buffered; each wave decodes its tile's
//    weights straight from HBM into MFMA B operands while the next
//    super-block's weights are in flight.
//    - Q4_K: the 6-bit sub-block scale is folded into the operand, B = sc q
//      (at most 945, exact in FP16), so the eight K = 32 MFMAs of a
//      super-block chain into one FP32 accumulator; the min term
//      sum_j m_j sum_k y_k is one more MFMA of the sub-block sums (high and
//      remainder in K slots 0..7 and 8..15) against the 6-bit mins. Then
//      acc * d - mins * dmin, times the row scale, per super-block in FP32.
//    - Q6_K: B = sc q with the signed 8-bit scale of the lane's 16-element
//      group (|sc q| <= 4064, rounded to FP16 above 2048, as the reference's
//      FP16 dequantization rounds d sc q), times d and the row scale.
//    The weights are the reference's FP16 dequantized values up to the FP32
//    factors d and dmin, and the activations FP16 as in the reference's own
//    FP16 GEMM (kernels/hip/gemm/wmma_gemm.hip load_a_tile / load_b_tile);
//    the products are exact and accumulate in FP32.
//
// Replaces, for batched verify shapes, the reference's per-matrix GEMV
// launches over all rows (kernels/hip/gemm/lm_head.hip:61-173 with MaxRows 16,
// engine/gpu/plan.go); no reference kernel on the verify path serves more
// than 16 rows.
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
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int kQ4K = YUUKA_DTYPE_Q4_K;
constexpr int kQ6K = YUUKA_DTYPE_Q6_K;
constexpr int kBgWaves = 8;
constexpr int kBgThreads = 64 * kBgWaves;
constexpr float kBgRange = 256.0f;  // |y / scale| <= kBgRange

// The prologue's output, in the order the GEMM stages it into LDS: rows
// padded to whole 16-row tiles (tiles = ceil(rows / 16); the padding rows are
// zero), super-block major so that one stage of a block of row tiles is one
// contiguous piece per tile:
//   h      [sb][tile][sub-block j][group g][row c][8 FP16]  (8 KB per tile)
//   sums   [sb][tile][row c][16 FP16]                       (512 B per tile)
//   scales [sb][tile * 16 + c] float
//   ss     [row][kBgSsGroups] float64 sums of squares of x over the
//          prologue workgroups' super-block groups (RMSNorm prologues: the
//          GEMM applies the row's 1/rms to its sums)
constexpr int kPrThreads = 512;                 // prologue workgroup: one super-block per wave
constexpr int kPrWaves = kPrThreads / 64;
constexpr int kBgSsGroups = 64 / kPrWaves;  // groups of kPrWaves super-blocks: K <= 16384
struct BgQuant {
    _Float16 *h;     // y / scale
    _Float16 *sums;  // sub-block sums of h: high parts (8) then remainders (8)
    float *scales;
    double *ss;
};

__host__ __device__ inline int bg_rows16(int rows) { return (rows + 15) & ~15; }

__host__ __device__ inline BgQuant bg_view(void *ws, int rows, int K) {
    uint8_t *p = static_cast<uint8_t *>(ws);
    const uint64_t r16 = (uint64_t)bg_rows16(rows);
    BgQuant q;
    q.h = reinterpret_cast<_Float16 *>(p);
    q.sums = reinterpret_cast<_Float16 *>(p + r16 * K * 2);
    q.scales = reinterpret_cast<float *>(p + r16 * K * 2 + r16 * (K / 256) * 32);
    q.ss = reinterpret_cast<double *>(p + r16 * K * 2 + r16 * (K / 256) * 36);  // 8-byte aligned: K % 256 == 0
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
// Sum over each aligned group of 8 lanes, in every lane of the group.
__device__ __forceinline__ float group8_sum(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, true));
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, true));
}

__device__ __forceinline__ uint32_t h2bits(_Float16 a, _Float16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// ---------------------------------------------------------------- prologue

// Where the prologue's x comes from: A.x, or (part != null) the split
// partial sums of the previous many-row GEMM, which the prologue finishes as
// bg_reduce_kernel would (sum in split order, + residual) and stores to out.
struct BgSrc {
    const float *part;  // [splits][rows][prow]
    const float *res;   // [rows][K] residual of the previous GEMM (may alias out), or null
    float *out;         // [rows][K] the previous GEMM's output
    uint64_t sstride;   // floats between splits (rows * prow)
    int splits;
    int swiglu;         // the previous GEMM's SwiGLU: gate columns [0, K), up [K, 2K) of each part row
    uint64_t prow;      // floats between rows of part (K, or 2K with swiglu)
};

// Workgroup (row, group of 8 P super-blocks). Wave w owns super-blocks w,
// w + 8, ... of the group (at most P of them) and lane l elements [4 l, +4)
// of each: x (or the split sums), the norm weights and the gate are loaded
// into registers in one round trip. With the row RMSNorm the group's float64
// sum of squares goes to q.ss and the values are quantized as x * w: the
// GEMM multiplies each row's sums by the row's 1 / rms, so no workgroup
// needs the whole row.
template <int P>
__global__ __launch_bounds__(kPrThreads) void bg_prologue_kernel(const FusedGemmArgs A, BgQuant q, const BgSrc src) {
    constexpr int W = kPrThreads / 64;
    __shared__ double red[W];
    const int row = blockIdx.x, K = A.K, nsb = K / 256;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint64_t rbase = (uint64_t)row * K;
    // super-blocks [sb0, sb0 + W P) of the row (grid y: the group)
    const int sb0 = (int)blockIdx.y * W * P;
    auto elem = [&](int i) { return (sb0 + wave + W * i) * 256 + 4 * lane; };
    auto live = [&](int i) { return sb0 + wave + W * i < nsb; };
    // where lane's four values, its sub-block sum and the row scale of
    // super-block sb go (lane: sub-block lane / 8, group (lane / 2) % 4, half lane % 2)
    const int tiles = bg_rows16(A.rows) / 16, tile = row >> 4, c = row & 15;
    auto h_at = [&](int sb) {
        return q.h + ((uint64_t)sb * tiles + tile) * 4096 + (lane >> 3) * 512 + ((lane >> 1) & 3) * 128 + c * 8 +
               (lane & 1) * 4;
    };
    auto sums_at = [&](int sb) { return q.sums + ((uint64_t)sb * tiles + tile) * 256 + c * 16 + (lane >> 3); };
    auto scale_at = [&](int sb) { return q.scales + (uint64_t)sb * tiles * 16 + row; };
    if (row >= A.rows) {  // a padding row of the last tile: zeros
#pragma unroll
        for (int i = 0; i < P; i++) {
            if (!live(i)) break;  // wave-uniform
            const int sb = sb0 + wave + W * i;
            *reinterpret_cast<uint2 *>(h_at(sb)) = make_uint2(0u, 0u);
            if ((lane & 7) == 0) {
                sums_at(sb)[0] = (_Float16)0.0f;
                sums_at(sb)[8] = (_Float16)0.0f;
            }
            if (lane == 0) *scale_at(sb) = 0.f;
        }
        return;
    }
    auto add4 = [](float4 &v, const float4 &w) {
        v.x += w.x;
        v.y += w.y;
        v.z += w.z;
        v.w += w.w;
    };
    float4 v[P], nw[P], z[P];
    if (src.part && src.swiglu) {
        // the previous GEMM's gate and up partial sums, each added in split
        // order, then SiLU(gate) * up (bg_reduce_kernel's arithmetic)
        constexpr int SG = P >= 4 ? 1 : 8 / P;
        float4 u[P];
        const uint64_t pbase = (uint64_t)row * src.prow;
#pragma unroll
        for (int i = 0; i < P; i++) v[i] = u[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int s0 = 0; s0 < src.splits; s0 += SG) {
            float4 tg[SG][P], tu[SG][P];
#pragma unroll
            for (int j = 0; j < SG; j++)
#pragma unroll
                for (int i = 0; i < P; i++)
                    if (s0 + j < src.splits && live(i)) {
                        const float *q = src.part + (uint64_t)(s0 + j) * src.sstride + pbase + elem(i);
                        tg[j][i] = *reinterpret_cast<const float4 *>(q);
                        tu[j][i] = *reinterpret_cast<const float4 *>(q + K);
                    }
#pragma unroll
            for (int j = 0; j < SG; j++)
#pragma unroll
                for (int i = 0; i < P; i++)
                    if (s0 + j < src.splits && live(i)) {
                        add4(v[i], tg[j][i]);
                        add4(u[i], tu[j][i]);
                    }
        }
#pragma unroll
        for (int i = 0; i < P; i++)
            if (live(i)) {
                v[i].x = __fmul_rn(silu_ref(v[i].x), u[i].x);
                v[i].y = __fmul_rn(silu_ref(v[i].y), u[i].y);
                v[i].z = __fmul_rn(silu_ref(v[i].z), u[i].z);
                v[i].w = __fmul_rn(silu_ref(v[i].w), u[i].w);
                *reinterpret_cast<float4 *>(src.out + rbase + elem(i)) = v[i];
            }
    } else if (src.part) {
        // the previous GEMM's split partial sums, added in split order, then
        // its residual; 16 loads in flight at a time
        constexpr int SG = P >= 8 ? 2 : 16 / P;
#pragma unroll
        for (int i = 0; i < P; i++) v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int s0 = 0; s0 < src.splits; s0 += SG) {
            float4 t[SG][P];
#pragma unroll
            for (int j = 0; j < SG; j++)
#pragma unroll
                for (int i = 0; i < P; i++)
                    if (s0 + j < src.splits && live(i))
                        t[j][i] = *reinterpret_cast<const float4 *>(src.part + (uint64_t)(s0 + j) * src.sstride + rbase +
                                                                    elem(i));
#pragma unroll
            for (int j = 0; j < SG; j++)
#pragma unroll
                for (int i = 0; i < P; i++)
                    if (s0 + j < src.splits && live(i)) add4(v[i], t[j][i]);
        }
#pragma unroll
        for (int i = 0; i < P; i++)
            if (live(i)) {
                const float4 r = *reinterpret_cast<const float4 *>(src.res + rbase + elem(i));
                v[i].x = __fadd_rn(v[i].x, r.x);
                v[i].y = __fadd_rn(v[i].y, r.y);
                v[i].z = __fadd_rn(v[i].z, r.z);
                v[i].w = __fadd_rn(v[i].w, r.w);
                *reinterpret_cast<float4 *>(src.out + rbase + elem(i)) = v[i];
            }
    } else {
#pragma unroll
        for (int i = 0; i < P; i++)
            if (live(i)) v[i] = *reinterpret_cast<const float4 *>(A.x + rbase + elem(i));
    }
    float4 hw = make_float4(0.f, 0.f, 0.f, 0.f);
    if (A.gate) {
        hw = *reinterpret_cast<const float4 *>(A.head_norm + ((4 * lane) & 127));
#pragma unroll
        for (int i = 0; i < P; i++)
            if (live(i)) z[i] = *reinterpret_cast<const float4 *>(A.gate + rbase + elem(i));
    } else if (A.norm) {
#pragma unroll
        for (int i = 0; i < P; i++)
            if (live(i)) nw[i] = *reinterpret_cast<const float4 *>(A.norm + elem(i));
    }
    if (A.norm && !A.gate) {
        // forward.go:460-470 rmsNorm: float64 sum of squares (this group's
        // part, waves in order; the GEMM adds the groups in order)
        double ss = 0.0;
#pragma unroll
        for (int i = 0; i < P; i++)
            if (live(i))
                ss += (double)v[i].x * (double)v[i].x + (double)v[i].y * (double)v[i].y +
                      (double)v[i].z * (double)v[i].z + (double)v[i].w * (double)v[i].w;
        ss = wave_sum_d(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        if (threadIdx.x == 0) {
            double t = 0.0;
#pragma unroll
            for (int w = 0; w < W; w++) t += red[w];
            q.ss[(uint64_t)row * kBgSsGroups + blockIdx.y] = t;
        }
    }
#pragma unroll
    for (int i = 0; i < P; i++) {
        if (!live(i)) break;  // wave-uniform
        const int sb = sb0 + wave + W * i;
        float4 y = v[i];
        if (A.gate) {
            // recurrent.go:39-50 gated head norm over heads of 128 (lanes 0..31
            // and 32..63 hold one head each): x * (scale * w) * gate
            double hs = (double)y.x * (double)y.x + (double)y.y * (double)y.y + (double)y.z * (double)y.z +
                        (double)y.w * (double)y.w;
            hs = row16_sum_d(hs);  // each 128-element head is two 16-lane rows
            hs = lane < 32 ? rl_d(hs, 0) + rl_d(hs, 16) : rl_d(hs, 32) + rl_d(hs, 48);
            const float mean = (float)(hs / 128.0);
            const float hsc = (float)(1.0 / sqrt((double)(mean + A.eps)));
            y.x = __fmul_rn(__fmul_rn(y.x, __fmul_rn(hsc, hw.x)), z[i].x);
            y.y = __fmul_rn(__fmul_rn(y.y, __fmul_rn(hsc, hw.y)), z[i].y);
            y.z = __fmul_rn(__fmul_rn(y.z, __fmul_rn(hsc, hw.z)), z[i].z);
            y.w = __fmul_rn(__fmul_rn(y.w, __fmul_rn(hsc, hw.w)), z[i].w);
        } else if (A.norm) {  // x * w; the row's 1 / rms scales the GEMM's sums
            y.x = __fmul_rn(y.x, nw[i].x);
            y.y = __fmul_rn(y.y, nw[i].y);
            y.z = __fmul_rn(y.z, nw[i].z);
            y.w = __fmul_rn(y.w, nw[i].w);
        }
        float m = fmaxf(fmaxf(fabsf(y.x), fabsf(y.y)), fmaxf(fabsf(y.z), fabsf(y.w)));
        m = wave_max_nonneg(m);
        const float inv = m > 0.f ? kBgRange / m : 0.f;
        const _Float16 h0 = (_Float16)(y.x * inv), h1 = (_Float16)(y.y * inv), h2 = (_Float16)(y.z * inv),
                       h3 = (_Float16)(y.w * inv);
        *reinterpret_cast<uint2 *>(h_at(sb)) = make_uint2(h2bits(h0, h1), h2bits(h2, h3));
        // sub-block lane >> 3: eight lanes of four values
        const float s = group8_sum(((float)h0 + (float)h1) + ((float)h2 + (float)h3));
        if ((lane & 7) == 0) {
            const _Float16 shi = (_Float16)s, slo = (_Float16)(s - (float)shi);
            _Float16 *sd = sums_at(sb);
            sd[0] = shi;
            sd[8] = slo;
        }
        if (lane == 0) *scale_at(sb) = m > 0.f ? m / kBgRange : 0.f;
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

// 8 bytes at an even byte address (Q6_K blocks are 210 B): two dword-aligned
// loads and a byte shift.
__device__ __forceinline__ uint64_t load8_even(const uint8_t *p) {
    const uint32_t sh = (uint32_t)reinterpret_cast<uintptr_t>(p) & 3;
    const uint32_t *w = reinterpret_cast<const uint32_t *>(p - sh);  // pointer arithmetic keeps the global address space
    const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
    const uint32_t lo = __builtin_amdgcn_alignbyte(w1, w0, sh);
    const uint32_t hi = __builtin_amdgcn_alignbyte(w2, w1, sh);
    return (uint64_t)lo | ((uint64_t)hi << 32);
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

// FP16 pairs from byte pairs: (x & mask) | 0x6400 in each 16-bit half is
// 1024 + x as FP16 (x < 1024).
__device__ __forceinline__ half2v magic_pair(uint32_t w, uint32_t mask) {
    uint32_t r;  // one v_and_or_b32 (written out: the compiler splits it when the and is shared)
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(w), "v"(mask), "v"(0x64006400u));
    return __builtin_bit_cast(half2v, r);
}
__device__ __forceinline__ half2v splat_h(float v) {
    const _Float16 h = (_Float16)v;
    return half2v{h, h};
}
// Operand of one K = 32 MFMA as four FP16 pairs.
__device__ __forceinline__ half8 pack8(half2v a, half2v b, half2v c, half2v d) {
    return half8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// LDS of one stage for NT row tiles, in the order of the quantized rows
// (BgQuant): A [tile][sub-block j][group g][row c][8 FP16], so that lane
// (c, g) reads the A operand of tile t, sub-block j at g 256 + c 16 + t 8192
// + j 1024 (16 consecutive lanes read 256 consecutive bytes, and all but the
// lane's own offset are instruction immediates), sub-block sums [tile][c][16
// FP16], row scales [16 NT] float. Two stages; the SwiGLU epilogue reuses
// the first.
template <int NT> struct BgLds {
    static constexpr int kRows = 16 * NT;
    static constexpr uint32_t A = 0;
    static constexpr uint32_t S = A + NT * 8192;
    static constexpr uint32_t X = S + NT * 512;
    static constexpr uint32_t stage = X + kRows * 4;
    static constexpr uint32_t total = 2 * stage;
};
static_assert(BgLds<9>::total + 16 * 9 * 4 <= 160 * 1024, "nine tiles (and the row norms) fit LDS");

// 16-byte global -> LDS copy of one lane (lane l writes [m0 + 16 l, +16)
// from base + voff, base uniform), as inline assembly so that the
// compiler's wait counts do not see it (it would otherwise wait for the
// weight loads before every LDS read). The main loop waits for the copies
// itself (vmcnt(0) before its barrier).
__device__ __forceinline__ void lds_copy16(const uint8_t *base, uint32_t voff, const uint8_t *lds_dst) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_dst);
    const uint64_t b = reinterpret_cast<uintptr_t>(base);
    const uint64_t sb = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b) |
                        ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32)) << 32);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sb), "s"(m0)
                 : "memory", "m0");
}

// Issues the copies of super-block sb of the block's tiles [T0, T0 + NT)
// into a stage — per tile one 8 KB piece, 16 bytes per thread, and the
// tiles' sums as one piece — and returns this thread's row scale (threads <
// 16 NT). Tiles past the last one are not copied: their rows' outputs are
// never stored.
template <int NT>
__device__ __forceinline__ float stage_issue(const BgArgs &A, uint8_t *stage, int T0, int tiles, int sb) {
    using LY = BgLds<NT>;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const uint32_t voff = threadIdx.x * 16;
    const int nt = min(NT, tiles - T0);
    const uint64_t piece = (uint64_t)sb * tiles + T0;
    const uint8_t *h = reinterpret_cast<const uint8_t *>(A.q.h) + piece * 8192;
#pragma unroll
    for (int t = 0; t < NT; t++)
        if (t < nt) lds_copy16(h + t * 8192, voff, stage + LY::A + t * 8192 + wave * 1024);
    if (voff < (uint32_t)nt * 512)
        lds_copy16(reinterpret_cast<const uint8_t *>(A.q.sums) + piece * 512, voff, stage + LY::S + wave * 1024);
    const int t = (int)threadIdx.x;
    return t < 16 * nt ? A.q.scales[piece * 16 + t] : 0.f;
}

// One super-block of the wave's tile against the NT row tiles of stage st
// (sub-block pairs outer, row tiles inner: two B operands live at a time,
// one FP32 accumulator per row tile), added into y. Rows past the block's
// end are computed like the others (a branch per tile would keep the
// scheduler from issuing the tiles' LDS reads ahead of their MFMAs).
template <int NT>
__device__ __forceinline__ void bg_super_q4(const WQ4 &cur, const uint8_t *st, float (&y)[NT][4]) {
    using LY = BgLds<NT>;
    const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
    const uint8_t *la = st + LY::A + g * 256 + c * 16;
    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const float d = h2f((uint16_t)(cur.hdr.x & 0xffffu));
    const float dmin = h2f((uint16_t)(cur.hdr.x >> 16));
    _Float16 mins[8];
#pragma unroll
    for (int jp = 0; jp < 4; jp++) {
        int sce, mne, sco, mno;
        scale_min_k4(2 * jp, cur.hdr.y, cur.hdr.z, cur.hdr.w, &sce, &mne);
        scale_min_k4(2 * jp + 1, cur.hdr.y, cur.hdr.z, cur.hdr.w, &sco, &mno);
        mins[2 * jp] = (_Float16)mne;
        mins[2 * jp + 1] = (_Float16)mno;
        // bytes b0..b7 of the lane: low nibbles are sub-block 2 jp, high
        // nibbles 2 jp + 1. Low: (1024 + q) sc - 1024 sc; high, masked in
        // place: (1024 + 16 q) (sc / 16) - 64 sc. Both are q sc exactly (one
        // rounding of an exact value below 2048).
        const uint32_t w0 = (uint32_t)cur.q[jp], w1 = (uint32_t)(cur.q[jp] >> 32);
        const uint32_t p01 = __builtin_amdgcn_perm(0u, w0, 0x0c010c00u), p23 = __builtin_amdgcn_perm(0u, w0, 0x0c030c02u);
        const uint32_t p45 = __builtin_amdgcn_perm(0u, w1, 0x0c010c00u), p67 = __builtin_amdgcn_perm(0u, w1, 0x0c030c02u);
        const half2v se = splat_h((float)sce), so = splat_h(0.0625f * (float)sco);
        const half2v ce = splat_h(-1024.f * (float)sce), co = splat_h(-64.f * (float)sco);
        const half8 be = pack8(__builtin_elementwise_fma(magic_pair(p01, 0x000F000Fu), se, ce),
                               __builtin_elementwise_fma(magic_pair(p23, 0x000F000Fu), se, ce),
                               __builtin_elementwise_fma(magic_pair(p45, 0x000F000Fu), se, ce),
                               __builtin_elementwise_fma(magic_pair(p67, 0x000F000Fu), se, ce));
        const half8 bo = pack8(__builtin_elementwise_fma(magic_pair(p01, 0x00F000F0u), so, co),
                               __builtin_elementwise_fma(magic_pair(p23, 0x00F000F0u), so, co),
                               __builtin_elementwise_fma(magic_pair(p45, 0x00F000F0u), so, co),
                               __builtin_elementwise_fma(magic_pair(p67, 0x00F000F0u), so, co));
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const half8 ae = *reinterpret_cast<const half8 *>(la + t * 8192 + (2 * jp) * 1024);
            const half8 ao = *reinterpret_cast<const half8 *>(la + t * 8192 + (2 * jp + 1) * 1024);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ae, be, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ao, bo, acc[t], 0, 0, 0);
        }
    }
    // min term: K slots 0..7 (lanes g = 0) and 8..15 (g = 1) hold the mins
    // against the sums' high parts and remainders
    const half8 bmin = g < 2 ? half8{mins[0], mins[1], mins[2], mins[3], mins[4], mins[5], mins[6], mins[7]} : half8{};
    const uint8_t *ls = st + LY::S + c * 32 + g * 16;
    const float *lxs = reinterpret_cast<const float *>(st + LY::X) + 4 * g;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const half8 as = g < 2 ? *reinterpret_cast<const half8 *>(ls + t * 512) : half8{};
        const f32x4 mn = __builtin_amdgcn_mfma_f32_16x16x32_f16(as, bmin, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        const float4 xs = *reinterpret_cast<const float4 *>(lxs + 16 * t);
        const float xsv[4] = {xs.x, xs.y, xs.z, xs.w};
#pragma unroll
        for (int i = 0; i < 4; i++) y[t][i] += xsv[i] * (d * acc[t][i] - dmin * mn[i]);
    }
}

template <int NT>
__device__ __forceinline__ void bg_super_q6(const WQ6 &cur, const uint8_t *st, float (&y)[NT][4]) {
    using LY = BgLds<NT>;
    const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
    const uint8_t *la = st + LY::A + g * 256 + c * 16;
    f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Q6_K: q = (ql | qh << 4) - 32, scale byte 2 j + (g >> 1) for the
    // lane's eight elements of sub-block j
    const float d = h2f((uint16_t)cur.d);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int half = j >> 2, qd = j & 3;
        const uint64_t lo4 = (cur.ql[2 * half + (qd & 1)] >> (4 * (qd >> 1))) & 0x0F0F0F0F0F0F0F0Full;
        const uint64_t hi2 = ((cur.qh[half] >> (2 * qd)) & 0x0303030303030303ull) << 4;
        const uint64_t u = lo4 | hi2;  // q + 32 per byte
        const uint32_t w0 = (uint32_t)u, w1 = (uint32_t)(u >> 32);
        const half2v s2 = splat_h((float)sbyte(cur.sc, 2 * j + (g >> 1)));
        const half2v off = splat_h(-1056.f);
        auto one = [&](uint32_t pq) __attribute__((always_inline)) {
            return (magic_pair(pq, 0x003F003Fu) + off) * s2;  // (1024 + q + 32) - 1056 = q, times sc
        };
        const half8 bj = pack8(one(__builtin_amdgcn_perm(0u, w0, 0x0c010c00u)), one(__builtin_amdgcn_perm(0u, w0, 0x0c030c02u)),
                               one(__builtin_amdgcn_perm(0u, w1, 0x0c010c00u)), one(__builtin_amdgcn_perm(0u, w1, 0x0c030c02u)));
#pragma unroll
        for (int t = 0; t < NT; t++)
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(*reinterpret_cast<const half8 *>(la + t * 8192 + j * 1024), bj,
                                                            acc[t], 0, 0, 0);
    }
    const float *lxs = reinterpret_cast<const float *>(st + LY::X) + 4 * g;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const float4 xs = *reinterpret_cast<const float4 *>(lxs + 16 * t);
        const float xsv[4] = {xs.x, xs.y, xs.z, xs.w};
#pragma unroll
        for (int i = 0; i < 4; i++) y[t][i] += xsv[i] * (d * acc[t][i]);
    }
}

// The main loop of one wave over the super-blocks (weights of dtype DT) of
// the block of row tiles [T0, T0 + NT): its tile's B operands are built once
// per super-block and multiplied with all NT row tiles. Two LDS stages and
// two weight register sets, unrolled by two so that each is a fixed one:
// super-block sb + 1 is copied and loaded while sb is multiplied. Every
// weight load is issued, its index clamped to the last super-block (loads
// under a branch would make the compiler copy the register sets).
// `pre` runs after the first super-block's copies and weight loads are
// issued and before the wait for them (its own loads are the youngest, so
// waiting for them costs nothing more).
template <int DT, int NT, class Pre>
__device__ __forceinline__ void bg_main(const BgArgs &A, uint8_t *lds, int T0, bool live, const uint8_t *wrow,
                                        float (&y)[NT][4], Pre pre) {
    using LY = BgLds<NT>;
    const int g = (threadIdx.x & 63) >> 4;
    const int tiles = bg_rows16(A.f.rows) / 16;
    // this split's super-blocks [sb_lo, nsb)
    const int nsb_all = A.f.K / 256;
    const int sb_lo = (int)((int64_t)nsb_all * blockIdx.z / A.splits);
    const int nsb = (int)((int64_t)nsb_all * (blockIdx.z + 1) / A.splits);
    constexpr int blk = DT == kQ4K ? 144 : 210;
    typedef typename std::conditional<DT == kQ4K, WQ4, WQ6>::type W;
    auto loadw = [&](W &w, int sb) __attribute__((always_inline)) {
        const uint8_t *b = wrow + (uint64_t)sb * blk;
        if constexpr (DT == kQ4K) load_q4(w, b, g);
        else load_q6(w, b, g);
    };
    auto super = [&](const W &w, const uint8_t *st) __attribute__((always_inline)) {
        if constexpr (DT == kQ4K) bg_super_q4<NT>(w, st, y);
        else bg_super_q6<NT>(w, st, y);
    };
    float *x0 = reinterpret_cast<float *>(lds + LY::X), *x1 = reinterpret_cast<float *>(lds + LY::stage + LY::X);
    W wa, wb;
    loadw(wa, sb_lo);
    float xs = stage_issue<NT>(A, lds, T0, tiles, sb_lo);
    pre();
    __builtin_amdgcn_s_waitcnt(0);
    if (threadIdx.x < LY::kRows) x0[threadIdx.x] = xs;
    __syncthreads();
#pragma unroll 1
    for (int sb = sb_lo; sb < nsb; sb += 2) {
        // stage 0 and wa hold sb; stage 1 and wb take sb + 1
        const bool more1 = sb + 1 < nsb;
        if (more1) xs = stage_issue<NT>(A, lds + LY::stage, T0, tiles, sb + 1);
        loadw(wb, min(sb + 1, nsb - 1));
        if (live) super(wa, lds);
        if (more1) {
            __builtin_amdgcn_s_waitcnt(0);  // the copies into stage 1 (and this thread's row scale)
            if (threadIdx.x < LY::kRows) x1[threadIdx.x] = xs;
        }
        __syncthreads();  // stage 1 complete; stage 0 read by every wave
        if (!more1) break;
        const bool more2 = sb + 2 < nsb;
        if (more2) xs = stage_issue<NT>(A, lds, T0, tiles, sb + 2);
        loadw(wa, min(sb + 2, nsb - 1));
        if (live) super(wb, lds + LY::stage);
        if (more2) {
            __builtin_amdgcn_s_waitcnt(0);
            if (threadIdx.x < LY::kRows) x0[threadIdx.x] = xs;
        }
        __syncthreads();
    }
}

template <int NT>
__global__ __launch_bounds__(kBgThreads) __attribute__((amdgpu_waves_per_eu(NT > 4 ? 2 : 4))) void bg_gemm_kernel(
    const BgArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int kRowsB = 16 * NT;
    const FusedGemmArgs &F = A.f;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = lane & 15, g = lane >> 4;
    const int m0 = blockIdx.y * kRowsB;
    const int mrows = min(kRowsB, F.rows - m0);

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

    float y[NT][4];
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) y[t][i] = 0.f;
    // RMSNorm prologue: the 1 / rms of the block's rows from the prologue's
    // group sums (added in group order; forward.go:460-470), published by
    // the main loop's first barrier
    __shared__ float row_inv[kRowsB];
    const bool rnorm = F.norm != nullptr && F.gate == nullptr;
    auto pre = [&]() __attribute__((always_inline)) {
        if (!rnorm || threadIdx.x >= kRowsB) return;
        const int row = min(m0 + (int)threadIdx.x, F.rows - 1), G = (F.K / 256 + kPrWaves - 1) / kPrWaves;
        const double *ps = A.q.ss + (uint64_t)row * kBgSsGroups;
        double v[kBgSsGroups];
#pragma unroll
        for (int gi = 0; gi < kBgSsGroups; gi++) v[gi] = ps[min(gi, G - 1)];
        double t = 0.0;
#pragma unroll
        for (int gi = 0; gi < kBgSsGroups; gi++)
            if (gi < G) t += v[gi];
        const float mean = (float)(t / (double)F.K);
        row_inv[threadIdx.x] = (float)(1.0 / sqrt((double)(mean + F.eps)));
    };
    if (S.dtype == kQ6K) bg_main<kQ6K, NT>(A, lds, m0 / 16, live, wrow, y, pre);
    else bg_main<kQ4K, NT>(A, lds, m0 / 16, live, wrow, y, pre);
    if (rnorm) {
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) y[t][i] = __fmul_rn(y[t][i], row_inv[16 * t + 4 * g + i]);
    }

    // epilogue: lane (c, g) holds rows 16 t + 4 g + i of channel n0 + c
    if (A.splits > 1) {  // partial sums of this split; bg_reduce_kernel finishes
        if (!live || n0 + c >= S.n) return;
        const int ncol = A.cols[F.nseg];
        float *pp = A.part + (uint64_t)blockIdx.z * F.rows * ncol + A.cols[seg] + n0 + c;
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = 16 * t + 4 * g + i;
                if (r < mrows) pp[(uint64_t)(m0 + r) * ncol] = y[t][i];
            }
        return;
    }
    if (A.swiglu) {
        __syncthreads();
        float *up = reinterpret_cast<float *>(lds);  // [4 tiles][rows][16]
        if (wave >= 4) {
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) up[((wave - 4) * kRowsB + 16 * t + 4 * g + i) * 16 + c] = y[t][i];
        }
        __syncthreads();
        if (wave < 4 && live && n0 + c < S.n) {
#pragma unroll
            for (int t = 0; t < NT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = 16 * t + 4 * g + i;
                    if (r >= mrows) continue;
                    const float u = up[(wave * kRowsB + r) * 16 + c];
                    S.out[(uint64_t)(m0 + r) * S.n + n0 + c] = __fmul_rn(silu_ref(y[t][i]), u);
                }
        }
        return;
    }
    if (!live || n0 + c >= S.n) return;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = 16 * t + 4 * g + i;
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

// Row tiles per workgroup for a launch of `rows` rows (measured at config
// shapes, prologue + GEMM per launch: 144 rows gate/up 50.1 / 54.7 / 64.2 /
// 60.7 us at 3 / 4 / 5 / 9 tiles; 68 rows 44.1 / 47.2 / 41.4 / 49.4 us;
// 40 rows 30.0 / 31.4 / 37.2 / 45.3 us). Five tiles (80 rows, one
// workgroup per CU) serve 49..80 rows in one block; otherwise blocks of 48
// rows (three tiles, two workgroups per CU).
int bg_tiles(int rows) { return rows > 48 && rows <= 80 ? 5 : 3; }

template <int NT> const void *bg_kernel_ptr() { return reinterpret_cast<const void *>(bg_gemm_kernel<NT>); }

// Resident workgroups of the NT-tile kernel on the device (cached).
int bg_resident(int nt) {
    static int res[10] = {0};  // by tile count
    if (!res[nt]) {
        int dev = 0, n = 0, per = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        const void *k = nt == 5 ? bg_kernel_ptr<5>() : bg_kernel_ptr<3>();
        const uint32_t lds = nt == 5 ? BgLds<5>::total : BgLds<3>::total;
        (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k, kBgThreads, lds) != hipSuccess || per <= 0) per = 1;
        res[nt] = n * per;
    }
    return res[nt];
}

// K splits for a launch of `wgs` workgroups over `nsb` super-blocks: the
// split count with the least estimated time, in super-block steps,
//   ceil(wgs * splits / CUs) * (ceil(nsb / splits) + 1) + 0.1 splits,
// i.e. the workgroups the busiest CU runs (one at a time: a CU's issue
// saturates with one workgroup) times each one's steps, the + 1 being its
// staging and epilogue and the last term the reduction. Fitted to a sweep
// of 1..12 splits over the config shapes at 40, 68 and 144 rows: the chosen
// splits cost 0.5 % more than the best of each shape (2.6 % for a count of
// resident-workgroup rounds).
int bg_splits(int wgs, int nsb, int nt) {
    (void)bg_resident(nt);  // sets the kernel's LDS attribute
    static int cus = 0;
    if (!cus) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cus = n;
    }
    int best = 1;
    double best_t = 1e30;
    for (int sp = 1; sp <= std::min(16, std::max(1, nsb / 2)); sp++) {
        const double k = (double)((wgs * sp + cus - 1) / cus);
        const double t = k * (double)((nsb + sp - 1) / sp + 1) + (sp > 1 ? 0.1 * sp : 0.0);
        if (t < best_t - 1e-9) {
            best_t = t;
            best = sp;
        }
    }
    return best;
}

uint64_t bg_quant_bytes(int rows, int K) {
    const uint64_t r16 = (uint64_t)bg_rows16(rows);
    return r16 * K * 2 + r16 * (K / 256) * 32 + r16 * (K / 256) * 4 + r16 * kBgSsGroups * 8;
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
    const int nt = bg_tiles(rows);
    *gy = (unsigned)((rows + 16 * nt - 1) / (16 * nt));
    *splits = bg_splits((int)(x * *gy), K / 256, nt);
}

void fused_gemm_rows_ws_parts(int rows, int K, const int *n, int nseg, bool swiglu, uint64_t *quant,
                              uint64_t *part) {
    unsigned gx, gy;
    int splits;
    bg_grid(n, nseg, swiglu, rows, K, &gx, &gy, &splits);
    int ncol = 0;
    for (int i = 0; i < nseg; i++) ncol += n[i];
    *quant = bg_quant_bytes(rows, K);
    *part = splits > 1 ? (uint64_t)splits * rows * ncol * 4 : 0;
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

// The arguments, grid and workspace view of one many-row launch.
static void bg_setup(const FusedGemmArgs &a, void *ws, BgArgs &A, unsigned &gx, unsigned &gy,
                     uint64_t part_off = 0) {
    A = BgArgs{};
    A.f = a;
    A.q = bg_view(ws, a.rows, a.K);
    A.swiglu = a.epilogue == kEpiSwiglu ? 1 : 0;
    // segment prefix in workgroups of 8 tiles (a workgroup never straddles two segments)
    A.tiles[0] = 0;
    for (int i = 0; i < a.nseg; i++) A.tiles[i + 1] = A.tiles[i] + (a.seg[i].n + 16 * kBgWaves - 1) / (16 * kBgWaves);
    for (int i = a.nseg + 1; i <= kFusedMaxSeg; i++) A.tiles[i] = A.tiles[a.nseg];
    int nn[kFusedMaxSeg];
    for (int i = 0; i < a.nseg; i++) nn[i] = a.seg[i].n;
    bg_grid(nn, a.nseg, A.swiglu != 0, a.rows, a.K, &gx, &gy, &A.splits);
    A.cols[0] = 0;
    for (int i = 0; i < a.nseg; i++) A.cols[i + 1] = A.cols[i] + a.seg[i].n;
    for (int i = a.nseg + 1; i <= kFusedMaxSeg; i++) A.cols[i] = A.cols[a.nseg];
    // split partial sums after the quantized rows, or at part_off (a chain's
    // common offset, past every member's quantized rows)
    A.part = reinterpret_cast<float *>(static_cast<uint8_t *>(ws) +
                                       (part_off ? part_off : (bg_quant_bytes(a.rows, a.K) + 255) & ~255ull));
}

static hipError_t bg_launch_prologue(const FusedGemmArgs &a, const BgQuant &q, const BgSrc &src, hipStream_t s) {
    // one workgroup per (row, group of 8 super-blocks), + the padding rows
    const int nsb = a.K / 256, W = kPrThreads / 64;
    if (nsb > W * kBgSsGroups) return hipErrorInvalidValue;  // K over 16384
    const dim3 grid((unsigned)bg_rows16(a.rows), (unsigned)((nsb + W - 1) / W));
    bg_prologue_kernel<1><<<grid, kPrThreads, 0, s>>>(a, q, src);
    return hipGetLastError();
}

// The GEMM, then (reduce and more than one split) the split reduction.
static hipError_t bg_launch_gemm(const BgArgs &A, unsigned gx, unsigned gy, bool reduce, hipStream_t s) {
    const FusedGemmArgs &a = A.f;
    const dim3 grid(gx, gy, (unsigned)A.splits);
    // (bg_grid's bg_resident call has set the kernel's LDS attribute)
    if (bg_tiles(a.rows) == 5) bg_gemm_kernel<5><<<grid, kBgThreads, BgLds<5>::total, s>>>(A);
    else bg_gemm_kernel<3><<<grid, kBgThreads, BgLds<3>::total, s>>>(A);
    if (reduce && A.splits > 1) {
        const uint64_t nout = (uint64_t)a.rows * (A.swiglu ? a.seg[0].n : A.cols[a.nseg]);
        bg_reduce_kernel<<<(unsigned)((nout + 255) / 256), 256, 0, s>>>(A);
    }
    return hipGetLastError();
}

hipError_t launch_fused_gemm_rows(const FusedGemmArgs &a, void *ws, hipStream_t s) {
    BgArgs A;
    unsigned gx, gy;
    bg_setup(a, ws, A, gx, gy);
    hipError_t err = bg_launch_prologue(a, A.q, BgSrc{}, s);
    if (err == hipSuccess) err = bg_launch_gemm(A, gx, gy, true, s);
    return err;
}

// Whether b's prologue can take a's split partial sums: a residual GEMM
// whose output b normalises, or a SwiGLU GEMM whose output b reads as it is
// (FFN gate/up -> down).
static bool bg_link(const FusedGemmArgs &a, const FusedGemmArgs &b) {
    const bool res_pair = a.epilogue == kEpiResidual && a.nseg == 1 && a.seg[0].res != nullptr && b.norm != nullptr;
    const bool glu_pair = a.epilogue == kEpiSwiglu && a.nseg == 2 && b.norm == nullptr;
    return (res_pair || glu_pair) && b.rows == a.rows && b.K == a.seg[0].n && b.x == a.seg[0].out &&
           b.gate == nullptr && b.K % 256 == 0;
}

hipError_t launch_fused_gemm_rows_chain(const FusedGemmArgs *g, int n, void *ws, uint64_t part_off, bool defer_last,
                                        hipStream_t s, BgDeferred *last) {
    *last = BgDeferred{};
    BgSrc src{};  // the previous member's partials, when this member's prologue takes them
    for (int i = 0; i < n; i++) {
        const FusedGemmArgs &a = g[i];
        BgArgs A;
        unsigned gx, gy;
        bg_setup(a, ws, A, gx, gy, part_off);
        const bool link = A.splits > 1 && i + 1 < n && bg_link(a, g[i + 1]);
        const bool defer = A.splits > 1 && i + 1 == n && defer_last && a.epilogue == kEpiResidual && a.nseg == 1 &&
                           a.seg[0].res != nullptr;
        hipError_t err = bg_launch_prologue(a, A.q, src, s);
        if (err == hipSuccess) err = bg_launch_gemm(A, gx, gy, !(link || defer), s);
        if (err != hipSuccess) return err;
        src = BgSrc{};
        if (link) {
            const bool glu = a.epilogue == kEpiSwiglu;
            src = BgSrc{A.part,    glu ? nullptr : a.seg[0].res,
                        a.seg[0].out, (uint64_t)a.rows * A.cols[a.nseg],
                        A.splits,  glu ? 1 : 0,
                        (uint64_t)A.cols[a.nseg]};
        }
        if (defer) *last = BgDeferred{true, A.part, (uint64_t)a.rows * a.seg[0].n, A.splits};
    }
    return hipSuccess;
}

}  // namespace yk
