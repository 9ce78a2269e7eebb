// fgemm_dev.h — device code of the fused verify GEMM (launched by
// k_fgemm.hip).
//
//   out_s[m, n] = epi( sum_k y[m, k] * dequant(W_s)[n, k] ),  m < rows <= 16
//
// One launch covers up to four weight matrices ("segments") that read the
// same activation rows — the q/k/v/z/alpha/beta projections of a layer, or
// the FFN gate/up pair — so a layer's projections cost one launch instead of
// one per matrix plus a quantization pass and a split-K reduction.
//
// y is x, or RMSNorm(x) * g when a norm weight is given
// (model/qwen35/forward.go:460-482 rmsNorm). The norm is applied as
//   y @ W^T = inv_rms(x) * ((x * g) @ W^T)
// so the activations are quantized without waiting for the row sum of
// squares; inv_rms (float64 sum, the reference's formula) scales the result.
//
// Per workgroup (512 threads = 8 waves):
//  * Prologue: x * g is quantized into LDS — one int16 value per element,
//    split into two int8 planes (q = 256 h + l), one scale per row and
//    256-element super-block (max |x| over it), and the exact int16 sums of
//    every 32-element sub-block (Q4_K min term). A lane quantizes one
//    8-element slice; a wave does two (row, super-block) units at a time.
//  * Main loop: the workgroup owns 16*TT output rows; its eight waves split
//    the super-blocks of K. Weights are read straight from HBM into registers
//    in MFMA operand order — lane (r, g) loads bytes [8g, 8g + 8) of each
//    32-byte quant group of row r — with later super-blocks' loads in flight
//    while the current one is multiplied. No LDS staging of weights and no
//    barriers inside the loop.
//  * Per 32-element sub-block the int32 MFMA result is scaled by the integer
//    sub-block scale in int32 (exact); per super-block d, dmin and the
//    activation scale are applied in FP32.
//  * Epilogue: the eight waves' partial sums are added in a fixed order
//    through LDS (deterministic), then stored, added to a residual, or
//    combined as SiLU(gate) * up.
//  * Launches whose activations fit LDS in one piece are persistent: each
//    workgroup quantizes once and then walks several row groups.
//
// Replaces, for the verify shapes, the reference's per-matrix quantized GEMV
// launches (kernels/hip/gemm/lm_head.hip:61-173 via bridge.cpp:3348-3371 and
// the qwen35 plan's per-projection ops, engine/gpu/plan.go).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdlib>

#include "fgemm.h"
#include "refmath.h"

namespace yk {
namespace {

typedef __attribute__((ext_vector_type(4))) int i32x4;
typedef short __attribute__((ext_vector_type(2))) s16x2;

constexpr int kQ4K = YUUKA_DTYPE_Q4_K;
constexpr int kQ6K = YUUKA_DTYPE_Q6_K;
constexpr int kQMax = 32639;  // |q| bound that keeps the high plane in int8
constexpr int kWaves = kFusedWaves;
constexpr int kThreads = 64 * kWaves;
// 1/rms of the rows: 16 floats per wave
constexpr uint32_t kInvBytes = kWaves * 16 * 4;
// Tiles per workgroup up to which the streaming kernel deals items to waves
// one by one (balanced mode, wk = 0).
constexpr int kBalMax = 4;



// Workgroup barrier that orders LDS only. __syncthreads() also fences
// global memory, which makes every wave wait for all of its outstanding
// weight loads at the barrier; the kernels here share data between waves
// through LDS alone (activation copies into LDS are waited for by the wave
// that issued them before it reaches a barrier).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ i32x4 mfma_i8(int64_t a, int64_t b) {
    const i32x4 zero = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, zero, 0, 0, 0);
}

// Plain 24-bit multiply-add. (Inline v_mad_i32_i24 asm reading MFMA results
// skips the compiler's MFMA-to-VALU wait states; keep this in C.)
__device__ __forceinline__ int mad24(int a, int b, int c) { return __mul24(a, b) + c; }

__device__ __forceinline__ int dot2(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s16x2, a), __builtin_bit_cast(s16x2, b), c, false);
}

__device__ __forceinline__ float half_lo(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)(h & 0xffffu))); }

// Signed q - 32 for eight packed unsigned 6-bit values (one per byte).
__device__ __forceinline__ uint64_t q6_to_i8(uint64_t q6) {
    const uint64_t t = q6 ^ 0x2020202020202020ull;
    const uint64_t s = t & 0x2020202020202020ull;
    return t | (s << 1) | (s << 2);
}

// Cross-lane steps on the DPP path (no LDS round trip): quad_perm [1,0,3,2]
// and [2,3,0,1] pair lanes at distance 1 and 2, row_ror 4 / 8 rotate inside
// a 16-lane row.
template <int CTRL>
__device__ __forceinline__ int dpp(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, true); }
template <int CTRL>
__device__ __forceinline__ float dppf(float v) { return __int_as_float(dpp<CTRL>(__float_as_int(v))); }
__device__ __forceinline__ float rdl(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }

// Maximum / sum over each 16-lane row, in every lane of the row.
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dppf<0xb1>(v));
    v = fmaxf(v, dppf<0x4e>(v));
    v = fmaxf(v, dppf<0x124>(v));
    return fmaxf(v, dppf<0x128>(v));
}
__device__ __forceinline__ float row_sum(float v) {
    v += dppf<0xb1>(v);
    v += dppf<0x4e>(v);
    v += dppf<0x124>(v);
    return v + dppf<0x128>(v);
}
// float64 sum over each 16-lane row, in every lane of the row.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t b = __double_as_longlong(v);
    const int lo = dpp<CTRL>((int)(uint32_t)b), hi = dpp<CTRL>((int)(uint32_t)(b >> 32));
    return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}
__device__ __forceinline__ double row_sum_d(double v) {
    v += dpp_d<0xb1>(v);
    v += dpp_d<0x4e>(v);
    v += dpp_d<0x124>(v);
    return v + dpp_d<0x128>(v);
}

// Sum over each quad, in every lane of the quad.
__device__ __forceinline__ int quad_sum(int v) {
    v += dpp<0xb1>(v);
    return v + dpp<0x4e>(v);
}

// LDS layout of one K chunk, RHO = 2 * rows live A rows (h plane rows
// 0..rows-1, l plane rows rows..2rows-1), RHOP = 16 * NA:
//   raw    [cap][rows][256] float    (the chunk's x, copied straight from HBM)
//   graw   [cap][256] float          (the chunk's norm weights)
//   zraw   [cap][rows][256] float    (the chunk's gate values, gated mode)
//   planes [cap * 8 sub-blocks][4 slices][RHO][8 B]
//   sums   [cap][RHOP][8] int16      (sub-block sums of each plane row)
//   xs     [cap][RHOP] float         (activation scale of each plane row)
//   nsq    [rows][nsb] float         (per super-block sums of x^2, norm)
//   junk   8 B per lane              (stores of units past the end)
// The tables hold `cap` super-blocks (the chunk capacity); `cnt` of them are
// live in the current chunk.
struct ActLayout {
    int rho, rhop, cap, cnt;
    uint32_t raw, graw, zraw, planes, sums, xs, nsq, junk, total;
    // staged: the raw copies of x (and g, z) live in LDS (act_fetch); the
    // streaming kernel keeps them in registers instead.
    __host__ __device__ ActLayout(int rows, int na, int cap_, int nsb, bool norm, int cnt_ = -1, bool gated = false,
                                  bool staged = true)
        : rho(2 * rows), rhop(16 * na), cap(cap_), cnt(cnt_ < 0 ? cap_ : cnt_) {
        raw = 0;
        graw = raw + (staged ? (uint32_t)cap * rows * 1024 : 0u);
        zraw = graw + (staged && norm ? (uint32_t)cap * 1024 : 0u);
        planes = zraw + (staged && gated ? (uint32_t)cap * rows * 1024 : 0u);
        sums = planes + (uint32_t)cap * 8 * 4 * rho * 8;
        xs = sums + (uint32_t)cap * rhop * 16;
        nsq = xs + (uint32_t)cap * rhop * 4;
        junk = nsq + (uint32_t)rows * nsb * 4;
        total = (junk + 512 + 15) & ~15u;
    }
};

typedef __attribute__((address_space(3))) void *lds_ptr_t;

// One wave-wide 16-byte-per-lane copy from global memory straight into LDS
// (lane l writes [dst + 16 l, +16)). Written as inline assembly so that the
// compiler's wait-count tracking does not see it: otherwise it waits for
// every outstanding vector load (the weight stream) before any later LDS
// access, as it cannot tell which loads target LDS. Callers wait for the
// copy themselves (s_waitcnt vmcnt) before reading it; the copies are
// issued before the weight loads, so the compiler's own counts for those
// stay exact (loads it does not know of only make its waits longer).
__device__ __forceinline__ void lds_copy16(const float *src, uint8_t *lds, uint32_t dst) {
    const uint32_t base = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds + dst));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(base) : "memory", "m0");
}

// Issues the chunk's activation (and norm weight) copies into LDS: one
// 1 KB wave load per (row, super-block), no registers held.
__device__ __forceinline__ void act_fetch(const FusedGemmArgs &A, const ActLayout &L, uint8_t *lds, int c0) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int M = A.rows;
    const int xunits = M * L.cnt, gunits = A.norm ? L.cnt : 0, zunits = A.gate ? xunits : 0;
    for (int u = wave; u < xunits + gunits + zunits; u += kWaves) {
        const float *src;
        uint32_t dst;
        if (u < xunits) {
            const int m = u / L.cnt, sbl = u - m * L.cnt;
            src = A.x + (size_t)m * A.K + (size_t)(c0 + sbl) * 256 + lane * 4;
            dst = L.raw + (uint32_t)(sbl * M + m) * 1024;
        } else if (u >= xunits + gunits) {
            const int uz = u - xunits - gunits;
            const int m = uz / L.cnt, sbl = uz - m * L.cnt;
            src = A.gate + (size_t)m * A.K + (size_t)(c0 + sbl) * 256 + lane * 4;
            dst = L.zraw + (uint32_t)(sbl * M + m) * 1024;
        } else {
            const int sbl = u - xunits;
            src = A.norm + (size_t)(c0 + sbl) * 256 + lane * 4;
            dst = L.graw + (uint32_t)sbl * 1024;
        }
        lds_copy16(src, lds, dst);
    }
}

// Row reductions (every lane of each 16-lane DPP row receives the row's
// result) for the prologue: unsigned maximum, FP32 and FP64 sums.
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
    v = max(v, (uint32_t)dpp<0xb1>((int)v));
    v = max(v, (uint32_t)dpp<0x4e>((int)v));
    v = max(v, (uint32_t)dpp<0x124>((int)v));
    return max(v, (uint32_t)dpp<0x128>((int)v));
}
// Sum over each group of 8 lanes (quad sums, then the mirrored half row).
__device__ __forceinline__ int oct_sum(int v) {
    v += dpp<0xb1>(v);
    v += dpp<0x4e>(v);
    return v + dpp<0x141>(v);
}
__device__ __forceinline__ uint32_t rl_u(uint32_t v, int l) { return (uint32_t)__builtin_amdgcn_readlane((int)v, l); }
__device__ __forceinline__ double rl_d(double v, int l) {
    const uint64_t b = __double_as_longlong(v);
    const uint32_t lo = rl_u((uint32_t)b, l), hi = rl_u((uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// x * inv rounded to the nearest integer q and offset by 128 sits in the low
// bits of this FP32 sum: bits = 0x4B400000 + q + 128 for |q| < 2^22, so byte 1
// is the high plane h = (q + 128) >> 8 and byte 0 XOR 0x80 the low plane
// l = q - 256 h (one fused multiply-add per element, round to nearest even).
constexpr float kRoundMagic = 12582912.0f + 128.0f;

// Quantizes super-blocks [c0, c0 + cnt) of every row from the LDS copy made
// by act_fetch. A (row, super-block) unit is one wave's work: lane s holds
// elements [4s, 4s + 4), i.e. sub-block s / 8, MFMA slice (s / 2) % 4, bytes
// 4 (s % 2) .. +4 of that slice. Reductions stay inside DPP rows; the four row
// results combine through readlane into scalars. Wave w owns units w, w + 8,
// ... (row-major over the chunk). The loop body is straight-line code over
// kUnits units at once (independent dependency chains interleave); units
// past the end are computed on a clamped index and their stores go to a
// per-lane scratch slot. MODE: 0 y = x, 1 y = x * g (RMSNorm weight, sums of
// x^2 recorded), 2 gated head norm.
template <int MODE>
__device__ __forceinline__ void act_prologue_m(const FusedGemmArgs &A, const ActLayout &L, uint8_t *lds, int c0,
                                               int nsb, float4 hw) {
    constexpr int kUnits = 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int M = A.rows;
    const int total = M * L.cnt;
    const int j = lane >> 3, g = (lane >> 1) & 3, hf = lane & 1;
    const uint32_t junk = L.junk + (uint32_t)lane * 8;
    const float *raw = reinterpret_cast<const float *>(lds + L.raw);
    const float *graw = reinterpret_cast<const float *>(lds + L.graw);
    const float *zraw = reinterpret_cast<const float *>(lds + L.zraw);
    for (int u0 = wave; u0 < total; u0 += kWaves * kUnits) {
        float v[kUnits][4], sq[kUnits];
        int m[kUnits], sbl[kUnits];
        bool live[kUnits];
#pragma unroll
        for (int k = 0; k < kUnits; k++) {
            const int u = min(u0 + kWaves * k, total - 1);
            live[k] = u0 + kWaves * k < total;
            m[k] = u / L.cnt;
            sbl[k] = u - m[k] * L.cnt;
            const float4 x = *reinterpret_cast<const float4 *>(raw + (sbl[k] * M + m[k]) * 256 + lane * 4);
            v[k][0] = x.x; v[k][1] = x.y; v[k][2] = x.z; v[k][3] = x.w;
            sq[k] = 0.0f;
            if constexpr (MODE == 1) {
                const float4 w = *reinterpret_cast<const float4 *>(graw + sbl[k] * 256 + lane * 4);
                sq[k] = fmaf(v[k][3], v[k][3], fmaf(v[k][2], v[k][2], fmaf(v[k][1], v[k][1], v[k][0] * v[k][0])));
                v[k][0] = __fmul_rn(v[k][0], w.x); v[k][1] = __fmul_rn(v[k][1], w.y);
                v[k][2] = __fmul_rn(v[k][2], w.z); v[k][3] = __fmul_rn(v[k][3], w.w);
            }
            if constexpr (MODE == 2) {
                // gated head norm: lanes [32h, 32h + 32) hold head h (two DPP rows)
                const float4 z = *reinterpret_cast<const float4 *>(zraw + (sbl[k] * M + m[k]) * 256 + lane * 4);
                double ss = 0.0;
#pragma unroll
                for (int i = 0; i < 4; i++) ss += (double)v[k][i] * (double)v[k][i];
                ss = row_sum_d(ss);
                const double h0 = rl_d(ss, 15) + rl_d(ss, 31), h1 = rl_d(ss, 47) + rl_d(ss, 63);
                const double hs = lane < 32 ? h0 : h1;
                const float mean = (float)(hs / 128.0);
                const float scale = (float)(1.0 / sqrt((double)(mean + A.eps)));
                v[k][0] = __fmul_rn(__fmul_rn(v[k][0], __fmul_rn(scale, hw.x)), z.x);
                v[k][1] = __fmul_rn(__fmul_rn(v[k][1], __fmul_rn(scale, hw.y)), z.y);
                v[k][2] = __fmul_rn(__fmul_rn(v[k][2], __fmul_rn(scale, hw.z)), z.z);
                v[k][3] = __fmul_rn(__fmul_rn(v[k][3], __fmul_rn(scale, hw.w)), z.w);
            }
        }
#pragma unroll
        for (int k = 0; k < kUnits; k++) {
            // max |v| over the unit (non-negative floats order as integers)
            const uint32_t a = max(max(__float_as_uint(v[k][0]) & 0x7fffffffu, __float_as_uint(v[k][1]) & 0x7fffffffu),
                                   max(__float_as_uint(v[k][2]) & 0x7fffffffu, __float_as_uint(v[k][3]) & 0x7fffffffu));
            const uint32_t ar = row_max_u32(a);
            const float amax = __uint_as_float(max(max(rl_u(ar, 15), rl_u(ar, 31)), max(rl_u(ar, 47), rl_u(ar, 63))));
            // xs * inv ~ 1 keeps every value exact to the quantization step;
            // the reciprocal keeps |v * inv| <= kQMax + 2^-10, so no clamp.
            const float xs = amax * (1.0f / (float)kQMax);
            const float inv = amax > 0.0f ? (float)kQMax * __builtin_amdgcn_rcpf(amax) : 0.0f;
            uint32_t t[4];
#pragma unroll
            for (int i = 0; i < 4; i++) t[i] = __float_as_uint(fmaf(v[k][i], inv, kRoundMagic));
            const uint32_t hp = __builtin_amdgcn_perm(t[1], t[0], 0x0c0c0501u) | __builtin_amdgcn_perm(t[3], t[2], 0x05010c0cu);
            const uint32_t lp = (__builtin_amdgcn_perm(t[1], t[0], 0x0c0c0400u) | __builtin_amdgcn_perm(t[3], t[2], 0x04000c0cu)) ^
                                0x80808080u;
            const uint32_t slot = L.planes + ((uint32_t)((sbl[k] * 8 + j) * 4 + g) * L.rho + m[k]) * 8 + 4 * hf;
            *reinterpret_cast<uint32_t *>(lds + (live[k] ? slot : junk)) = hp;
            *reinterpret_cast<uint32_t *>(lds + (live[k] ? slot + (uint32_t)M * 8 : junk + 4)) = lp;
            // exact int16 sums of both planes per 32-element sub-block
            const int hs = oct_sum(__builtin_amdgcn_sdot4((int)hp, 0x01010101, 0, false));
            const int ls = oct_sum(__builtin_amdgcn_sdot4((int)lp, 0x01010101, 0, false));
            const bool lead = live[k] && (lane & 7) == 0;
            const uint32_t sh = L.sums + (((uint32_t)sbl[k] * L.rhop + m[k]) * 8 + j) * 2;
            const uint32_t sl = L.sums + (((uint32_t)sbl[k] * L.rhop + M + m[k]) * 8 + j) * 2;
            *reinterpret_cast<int16_t *>(lds + (lead ? sh : junk)) = (int16_t)hs;
            *reinterpret_cast<int16_t *>(lds + (lead ? sl : junk + 2)) = (int16_t)ls;
            const bool first = live[k] && lane == 0;
            const uint32_t xh = L.xs + ((uint32_t)sbl[k] * L.rhop + m[k]) * 4;
            const uint32_t xl = L.xs + ((uint32_t)sbl[k] * L.rhop + M + m[k]) * 4;
            *reinterpret_cast<float *>(lds + (first ? xh : junk)) = xs;
            *reinterpret_cast<float *>(lds + (first ? xl : junk + 4)) = xs;
            if constexpr (MODE == 1) {
                const float r = row_sum(sq[k]);
                const float tot = (rdl(r, 15) + rdl(r, 31)) + (rdl(r, 47) + rdl(r, 63));
                const uint32_t nq = L.nsq + (uint32_t)(m[k] * nsb + c0 + sbl[k]) * 4;
                *reinterpret_cast<float *>(lds + (first ? nq : junk)) = tot;
            }
        }
    }
    // rows past 2M of the padded tables read as zero
    float *xsv = reinterpret_cast<float *>(lds + L.xs);
    for (int idx = threadIdx.x; idx < L.cnt * L.rhop; idx += kThreads) {
        const int rho = idx % L.rhop;
        if (rho >= L.rho) {
            xsv[idx] = 0.0f;
            *reinterpret_cast<uint4 *>(lds + L.sums + (uint32_t)idx * 16) = make_uint4(0, 0, 0, 0);
        }
    }
}

// Head-norm weights of this lane's 4 prologue elements (position 4 (s % 32)
// in its head), gated mode only. Loaded at kernel start, before the weight
// stream, so that waiting for them does not wait for the weights.
__device__ __forceinline__ float4 head_norm_lane(const FusedGemmArgs &A) {
    if (!A.gate) return make_float4(0.f, 0.f, 0.f, 0.f);
    return *reinterpret_cast<const float4 *>(A.head_norm + (threadIdx.x & 31) * 4);
}

__device__ __forceinline__ void act_prologue(const FusedGemmArgs &A, const ActLayout &L, uint8_t *lds, int c0,
                                             int nsb, float4 hw) {
    if (A.gate) act_prologue_m<2>(A, L, lds, c0, nsb, hw);
    else if (A.norm) act_prologue_m<1>(A, L, lds, c0, nsb, hw);
    else act_prologue_m<0>(A, L, lds, c0, nsb, hw);
}

// Quantization of the streaming kernel's units from registers. A unit (row
// m, super-block sb: 256 elements) belongs to one 16-lane DPP row: lane s of
// the row holds elements [16 s, 16 s + 16), i.e. sub-block s / 2 and MFMA
// slices 2 (s % 2) and 2 (s % 2) + 1. Every reduction stays inside the row
// (no cross-row exchange). Unit-step k of wave w covers units 4 (w + 8 k) +
// row; xr[k][0..3] hold the lane's 16 values (gr: norm weights, zr: gate),
// loaded at kernel start before the weight stream. Units past the end
// compute on a clamped index and store to the per-lane scratch slot.
template <int MODE, int KS>
__device__ __forceinline__ void act_prologue_regs(const FusedGemmArgs &A, const ActLayout &L, uint8_t *lds, int nsb,
                                                  const float4 (&xr)[KS][4], const float4 (&gr)[KS][4],
                                                  const float4 (&zr)[KS][4], const float4 (&hw)[4]) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int s16 = lane & 15, row = lane >> 4;
    const int M = A.rows;
    const int total = M * nsb;
    const int j = s16 >> 1, g0 = (s16 & 1) * 2;
    const uint32_t junk = L.junk + (uint32_t)lane * 8;
#pragma unroll
    for (int k = 0; k < KS; k++) {
        if (4 * (wave + kWaves * k) >= total) break;  // wave-uniform
        const int uu = 4 * (wave + kWaves * k) + row;
        const bool live = uu < total;
        const int u = min(uu, total - 1);
        const int m = u / nsb, sbl = u - m * nsb;
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            v[4 * q + 0] = xr[k][q].x; v[4 * q + 1] = xr[k][q].y;
            v[4 * q + 2] = xr[k][q].z; v[4 * q + 3] = xr[k][q].w;
        }
        float sq = 0.0f;
        if constexpr (MODE == 1) {
#pragma unroll
            for (int i = 0; i < 16; i++) sq = fmaf(v[i], v[i], sq);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                v[4 * q + 0] = __fmul_rn(v[4 * q + 0], gr[k][q].x); v[4 * q + 1] = __fmul_rn(v[4 * q + 1], gr[k][q].y);
                v[4 * q + 2] = __fmul_rn(v[4 * q + 2], gr[k][q].z); v[4 * q + 3] = __fmul_rn(v[4 * q + 3], gr[k][q].w);
            }
        }
        if constexpr (MODE == 2) {
            // gated head norm: a 128-element head is 8 lanes
            double ss = 0.0;
#pragma unroll
            for (int i = 0; i < 16; i++) ss += (double)v[i] * (double)v[i];
            ss += dpp_d<0xb1>(ss);
            ss += dpp_d<0x4e>(ss);
            ss += dpp_d<0x141>(ss);
            const float mean = (float)(ss / 128.0);
            const float scale = (float)(1.0 / sqrt((double)(mean + A.eps)));
#pragma unroll
            for (int q = 0; q < 4; q++) {
                v[4 * q + 0] = __fmul_rn(__fmul_rn(v[4 * q + 0], __fmul_rn(scale, hw[q].x)), zr[k][q].x);
                v[4 * q + 1] = __fmul_rn(__fmul_rn(v[4 * q + 1], __fmul_rn(scale, hw[q].y)), zr[k][q].y);
                v[4 * q + 2] = __fmul_rn(__fmul_rn(v[4 * q + 2], __fmul_rn(scale, hw[q].z)), zr[k][q].z);
                v[4 * q + 3] = __fmul_rn(__fmul_rn(v[4 * q + 3], __fmul_rn(scale, hw[q].w)), zr[k][q].w);
            }
        }
        uint32_t a = 0;
#pragma unroll
        for (int i = 0; i < 16; i++) a = max(a, __float_as_uint(v[i]) & 0x7fffffffu);
        const float amax = __uint_as_float(row_max_u32(a));
        // xs * inv ~ 1 keeps every value exact to the quantization step;
        // the reciprocal keeps |v * inv| <= kQMax + 2^-10, so no clamp.
        const float xs = amax * (1.0f / (float)kQMax);
        const float inv = amax > 0.0f ? (float)kQMax * __builtin_amdgcn_rcpf(amax) : 0.0f;
        uint32_t t[16];
#pragma unroll
        for (int i = 0; i < 16; i++) t[i] = __float_as_uint(fmaf(v[i], inv, kRoundMagic));
        uint32_t hp[4], lp[4];
#pragma unroll
        for (int d = 0; d < 4; d++) {
            hp[d] = __builtin_amdgcn_perm(t[4 * d + 1], t[4 * d], 0x0c0c0501u) |
                    __builtin_amdgcn_perm(t[4 * d + 3], t[4 * d + 2], 0x05010c0cu);
            lp[d] = (__builtin_amdgcn_perm(t[4 * d + 1], t[4 * d], 0x0c0c0400u) |
                     __builtin_amdgcn_perm(t[4 * d + 3], t[4 * d + 2], 0x04000c0cu)) ^
                    0x80808080u;
        }
        // slices g0 (elements 0..7 of the lane) and g0 + 1 (8..15)
        const uint32_t s0 = L.planes + ((uint32_t)((sbl * 8 + j) * 4 + g0) * L.rho + m) * 8;
        const uint32_t s1 = s0 + (uint32_t)L.rho * 8;
        *reinterpret_cast<uint2 *>(lds + (live ? s0 : junk)) = make_uint2(hp[0], hp[1]);
        *reinterpret_cast<uint2 *>(lds + (live ? s1 : junk)) = make_uint2(hp[2], hp[3]);
        *reinterpret_cast<uint2 *>(lds + (live ? s0 + (uint32_t)M * 8 : junk)) = make_uint2(lp[0], lp[1]);
        *reinterpret_cast<uint2 *>(lds + (live ? s1 + (uint32_t)M * 8 : junk)) = make_uint2(lp[2], lp[3]);
        // exact int16 sums of both planes per 32-element sub-block (2 lanes)
        int hs = 0, ls = 0;
#pragma unroll
        for (int d = 0; d < 4; d++) {
            hs = __builtin_amdgcn_sdot4((int)hp[d], 0x01010101, hs, false);
            ls = __builtin_amdgcn_sdot4((int)lp[d], 0x01010101, ls, false);
        }
        hs += dpp<0xb1>(hs);
        ls += dpp<0xb1>(ls);
        const bool lead = live && (s16 & 1) == 0;
        const uint32_t sh = L.sums + (((uint32_t)sbl * L.rhop + m) * 8 + j) * 2;
        const uint32_t sl = L.sums + (((uint32_t)sbl * L.rhop + M + m) * 8 + j) * 2;
        *reinterpret_cast<int16_t *>(lds + (lead ? sh : junk)) = (int16_t)hs;
        *reinterpret_cast<int16_t *>(lds + (lead ? sl : junk + 2)) = (int16_t)ls;
        const bool first = live && s16 == 0;
        const uint32_t xh = L.xs + ((uint32_t)sbl * L.rhop + m) * 4;
        const uint32_t xl = L.xs + ((uint32_t)sbl * L.rhop + M + m) * 4;
        *reinterpret_cast<float *>(lds + (first ? xh : junk)) = xs;
        *reinterpret_cast<float *>(lds + (first ? xl : junk + 4)) = xs;
        if constexpr (MODE == 1) {
            const float tot = row_sum(sq);
            const uint32_t nq = L.nsq + (uint32_t)(m * nsb + sbl) * 4;
            *reinterpret_cast<float *>(lds + (first ? nq : junk)) = tot;
        }
    }
    // rows past 2M of the padded tables read as zero
    float *xsv = reinterpret_cast<float *>(lds + L.xs);
    for (int idx = threadIdx.x; idx < nsb * L.rhop; idx += kThreads) {
        const int rho = idx % L.rhop;
        if (rho >= L.rho) {
            xsv[idx] = 0.0f;
            *reinterpret_cast<uint4 *>(lds + L.sums + (uint32_t)idx * 16) = make_uint4(0, 0, 0, 0);
        }
    }
}

// Buffer offset past every weight range: loads there return zero and make
// no memory request.
constexpr uint32_t kOutOfRange = 0xC0000000u;

// Staged weight bytes of one 16-row tile for one super-block.
// K order of the weight and activation operands: MFMA lane group g holds
// the 8-byte chunk kperm(g) of each 32-element sub-block (0, 2, 1, 3). The
// product sums over K, so any order is exact as long as both operands
// follow it; this one lets a Q4_K lane load its quant bytes as 16-byte
// pieces (64 contiguous bytes of every channel per load).
__device__ __forceinline__ int kperm(int g) { return ((g & 1) << 1) | (g >> 1); }

struct Q4Stage {
    i32x4 hdr;      // d | dmin, 12 scale bytes
    uint4 q16[2];   // bytes [16 + 32 (2 h + (g >> 1)) + 16 (g & 1), +16) for h = 0, 1
};
// Q6_K blocks (210 B) are only 2-byte aligned: a stage holds the raw
// dword-aligned windows of its pieces as loaded, and the byte shift `sh`
// (0 or 2, the same for every piece of a lane) is applied when the stage is
// multiplied, so that issuing a stage never waits for its loads.
struct Q6Stage {
    uint32_t ql[4][3];  // [n][half]: window of bytes n*64 + half*32 + 8g
    uint32_t qh[2][3];  // window of bytes 128 + n*32 + 8g
    i32x4 sc;           // window of the 16 int8 scales
    uint32_t w4;        // the dword after it (holds d)
    uint32_t sh;
};

// Stage of a launch whose segments mix Q4_K and Q6_K (dtype uniform per tile).
struct MixStage {
    Q4Stage q4;
    Q6Stage q6;
    int dt;
};

template <int DT> struct StageOf;
template <> struct StageOf<kQ4K> { using T = Q4Stage; };
template <> struct StageOf<kQ6K> { using T = Q6Stage; };
template <> struct StageOf<0> { using T = MixStage; };

__device__ __forceinline__ void issue(Q4Stage &S, __amdgpu_buffer_rsrc_t rs, uint32_t row_off, int g) {
    S.hdr = __builtin_amdgcn_raw_buffer_load_b128(rs, row_off, 0, 0);
#pragma unroll
    for (int h = 0; h < 2; h++)
        S.q16[h] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, row_off + 16 + 32 * (2 * h + (g >> 1)) + 16 * (g & 1), 0, 0));
}

// The four 8-byte quant pieces of p-blocks 0..3 in the kperm order: lanes
// 0..31 loaded p-block 2 h, lanes 32..63 p-block 2 h + 1 (16 bytes each);
// one lane-half swap of each dword gives every lane its chunk of both.
__device__ __forceinline__ void q4_pieces(const Q4Stage &S, uint64_t (&qs)[4]) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const auto lo = __builtin_amdgcn_permlane32_swap(S.q16[h].x, S.q16[h].z, true, false);
        const auto hi = __builtin_amdgcn_permlane32_swap(S.q16[h].y, S.q16[h].w, true, false);
        qs[2 * h] = (uint64_t)lo[0] | ((uint64_t)hi[0] << 32);
        qs[2 * h + 1] = (uint64_t)lo[1] | ((uint64_t)hi[1] << 32);
    }
}

__device__ __forceinline__ void issue(Q6Stage &S, __amdgpu_buffer_rsrc_t rs, uint32_t row_off, int g) {
    typedef __attribute__((ext_vector_type(3))) int i32x3;
    const uint32_t base = row_off & ~3u;
    auto win = [&](uint32_t (&w)[3], uint32_t off) __attribute__((always_inline)) {
        const i32x3 v = __builtin_bit_cast(i32x3, __builtin_amdgcn_raw_buffer_load_b96(rs, base + off, 0, 0));
        w[0] = (uint32_t)v[0];
        w[1] = (uint32_t)v[1];
        w[2] = (uint32_t)v[2];
    };
#pragma unroll
    for (int n = 0; n < 2; n++) {
        win(S.ql[2 * n], n * 64 + 8 * kperm(g));
        win(S.ql[2 * n + 1], n * 64 + 32 + 8 * kperm(g));
        win(S.qh[n], 128 + n * 32 + 8 * kperm(g));
    }
    S.sc = __builtin_amdgcn_raw_buffer_load_b128(rs, base + 192, 0, 0);
    S.w4 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, base + 208, 0, 0);
    S.sh = row_off & 3u;
}

// The 8 bytes of a piece window at byte shift sh.
__device__ __forceinline__ uint64_t q6_piece(const uint32_t (&w)[3], uint32_t sh) {
    const uint32_t lo = __builtin_amdgcn_alignbyte(w[1], w[0], sh);
    const uint32_t hi = __builtin_amdgcn_alignbyte(w[2], w[1], sh);
    return (uint64_t)lo | ((uint64_t)hi << 32);
}

// One tile, one super-block: int32 sums per plane row, then the FP32 update
// acc += xs * (d * sum(sc * dot) - dmin * sum(min * xsum)).
template <int NA>
__device__ __forceinline__ void compute(const Q4Stage &S, const int64_t (&xa)[NA][8], const uint32_t (&sxp)[NA][4][4],
                                        const float (&xsr)[NA][4], float (&acc)[NA][4]) {
    const uint32_t h0 = (uint32_t)S.hdr[0], q0 = (uint32_t)S.hdr[1], q1 = (uint32_t)S.hdr[2], q2 = (uint32_t)S.hdr[3];
    const float d = half_lo(h0), dmin = half_lo(h0 >> 16);
    uint64_t qs[4];
    q4_pieces(S, qs);
    // getScaleMinK4 (tensor/quant.go:96-103) for all eight sub-blocks
    const uint32_t sc_lo = q0 & 0x3f3f3f3fu;
    const uint32_t sc_hi = (q2 & 0x0f0f0f0fu) | ((q0 >> 2) & 0x30303030u);
    const uint32_t mn_lo = q1 & 0x3f3f3f3fu;
    const uint32_t mn_hi = ((q2 >> 4) & 0x0f0f0f0fu) | ((q1 >> 2) & 0x30303030u);
    const uint32_t mp[4] = {__builtin_amdgcn_perm(0u, mn_lo, 0x0c010c00u), __builtin_amdgcn_perm(0u, mn_lo, 0x0c030c02u),
                            __builtin_amdgcn_perm(0u, mn_hi, 0x0c010c00u), __builtin_amdgcn_perm(0u, mn_hi, 0x0c030c02u)};
    int acci[NA][4];
#pragma unroll
    for (int a = 0; a < NA; a++)
#pragma unroll
        for (int i = 0; i < 4; i++) acci[a][i] = 0;
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const int64_t blo = (int64_t)(qs[p] & 0x0f0f0f0f0f0f0f0full);
        const int64_t bhi = (int64_t)((qs[p] >> 4) & 0x0f0f0f0f0f0f0f0full);
        const uint32_t scw = p < 2 ? sc_lo : sc_hi;
        const int s0 = (int)__builtin_amdgcn_ubfe(scw, 16 * (p & 1), 8);
        const int s1 = (int)__builtin_amdgcn_ubfe(scw, 16 * (p & 1) + 8, 8);
#pragma unroll
        for (int a = 0; a < NA; a++) {
            const i32x4 c0 = mfma_i8(xa[a][2 * p], blo);
            const i32x4 c1 = mfma_i8(xa[a][2 * p + 1], bhi);
#pragma unroll
            for (int i = 0; i < 4; i++) acci[a][i] = mad24(s1, c1[i], mad24(s0, c0[i], acci[a][i]));
        }
    }
#pragma unroll
    for (int a = 0; a < NA; a++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int mm = 0;
#pragma unroll
            for (int p = 0; p < 4; p++) mm = dot2(mp[p], sxp[a][i][p], mm);
            acc[a][i] += xsr[a][i] * (d * (float)acci[a][i] - dmin * (float)mm);
        }
}

template <int NA>
__device__ __forceinline__ void compute(const Q6Stage &S, const int64_t (&xa)[NA][8], const uint32_t (&)[NA][4][4],
                                        const float (&xsr)[NA][4], float (&acc)[NA][4], int g) {
    uint64_t ql[4], qh[2];
#pragma unroll
    for (int i = 0; i < 4; i++) ql[i] = q6_piece(S.ql[i], S.sh);
#pragma unroll
    for (int i = 0; i < 2; i++) qh[i] = q6_piece(S.qh[i], S.sh);
    uint32_t scv[4];
    scv[0] = __builtin_amdgcn_alignbyte((uint32_t)S.sc[1], (uint32_t)S.sc[0], S.sh);
    scv[1] = __builtin_amdgcn_alignbyte((uint32_t)S.sc[2], (uint32_t)S.sc[1], S.sh);
    scv[2] = __builtin_amdgcn_alignbyte((uint32_t)S.sc[3], (uint32_t)S.sc[2], S.sh);
    scv[3] = __builtin_amdgcn_alignbyte(S.w4, (uint32_t)S.sc[3], S.sh);
    const float d = half_lo(S.w4 >> (8 * S.sh));
    int acci[NA][4];
#pragma unroll
    for (int a = 0; a < NA; a++)
#pragma unroll
        for (int i = 0; i < 4; i++) acci[a][i] = 0;
    const bool first = kperm(g) < 2;  // lanes holding elements 0..15 of each 32
#pragma unroll
    for (int c = 0; c < 8; c++) {
        const int n = c >> 2, qd = c & 3;
        const uint64_t lo = (ql[2 * n + (qd & 1)] >> (4 * (qd >> 1))) & 0x0f0f0f0f0f0f0f0full;
        const uint64_t hi = ((qh[n] >> (2 * qd)) & 0x0303030303030303ull) << 4;
        const int64_t q = (int64_t)q6_to_i8(lo | hi);
        const int64_t b0 = first ? q : 0, b1 = first ? 0 : q;
        const uint32_t scw = scv[c >> 1];
        const int s0 = (int)(int8_t)__builtin_amdgcn_ubfe(scw, 16 * (c & 1), 8);
        const int s1 = (int)(int8_t)__builtin_amdgcn_ubfe(scw, 16 * (c & 1) + 8, 8);
#pragma unroll
        for (int a = 0; a < NA; a++) {
            const i32x4 c0 = mfma_i8(xa[a][c], b0);
            const i32x4 c1 = mfma_i8(xa[a][c], b1);
#pragma unroll
            for (int i = 0; i < 4; i++) acci[a][i] = mad24(s1, c1[i], mad24(s0, c0[i], acci[a][i]));
        }
    }
#pragma unroll
    for (int a = 0; a < NA; a++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[a][i] += xsr[a][i] * (d * (float)acci[a][i]);
}

// Super-block sb of the 16-row tile whose row 0 of this lane starts at
// row_off, in the stage's format.
__device__ __forceinline__ void issue_any(Q4Stage &S, __amdgpu_buffer_rsrc_t rs, uint32_t row_off, uint32_t sb, int g, int) {
    issue(S, rs, row_off + sb * 144u, g);
}
__device__ __forceinline__ void issue_any(Q6Stage &S, __amdgpu_buffer_rsrc_t rs, uint32_t row_off, uint32_t sb, int g, int) {
    issue(S, rs, row_off + sb * 210u, g);
}
__device__ __forceinline__ void issue_any(MixStage &S, __amdgpu_buffer_rsrc_t rs, uint32_t row_off, uint32_t sb, int g,
                                          int dt) {
    // both formats' loads are always issued, the other one at offsets past
    // the buffer (zero, no memory request): no branch around loads, so the
    // compiler never copies a stage whose loads are in flight
    S.dt = dt;
    const bool q4 = dt == kQ4K;
    issue(S.q4, rs, q4 ? row_off + sb * 144u : kOutOfRange, g);
    issue(S.q6, rs, q4 ? kOutOfRange : row_off + sb * 210u, g);
}
template <int NA>
__device__ __forceinline__ void compute_any(const Q4Stage &S, const int64_t (&xa)[NA][8], const uint32_t (&sxp)[NA][4][4],
                                            const float (&xsr)[NA][4], float (&acc)[NA][4], int) {
    compute<NA>(S, xa, sxp, xsr, acc);
}
template <int NA>
__device__ __forceinline__ void compute_any(const Q6Stage &S, const int64_t (&xa)[NA][8], const uint32_t (&sxp)[NA][4][4],
                                            const float (&xsr)[NA][4], float (&acc)[NA][4], int g) {
    compute<NA>(S, xa, sxp, xsr, acc, g);
}
template <int NA>
__device__ __forceinline__ void compute_any(const MixStage &S, const int64_t (&xa)[NA][8], const uint32_t (&sxp)[NA][4][4],
                                            const float (&xsr)[NA][4], float (&acc)[NA][4], int g) {
    if (S.dt == kQ4K) compute<NA>(S.q4, xa, sxp, xsr, acc);
    else compute<NA>(S.q6, xa, sxp, xsr, acc, g);
}

template <int NA>
__device__ __forceinline__ void load_act(const uint8_t *lds, const ActLayout &L, int sbl, int r, int g,
                                         int64_t (&xa)[NA][8], uint32_t (&sxp)[NA][4][4], float (&xsr)[NA][4],
                                         bool want_sums) {
#pragma unroll
    for (int a = 0; a < NA; a++) {
        // rows past 2M read the last plane row: MFMA output row i depends on
        // A row i only, and the outputs of those rows are never read (integer
        // products, so no NaN either); a branch per lane would cost moves
        const int rho = min(16 * a + r, L.rho - 1), gk = kperm(g);  // the weights' K order
#pragma unroll
        for (int j = 0; j < 8; j++)
            xa[a][j] = *reinterpret_cast<const int64_t *>(lds + L.planes + ((uint32_t)((sbl * 8 + j) * 4 + gk) * L.rho + rho) * 8);
        const float4 xv = *reinterpret_cast<const float4 *>(lds + L.xs + ((uint32_t)sbl * L.rhop + 16 * a + 4 * g) * 4);
        xsr[a][0] = xv.x;
        xsr[a][1] = xv.y;
        xsr[a][2] = xv.z;
        xsr[a][3] = xv.w;
        if (want_sums) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint4 sv = *reinterpret_cast<const uint4 *>(lds + L.sums + ((uint32_t)sbl * L.rhop + 16 * a + 4 * g + i) * 16);
                sxp[a][i][0] = sv.x;
                sxp[a][i][1] = sv.y;
                sxp[a][i][2] = sv.z;
                sxp[a][i][3] = sv.w;
            }
        }
    }
}

// Prefetch depth (super-blocks in flight per wave).
template <int DT, int TT> struct Depth { static constexpr int value = 2; };

// One K chunk: the wave's first super-blocks are requested before the
// activation prologue runs, so HBM latency overlaps the quantization; the
// rest stream through a ring of Depth register stages. Wave w owns the
// chunk's super-blocks w, w + kWaves, ...
template <int DT, int TT, int NA>
__device__ __forceinline__ void chunk_pass(const FusedGemmArgs &A, const ActLayout &L, uint8_t *lds, int c0, int nsb,
                                           const __amdgpu_buffer_rsrc_t (&rs)[TT], const uint32_t (&row_off)[TT],
                                           float (&acc)[TT][NA][4], bool prologue) {
    using Stage = typename StageOf<DT>::T;
    constexpr int D = Depth<DT, TT>::value;
    constexpr uint32_t blk = DT == kQ4K ? 144u : 210u;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;
    const int mine = wave < L.cnt ? (L.cnt - wave + kWaves - 1) / kWaves : 0;
    Stage st[D][TT];
    if (prologue) act_fetch(A, L, lds, c0);
#pragma unroll
    for (int d = 0; d < D; d++)
        if (d < mine) {
#pragma unroll
            for (int t = 0; t < TT; t++) issue(st[d][t], rs[t], row_off[t] + (uint32_t)(c0 + wave + kWaves * d) * blk, g);
        }
    if (prologue) {
        // the LDS copies (issued before the weights) are complete once the
        // counter drains; the weights are already in flight behind them
        __builtin_amdgcn_s_waitcnt(0);
        lds_barrier();
        act_prologue(A, L, lds, c0, nsb, head_norm_lane(A));
        lds_barrier();
    }
    for (int base = 0; base < mine; base += D) {
#pragma unroll
        for (int d = 0; d < D; d++) {
            const int i = base + d;
            // keeps this stage's activation reads from being hoisted into
            // the previous stage (that multiplies live registers)
            __builtin_amdgcn_sched_barrier(0);
            if (i < mine) {
                int64_t xa[NA][8];
                uint32_t sxp[NA][4][4];
                float xsr[NA][4];
                load_act<NA>(lds, L, wave + kWaves * i, r, g, xa, sxp, xsr, DT == kQ4K);
#pragma unroll
                for (int t = 0; t < TT; t++) {
                    if constexpr (DT == kQ4K) compute<NA>(st[d][t], xa, sxp, xsr, acc[t]);
                    else compute<NA>(st[d][t], xa, sxp, xsr, acc[t], g);
                }
                if (i + D < mine) {
#pragma unroll
                    for (int t = 0; t < TT; t++)
                        issue(st[d][t], rs[t], row_off[t] + (uint32_t)(c0 + wave + kWaves * (i + D)) * blk, g);
                }
            }
        }
    }
}

__device__ __forceinline__ float silu_mul(float g, float u) { return __fmul_rn(__fmul_rn(g, sigmoid_ref(g)), u); }

// Output map of a store epilogue (FusedSeg::act) for output row n.
__device__ __forceinline__ float out_map(const FusedSeg &S, float v, int n) {
    switch (S.act) {
    case 1: return silu_ref(v);
    case 2: return sigmoid_ref(v);
    case 3: return (float)exp((double)__fmul_rn(softplus_ref(__fadd_rn(v, S.p0[n])), S.p1[n]));
    default: return v;
    }
}

// TT: 16-row tiles per group (for SwiGLU, TT/2 gate tiles then TT/2 up tiles
// over the same rows). NA: 16-row A tiles (rows <= 8: 1, <= 16: 2).
// DTM: kQ4K or kQ6K for single-dtype launches, 0 for a per-segment switch.
// Row group `grp`: segment, first output row and the weight rows of its
// tiles (uniform per workgroup).
template <int TT>
struct GroupRows {
    int s, n0, N, dt;
    __amdgpu_buffer_rsrc_t rs[TT];
    uint32_t row_off[TT];
    __device__ __forceinline__ GroupRows(const FusedGemmArgs &A, int grp, int rows_out, bool swiglu, int r) {
        s = 0;
#pragma unroll
        for (int i = 1; i < kFusedMaxSeg; i++)
            if (i < A.nseg && grp >= A.seg[i].wg_begin) s = i;
        n0 = (grp - A.seg[s].wg_begin) * rows_out;
        N = A.seg[s].n;
        dt = A.seg[s].dtype;
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const FusedSeg &S = A.seg[swiglu && t >= TT / 2 ? 1 : s];
            const int tile_row = swiglu ? (t % (TT / 2)) * 16 : t * 16;
            const int n = min(n0 + tile_row + r, N - 1);
            rs[t] = __builtin_amdgcn_make_buffer_rsrc((void *)S.w, (short)0, (int)S.w_bytes, 0x00020000);
            row_off[t] = (uint32_t)n * S.row_bytes;
        }
    }
};

// inv_rms of every row from the per super-block sums of squares (float64
// sum in super-block order, the reference's formula).
__device__ __forceinline__ void compute_inv_rms(const FusedGemmArgs &A, const ActLayout &L0, const uint8_t *lds,
                                                float *inv_rms, int nsb) {
    if (A.norm && threadIdx.x < (unsigned)A.rows) {
        const float *nsq = reinterpret_cast<const float *>(lds + L0.nsq);
        double sum = 0.0;
        for (int sb = 0; sb < nsb; sb++) sum += (double)nsq[threadIdx.x * nsb + sb];
        const float mean = (float)(sum / (double)A.K);
        inv_rms[threadIdx.x] = (float)(1.0 / sqrt((double)(mean + A.eps)));
    }
}

// Fixed-order sum of the waves' partials of one group, then the epilogue.
template <int TT, int NA>
__device__ __forceinline__ void group_epilogue(const FusedGemmArgs &A, float *red, const float *inv_rms,
                                               const float (&acc)[TT][NA][4], int n0, int N, int s, int rows_out,
                                               bool swiglu) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int M = A.rows;
    lds_barrier();  // the previous group's partials are consumed
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int a = 0; a < NA; a++)
#pragma unroll
            for (int i = 0; i < 4; i++) red[(((wave * TT + t) * NA + a) * 4 + i) * 64 + lane] = acc[t][a][i];
    lds_barrier();
    auto partial = [&](int t, int rho, int col) {
        const int a = rho >> 4, g = (rho & 15) >> 2, i = rho & 3;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) v += red[(((w * TT + t) * NA + a) * 4 + i) * 64 + g * 16 + col];
        return v;
    };
    auto value = [&](int t, int m, int col) {
        float v = 256.0f * partial(t, m, col) + partial(t, M + m, col);
        if (A.norm) v *= inv_rms[m];
        return v;
    };
    for (int idx = threadIdx.x; idx < rows_out * M; idx += kThreads) {
        const int m = idx / rows_out, rr = idx % rows_out;
        const int n = n0 + rr;
        if (n >= N) continue;
        const int t = rr >> 4, col = rr & 15;
        const size_t o = (size_t)m * N + n;
        if (swiglu) {
            const float gv = value(t, m, col), uv = value(t + TT / 2, m, col);
            A.seg[0].out[o] = silu_mul(gv, uv);
        } else {
            float v = value(t, m, col);
            if (A.epilogue == kEpiResidual) v += A.seg[s].res[o];
            else v = out_map(A.seg[s], v, n);
            A.seg[s].out[o] = v;
        }
    }
}

// Vector-memory loads one weight stage issues per 16-row tile.
template <int DT> struct StageLoads { static constexpr int value = DT == kQ4K ? 5 : 8; };

// s_waitcnt for "at most N vector-memory loads outstanding" (export and LDS
// counters left alone).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// 1 / rms of row `lane` (lanes < rows) from the per super-block sums of
// squares (float64 sum in super-block order, the reference's formula).
__device__ __forceinline__ float lane_inv_rms(const FusedGemmArgs &A, const float *nsq, int nsb) {
    const int lane = threadIdx.x & 63;
    float inv = 1.0f;
    if (A.norm && lane < A.rows) {
        double sum = 0.0;
        for (int sb = 0; sb < nsb; sb++) sum += (double)nsq[lane * nsb + sb];
        const float mean = (float)(sum / (double)A.K);
        inv = (float)(1.0 / sqrt((double)(mean + A.eps)));
    }
    return inv;
}

// Ring mode's outputs: tile c of the workgroup's [t0, t1) belongs to row
// group (c - t0) % wr as its (c - t0) / wr-th tile; every output sums the
// row group's wk K-group partials in K-group order (deterministic), then
// the epilogue. The partial of (row group rg, K group kg, tile k) sits at
// red + ((rg wk + kg) niter + k) TT NA 256 floats.
template <int TT, int NA>
__device__ __forceinline__ void ring_epilogue(const FusedGemmArgs &A, const float *red, const float *my_inv, int t0,
                                              int t1, int wr, int wk, int niter, int rows_out, bool swiglu) {
    constexpr int kSlot = TT * NA * 256;
    const int M = A.rows, per_tile = rows_out * M;
    for (int idx = threadIdx.x; idx < (t1 - t0) * per_tile; idx += kThreads) {
        const int c = idx / per_tile, rem = idx - c * per_tile;
        const int m = rem / rows_out, rr = rem - m * rows_out;
        const GroupRows<TT> Gr(A, t0 + c, rows_out, swiglu, 0);
        const int n = Gr.n0 + rr;
        if (n >= Gr.N) continue;
        const int rg = c % wr, k = c / wr;
        const int t = rr >> 4, col = rr & 15;
        float val[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int tt = t + h * (TT / 2);
            const int ah = m >> 4, gh = (m & 15) >> 2, eh = m & 3;
            const int rl = M + m, al = rl >> 4, gl = (rl & 15) >> 2, el = rl & 3;
            float ph = 0.0f, pl = 0.0f;
            for (int kg = 0; kg < wk; kg++) {
                const float *p = red + ((size_t)(rg * wk + kg) * niter + k) * kSlot;
                ph += p[((tt * NA + ah) * 4 + eh) * 64 + gh * 16 + col];
                pl += p[((tt * NA + al) * 4 + el) * 64 + gl * 16 + col];
            }
            float v = 256.0f * ph + pl;
            if (A.norm) v *= my_inv[m];
            val[h] = v;
            if (!swiglu) break;
        }
        const size_t o = (size_t)m * Gr.N + n;
        if (swiglu) {
            A.seg[0].out[o] = silu_mul(val[0], val[1]);
        } else {
            float v = val[0];
            if (A.epilogue == kEpiResidual) v += A.seg[Gr.s].res[o];
            else v = out_map(A.seg[Gr.s], v, n);
            A.seg[Gr.s].out[o] = v;
        }
    }
}

// Balanced mode's outputs: every (tile, row, channel) of the workgroup's
// cnt tiles sums the eight waves' partials in wave order (deterministic),
// then the epilogue. Wave w's partial of tile c sits at red + (w kBalMax + c)
// TT NA 256 floats.
template <int TT, int NA>
__device__ __forceinline__ void bal_epilogue(const FusedGemmArgs &A, const float *red, const float *my_inv, int t0,
                                             int cnt, int rows_out, bool swiglu) {
    constexpr int kSlot = TT * NA * 256;
    const int M = A.rows, per_tile = rows_out * M;
    for (int idx = threadIdx.x; idx < cnt * per_tile; idx += kThreads) {
        const int c = idx / per_tile, rem = idx - c * per_tile;
        const int m = rem / rows_out, rr = rem - m * rows_out;
        const GroupRows<TT> Gr(A, t0 + c, rows_out, swiglu, 0);
        const int n = Gr.n0 + rr;
        if (n >= Gr.N) continue;
        const int t = rr >> 4, col = rr & 15;
        const float ir = my_inv[m];
        float val[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int tt = t + h * (TT / 2);
            const int ah = m >> 4, gh = (m & 15) >> 2, eh = m & 3;
            const int rl = M + m, al = rl >> 4, gl = (rl & 15) >> 2, el = rl & 3;
            float ph = 0.0f, pl = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; w++) {
                const float *wr_ = red + ((size_t)w * kBalMax + c) * kSlot;
                ph += wr_[((tt * NA + ah) * 4 + eh) * 64 + gh * 16 + col];
                pl += wr_[((tt * NA + al) * 4 + el) * 64 + gl * 16 + col];
            }
            float v = 256.0f * ph + pl;
            if (A.norm) v *= ir;
            val[h] = v;
            if (!swiglu) break;
        }
        const size_t o = (size_t)m * Gr.N + n;
        if (swiglu) {
            *(A.seg[0].out + o) = silu_mul(val[0], val[1]);
        } else {
            float v = val[0];
            if (A.epilogue == kEpiResidual) v += *(A.seg[Gr.s].res + o);
            else v = out_map(A.seg[Gr.s], v, n);
            *(A.seg[Gr.s].out + o) = v;
        }
    }
}

// Single-dtype launch (rows <= 8) whose quantized activations fit LDS in one
// piece. Workgroup b owns the contiguous row tiles [b G / R, (b + 1) G / R) of
// the G tiles (R workgroups), so tile counts differ by at most one. Its eight
// waves form A.wr row groups x A.wk K groups: row group rg takes the
// workgroup's tiles rg, rg + wr, ...; wave (rg, kg) owns super-blocks kg,
// kg + wk, ... of each. Each wave first loads its own activation units
// (rows x super-blocks, at most KU) into registers, then requests its first
// two weight stages, and quantizes its units while the weights are in
// flight (the compiler waits for the activation loads only: they are older).
// After one barrier the (tile, super-block) items stream through the two
// register stages (kRing) across tiles, so the next tile's weights are in
// flight while the current one is stored. With wk = 1 (large launches such as the
// LM head) a wave owns whole rows and stores its own results.
// Register stages of the weight ring (items in flight per wave).
// (one stage measured slower for the Q6_K LM head: 82 -> 88 us)
template <int DT, int TT> struct RingDepth {
    static constexpr int value = 2;
};

template <int DT, int TT, int KU, int MODE, bool BAL>
__device__ __forceinline__ void stream_groups(const FusedGemmArgs &A, uint8_t *lds, float *inv_w, float *red,
                                              int rows_out, bool swiglu) {
    constexpr int NA = 1;
    constexpr int kRing = RingDepth<DT, TT>::value;
    static_assert(kRing == 1 || kRing == 2, "one or two register stages");
    using Stage = typename StageOf<DT>::T;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r = lane & 15, g = lane >> 4;
    const int nsb = A.K / 256;
    // A.wk == 0 selects balanced mode; the row-group x K-group shape below is
    // only used by the ring path (the guard keeps the divisions defined)
    const int wk = BAL || A.wk < 1 ? 1 : A.wk, wr = kWaves / wk;
    const int rg = wave / wk, kg = wave - rg * wk;
    const ActLayout L(A.rows, NA, nsb, nsb, MODE == 1, -1, MODE == 2, false);
    const int mine = kg < nsb ? (nsb - kg + wk - 1) / wk : 0;  // super-blocks per tile
    const int G = A.groups, R = (int)gridDim.x, b = (int)blockIdx.x;
    const int t0 = (int)((int64_t)b * G / R), t1 = (int)((int64_t)(b + 1) * G / R);
    const int niter = (t1 - t0 + wr - 1) / wr;
    auto tile_of = [&](int k) __attribute__((always_inline)) { return t0 + k * wr + rg; };
    const int ntile = rg < t1 - t0 ? (t1 - t0 - rg + wr - 1) / wr : 0;
    const int total = ntile * mine;
    float *my_inv = inv_w + wave * 16;
    // ---- this wave's activation units: unit-step k, DPP row `row` holds unit
    //      4 (wave + 8 k) + row, lane s16 its elements [16 s16, +16)
    constexpr int KS = KU / 4;
    float4 xr[KS][4], gr[KS][4], zr[KS][4], hw[4];
    auto load_x = [&]() __attribute__((always_inline)) {
        const int units = A.rows * nsb;
        const int s16 = lane & 15, row = lane >> 4;
        if constexpr (MODE == 2) {
#pragma unroll
            for (int q = 0; q < 4; q++) hw[q] = *reinterpret_cast<const float4 *>(A.head_norm + (s16 & 7) * 16 + 4 * q);
        }
#pragma unroll
        for (int k = 0; k < KS; k++) {
            const int u = min(4 * (wave + kWaves * k) + row, units - 1);
            const int m = u / nsb, sb = u - m * nsb;
            const uint32_t off = (uint32_t)(m * A.K + sb * 256 + 16 * s16);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                xr[k][q] = *reinterpret_cast<const float4 *>(A.x + off + 4 * q);
                if constexpr (MODE == 1) gr[k][q] = *reinterpret_cast<const float4 *>(A.norm + sb * 256 + 16 * s16 + 4 * q);
                if constexpr (MODE == 2) zr[k][q] = *reinterpret_cast<const float4 *>(A.gate + off + 4 * q);
            }
        }
    };
    // the activations are requested first, then the first weight stages
    load_x();
    __builtin_amdgcn_sched_barrier(0);

    auto zero = [&](float (&acc)[TT][NA][4]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int a = 0; a < NA; a++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[t][a][e] = 0.0f;
    };
    auto compute_item = [&](const Stage (&S)[TT], int sb, float (&acc)[TT][NA][4]) __attribute__((always_inline)) {
        int64_t xa[NA][8];
        uint32_t sxp[NA][4][4];
        float xsr[NA][4];
        load_act<NA>(lds, L, sb, r, g, xa, sxp, xsr, DT != kQ6K);
#pragma unroll
        for (int t = 0; t < TT; t++) compute_any<NA>(S[t], xa, sxp, xsr, acc[t], g);
    };
    if constexpr (BAL) {
        // ---- balanced mode (at most kBalMax tiles per workgroup): the
        //      workgroup's (tile, super-block) items, tile-major, are dealt
        //      round-robin to the eight waves; each wave keeps one partial per
        //      tile in LDS, and every tile's outputs sum the eight partials in
        //      wave order after one barrier.
        const int cnt = t1 - t0, I = cnt * nsb;
        const int nmine = wave < I ? (I - wave + kWaves - 1) / kWaves : 0;
        // A ring slot past the wave's last item still issues its loads (a
        // fixed load count keeps the compiler's wait counts exact), at an
        // offset beyond the buffer's range: they return zero without a
        // memory request instead of re-reading a live item.
        auto issue_slot = [&](Stage (&S)[TT], int q) __attribute__((always_inline)) {
            const bool live = q < nmine;
            const int ii = live ? wave + q * kWaves : 0;
            const int c = ii / nsb, sb = ii - c * nsb;
            const GroupRows<TT> Gr(A, t0 + c, rows_out, swiglu, r);
#pragma unroll
            for (int t = 0; t < TT; t++)
                issue_any(S[t], Gr.rs[t], live ? Gr.row_off[t] : kOutOfRange, live ? (uint32_t)sb : 0u, g, Gr.dt);
        };
        constexpr int kSlot = TT * NA * 256;  // floats of one wave's partial of one tile
        float *myr = red + (size_t)wave * kBalMax * kSlot;
        // Register stages per wave: more weight requests in flight per CU
        // lower the stream rate (three or four stages made every launch
        // slower); two-tile items (FFN gate/up) run best with one stage, the
        // other launches with two.
        constexpr int kD = TT == 2 ? 1 : 2;
        Stage sbr[kD][TT];
        // issued unconditionally (under a branch the compiler's wait counts
        // lose track and the prologue would wait for these weights too)
#pragma unroll
        for (int d = 0; d < kD; d++) issue_slot(sbr[d], d);
        __builtin_amdgcn_sched_barrier(0);
        for (int idx = lane; idx < cnt * kSlot / 4; idx += 64)
            reinterpret_cast<float4 *>(myr)[idx] = make_float4(0.f, 0.f, 0.f, 0.f);
        act_prologue_regs<MODE, KS>(A, L, lds, nsb, xr, gr, zr, hw);
        lds_barrier();
        {
            const float v = lane_inv_rms(A, reinterpret_cast<const float *>(lds + L.nsq), nsb);
            if (lane < 16) my_inv[lane] = v;
        }
        float acc[TT][NA][4];
        zero(acc);
        auto flush = [&](int c) __attribute__((always_inline)) {
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int a = 0; a < NA; a++)
#pragma unroll
                    for (int e = 0; e < 4; e++) myr[c * kSlot + ((t * NA + a) * 4 + e) * 64 + lane] = acc[t][a][e];
        };
        int cur = nmine > 0 ? wave / nsb : 0;
        // two items per iteration, each stage in its own code path: a loop
        // over a switch on q % kD lets the compiler merge the cases and
        // rotate the stages through register copies, each of which waits
        // for the loads in flight
        auto step = [&](Stage (&S)[TT], int q) __attribute__((always_inline)) {
            // q >= nmine (the last round of a count that kD does not divide):
            // a stage issued past the end, all-zero weights; it multiplies
            // into the current tile's partial exactly
            const int qq = min(q, nmine - 1);
            const int ii = wave + kWaves * qq, c = ii / nsb, sbi = ii - c * nsb;
            if (c != cur) {
                flush(cur);
                zero(acc);
                cur = c;
            }
            compute_item(S, sbi, acc);
            __builtin_amdgcn_sched_barrier(0);
            issue_slot(S, q + kD);
        };
        for (int q = 0; q < nmine; q += kD) {
#pragma unroll
            for (int d = 0; d < kD; d++) step(sbr[d], q + d);
        }
        if (nmine > 0) flush(cur);
        lds_barrier();
        bal_epilogue<TT, NA>(A, red, my_inv, t0, cnt, rows_out, swiglu);
        return;
    }

    // ring item i of this wave: tile tile_of(i / mine), super-block
    // kg + wk (i % mine); items past the wave's last are issued at offsets
    // beyond the buffers (zero, no memory request) so that every issue is
    // unconditional
    auto issue_at = [&](Stage (&S)[TT], int i) __attribute__((always_inline)) {
        const bool live = i < total;
        const int k = live ? i / mine : 0, j = live ? i - k * mine : 0;
        const GroupRows<TT> Gr(A, tile_of(k), rows_out, swiglu, r);
#pragma unroll
        for (int t = 0; t < TT; t++)
            issue_any(S[t], Gr.rs[t], live ? Gr.row_off[t] : kOutOfRange, live ? (uint32_t)(kg + wk * j) : 0u, g,
                      Gr.dt);
    };
    Stage st[kRing][TT];
#pragma unroll
    for (int d = 0; d < kRing; d++) issue_at(st[d], d);
    __builtin_amdgcn_sched_barrier(0);
    act_prologue_regs<MODE, KS>(A, L, lds, nsb, xr, gr, zr, hw);
    lds_barrier();
    {
        const float v = lane_inv_rms(A, reinterpret_cast<const float *>(lds + L.nsq), nsb);
        if (lane < 16) my_inv[lane] = v;
    }
    // two items per iteration, each stage in its own code path (see the
    // balanced mode). A tile's partial goes to LDS after its last item and
    // every output is formed after the loop: an epilogue inside the loop
    // (global stores, residual loads) would make the compiler wait for the
    // weight loads in flight at each tile's end.
    constexpr int kSlot = TT * NA * 256;  // floats of one wave's partial of one tile
    float *myr = red + (size_t)(rg * wk + kg) * niter * kSlot;
    float acc[TT][NA][4];
    zero(acc);
    auto step = [&](Stage (&S)[TT], int i) __attribute__((always_inline)) {
        // an odd count's last pair holds one item past the end: its stage
        // was issued at offsets beyond the buffers (all-zero weights, so the
        // multiply adds exact zeros) and it stores no partial
        const bool live = i < total;
        const int k = live ? i / mine : 0, j = live ? i - k * mine : 0;
        compute_item(S, kg + wk * j, acc);
        // every read of the stage precedes its refill, so the refill can
        // take the stage's own registers (no copies of loads in flight)
        __builtin_amdgcn_sched_barrier(0);
        issue_at(S, i + kRing);
        if (live && j == mine - 1) {
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int a = 0; a < NA; a++)
#pragma unroll
                    for (int e = 0; e < 4; e++) myr[k * kSlot + ((t * NA + a) * 4 + e) * 64 + lane] = acc[t][a][e];
            zero(acc);
        }
    };
    for (int i = 0; i < total; i += kRing) {
#pragma unroll
        for (int d = 0; d < kRing; d++) step(st[d], i + d);
    }
    lds_barrier();
    ring_epilogue<TT, NA>(A, red, my_inv, t0, t1, wr, wk, niter, rows_out, swiglu);
}
}  // namespace

// ---- host-side shape of a streaming launch

// Compute units of the current device.
inline int device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 1;
    }
    return cus;
}

// Workgroups that are resident at once: a persistent grid never exceeds it,
// so no group waits for a second round.
inline unsigned resident_wgs(const void *fn, uint32_t lds) {
    const int cus = device_cus();
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kThreads, lds) != hipSuccess || per_cu <= 0)
        per_cu = 1;
    return (unsigned)(per_cu * cus);
}

// Streaming-kernel shape of a launch, or false when it takes the chunked path:
// one dtype, rows <= 8, 1 or 2 tiles, activation units per wave within the
// register bucket of the prologue mode, quantized activations in LDS.
// *balanced: at most kBalMax row tiles per workgroup (one workgroup per CU:
// 512 threads at more than 128 VGPRs).
inline bool stream_shape(const FusedGemmArgs &a, int tt, bool mixed, int *ku, int *mode, uint32_t *lds,
                         bool *balanced) {
    if (a.rows > 8 || (tt != 1 && tt != 2) || ((mixed || a.seg[0].dtype == kQ6K) && tt != 1)) return false;
    const int nsb = a.K / 256;
    *mode = a.gate ? 2 : (a.norm ? 1 : 0);
    *ku = (a.rows * nsb + kWaves - 1) / kWaves;
    const int cap = *mode == 2 ? 8 : (*mode == 1 ? 16 : 24);
    if (*ku > cap) return false;
    const ActLayout L(a.rows, 1, nsb, nsb, *mode == 1, -1, *mode == 2, false);
    const int R = std::min(a.groups, device_cus());
    *balanced = (a.groups + R - 1) / R <= kBalMax;
    *lds = L.total + kInvBytes + (uint32_t)kWaves * (*balanced ? kBalMax : 1) * tt * 4 * 64 * 4;
    return *lds <= kFusedLds;
}

// Row-group bookkeeping of a launch (segments' first groups, group count).
inline FusedGemmArgs with_groups(const FusedGemmArgs &a, int tt, unsigned *grid_out) {
    const int rows_out = a.epilogue == kEpiSwiglu ? 8 * tt : 16 * tt;
    FusedGemmArgs b = a;
    unsigned grid = 0;
    for (int i = 0; i < b.nseg; i++) {
        b.seg[i].wg_begin = (int)grid;
        if (b.epilogue == kEpiSwiglu && i == 1) {  // the up matrix shares the gate's groups
            b.seg[i].wg_begin = 1 << 30;
            continue;
        }
        grid += (unsigned)((b.seg[i].n + rows_out - 1) / rows_out);
    }
    b.groups = (int)grid;
    *grid_out = grid;
    return b;
}

}  // namespace yk
