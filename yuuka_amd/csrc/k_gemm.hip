// k_gemm.hip — verify GEMM for K-quant weights on gfx950 (wave64, int8 MFMA).
//
//   out[m, n] = sum_k x[m, k] * dequant(W)[n, k],   m < rows <= 16
//
// Replaces the reference's FP32-FMA streaming kernel
// (kernels/hip/gemm/lm_head.hip:61-173, launched from bridge.cpp:3348-3371).
//
// Scheme (all integer arithmetic is exact):
//  * x is quantized per row to q = round(x / xs) with |q| <= 32639 and split
//    into two int8 planes q = 256*h + l, h,l in [-128, 127]. Rows 0..M-1 of
//    the MFMA A operand carry h, rows M..2M-1 carry l (one 16-row A tile
//    holds both planes for M <= 8, two tiles for M <= 16).
//  * Weights are decoded to int8 in registers straight from the packed bytes
//    (Q4_K: the 4-bit quant; Q6_K: the signed 6-bit quant q-32) and fed as the
//    B operand of v_mfma_i32_16x16x32_i8. One MFMA covers one 32-element
//    Q4_K sub-block (one scale); Q6_K uses two MFMAs per 32 elements, each
//    with the other 16-element scale group zeroed.
//  * Per sub-block the int32 MFMA result is multiplied by the integer 6/8-bit
//    scale and accumulated in int32 (exact); the Q4_K min term uses the exact
//    integer sums of the quantized activations per sub-block. Only the
//    per-super-block fp16 scale d (and dmin) is applied in FP32.
//  * Each wave owns 64 output rows (four 16-row tiles, so every A operand is
//    reused four times) and a contiguous range of 256-element super-blocks.
//    The wave stages the 64 rows' bytes of one super-block in LDS with
//    coalesced 128-bit buffer loads (out-of-range bytes read as zero), then
//    reads them back in MFMA layout. The four waves of a workgroup split K;
//    larger K is also split across workgroups, and the last workgroup of a
//    64-row block (atomic ticket) sums the partials in a fixed order, so the
//    result is deterministic.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <algorithm>
#include <cstdlib>

#include "internal.h"

namespace yk {
namespace {

typedef __attribute__((ext_vector_type(4))) int i32x4;

constexpr int kQ4K = YUUKA_DTYPE_Q4_K;
constexpr int kQ6K = YUUKA_DTYPE_Q6_K;
constexpr int kQMax = 32639;  // keeps the high plane within int8

// Bytes of one staged row block in LDS: Q4_K blocks are 144 B and 16-byte
// aligned; Q6_K blocks are 210 B and only 2-byte aligned, so 224 B are staged
// from the 16-byte boundary below the block.
template <int DT> struct Fmt;
template <> struct Fmt<kQ4K> { static constexpr int block = 144, chunks = 9; };
template <> struct Fmt<kQ6K> { static constexpr int block = 210, chunks = 14; };

// --------------------------------------------------------------------------
// Activation quantizer: one workgroup per row.
// Layout written (bytes, base xq):
//   [0, 64)            float xs[16] (row scales; x ~= xs * q)
//   [64, 64 + A)       int8 planes [na][K/8][16][8]
//   [64 + A, ...)      int32 sub-block sums [na][K/32][16]
// where A = na * K * 16 and row rho of tile a is rho = 16a + r.
// --------------------------------------------------------------------------
// One thread per 8-element K slice; grid (rows, ceil(K/2048)). Every
// workgroup recomputes its row's maximum (the row is L2-resident).
__global__ __launch_bounds__(256) void quantize_x_kernel(const float *__restrict__ x, int K,
                                                         int M, int na, uint8_t *__restrict__ xq) {
    const int m = blockIdx.x;
    const float *row = x + (size_t)m * K;
    __shared__ float red[4];
    float amax = 0.0f;
    for (int k = threadIdx.x * 4; k < K; k += 1024) {
        const float4 v = *reinterpret_cast<const float4 *>(row + k);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float xs = amax > 0.0f ? amax / (float)kQMax : 0.0f;
    const float inv = amax > 0.0f ? (float)kQMax / amax : 0.0f;
    float *scales = reinterpret_cast<float *>(xq);
    int8_t *planes = reinterpret_cast<int8_t *>(xq + 64);
    // int16 sub-block sums [na][K/256][16 rho][8 sub-blocks]
    int16_t *sums = reinterpret_cast<int16_t *>(xq + 64 + (size_t)na * K * 16);
    if (blockIdx.y == 0 && threadIdx.x == 0) scales[m] = xs;
    const int rho_h = m, rho_l = M + m;
    const int ks = blockIdx.y * 256 + threadIdx.x;  // K slice of 8 elements
    const bool live = ks < K / 8;
    int sh = 0, sl = 0;
    if (live) {
        uint64_t ph = 0, pl = 0;
        const float4 a = *reinterpret_cast<const float4 *>(row + ks * 8);
        const float4 b = *reinterpret_cast<const float4 *>(row + ks * 8 + 4);
        const float v8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float v = rintf(v8[i] * inv);
            v = fminf(fmaxf(v, -(float)kQMax), (float)kQMax);
            const int q = (int)v;
            const int h = (q + 128) >> 8;
            const int l = q - h * 256;
            sh += h;
            sl += l;
            ph |= (uint64_t)(uint8_t)(int8_t)h << (8 * i);
            pl |= (uint64_t)(uint8_t)(int8_t)l << (8 * i);
        }
        *reinterpret_cast<uint64_t *>(planes + ((size_t)(rho_h / 16) * (K / 8) + ks) * 128 + (rho_h % 16) * 8) = ph;
        *reinterpret_cast<uint64_t *>(planes + ((size_t)(rho_l / 16) * (K / 8) + ks) * 128 + (rho_l % 16) * 8) = pl;
    }
    // four consecutive slices form one 32-element sub-block
    sh += __shfl_xor(sh, 1);
    sh += __shfl_xor(sh, 2);
    sl += __shfl_xor(sl, 1);
    sl += __shfl_xor(sl, 2);
    if (live && (ks & 3) == 0) {
        const int s = ks >> 2;
        sums[((size_t)(rho_h / 16) * (K / 256) + s / 8) * 128 + (rho_h % 16) * 8 + s % 8] = (int16_t)sh;
        sums[((size_t)(rho_l / 16) * (K / 256) + s / 8) * 128 + (rho_l % 16) * 8 + s % 8] = (int16_t)sl;
    }
    // Unused rows of the last tile are zero (row 0's workgroups write them).
    if (m == 0 && live) {
        for (int rho = 2 * M; rho < 16 * na; rho++) {
            *reinterpret_cast<uint64_t *>(planes + ((size_t)(rho / 16) * (K / 8) + ks) * 128 + (rho % 16) * 8) = 0;
            if ((ks & 3) == 0) {
                const int sbk = ks >> 2;
                sums[((size_t)(rho / 16) * (K / 256) + sbk / 8) * 128 + (rho % 16) * 8 + sbk % 8] = 0;
            }
        }
    }
}

__device__ __forceinline__ i32x4 mfma_i8(int64_t a, int64_t b) {
    const i32x4 zero = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, zero, 0, 0, 0);
}

__device__ __forceinline__ int mad24(int a, int b, int c) { return __mul24(a, b) + c; }

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)h));
}

// Reads 8 bytes at a 2-byte aligned byte offset `off` of the LDS array.
__device__ __forceinline__ uint64_t lds_read8_a2(const uint8_t *lds_base, int off) {
    const uint32_t *w = reinterpret_cast<const uint32_t *>(lds_base + (off & ~3));
    const uint32_t w0 = w[0], w1 = w[1], w2 = w[2];
    const uint32_t lo = __builtin_amdgcn_alignbyte(w1, w0, off & 3);
    const uint32_t hi = __builtin_amdgcn_alignbyte(w2, w1, off & 3);
    return (uint64_t)lo | ((uint64_t)hi << 32);
}

// Signed 6-bit q-32 for eight packed 6-bit values (one per byte).
__device__ __forceinline__ uint64_t q6_to_i8(uint64_t q6) {
    const uint64_t t = q6 ^ 0x2020202020202020ull;
    const uint64_t s = t & 0x2020202020202020ull;
    return t | (s << 1) | (s << 2);
}

template <int DT, int NA>
struct Layout {
    static constexpr int W_BYTES = 64 * Fmt<DT>::chunks * 16;        // staged weights
    static constexpr int XA_BYTES = NA * 4096;                        // int8 planes, one super-block
    static constexpr int SX_BYTES = DT == kQ4K ? NA * 512 : 0;        // sub-block sums
    static constexpr int WAVE_BYTES = W_BYTES + XA_BYTES + SX_BYTES;
    static constexpr int XA_LOADS = NA * 4;                           // 16 B per lane each
    static constexpr int SX_LOADS = DT == kQ4K ? (NA * 512 + 1023) / 1024 : 0;
};

template <int DT, int NA>
__global__ __launch_bounds__(256) void gemm_kq_kernel(const uint8_t *__restrict__ w,
                                                      uint32_t w_bytes, uint32_t row_bytes,
                                                      const uint8_t *__restrict__ xq,
                                                      float *out, int N, int K,
                                                      int M, int splits, int spw,
                                                      float *__restrict__ partials, const float *residual) {
    using L = Layout<DT, NA>;
    constexpr int BB = Fmt<DT>::block;
    constexpr int CH = Fmt<DT>::chunks;
    constexpr int STRIDE = CH * 16;  // LDS bytes per staged row
    extern __shared__ __align__(16) uint8_t lds[];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int r = lane & 15;
    const int g = lane >> 4;
    const int rb = blockIdx.x / splits;
    const int split = blockIdx.x % splits;
    const int n_base = rb * 64;
    const int nsb = K / 256;
    const int sb_begin = (split * 4 + wave) * spw;
    const int iters = spw;  // identical trip count in every wave

    const int wave_off = wave * L::WAVE_BYTES;
    uint8_t *stage = lds + wave_off;
    const int xa_off = wave_off + L::W_BYTES;
    const int sx_off = xa_off + L::XA_BYTES;
    const float *xs = reinterpret_cast<const float *>(xq);
    const uint8_t *planes = xq + 64;
    const uint8_t *sums = xq + 64 + (size_t)NA * K * 16;

    // Out-of-range chunks read as zero; the bound is rounded up to the
    // 16-byte granule of the last valid byte, so no valid byte is dropped.
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)w, (short)0, (int)((w_bytes + 15u) & ~15u), 0x00020000);

    float acc[4][NA][4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int a = 0; a < NA; a++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[t][a][i] = 0.0f;

    // Registers of the super-block in flight: weights (chunk c = lane + 64 i),
    // activation planes and sums (contiguous per super-block).
    i32x4 pre[CH];
    i32x4 pre_xa[L::XA_LOADS];
    i32x4 pre_sx[L::SX_LOADS > 0 ? L::SX_LOADS : 1];

    auto issue = [&](int sb) {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int c = lane + 64 * i;
            const int row = c / CH;
            const int part = c % CH;
            int n = n_base + row;
            if (n >= N) n = N - 1;
            const uint32_t start = (uint32_t)n * row_bytes + (uint32_t)sb * BB;
            pre[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (start & ~15u) + part * 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < L::XA_LOADS; i++) {
            const int a = i >> 2, part = i & 3;
            pre_xa[i] = *reinterpret_cast<const i32x4 *>(planes + ((size_t)a * (K / 8) + (size_t)sb * 32) * 128 +
                                                         part * 1024 + lane * 16);
        }
#pragma unroll
        for (int i = 0; i < L::SX_LOADS; i++) {
            const int byte = i * 1024 + lane * 16;
            if (byte < L::SX_BYTES) {
                const int a = byte / 512, rem = byte % 512;
                pre_sx[i] = *reinterpret_cast<const i32x4 *>(sums + ((size_t)a * (K / 32) + (size_t)sb * 8) * 64 + rem);
            }
        }
    };
    auto commit = [&]() {
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int c = lane + 64 * i;
            *reinterpret_cast<i32x4 *>(stage + (c / CH) * STRIDE + (c % CH) * 16) = pre[i];
        }
#pragma unroll
        for (int i = 0; i < L::XA_LOADS; i++)
            *reinterpret_cast<i32x4 *>(lds + xa_off + i * 1024 + lane * 16) = pre_xa[i];
#pragma unroll
        for (int i = 0; i < L::SX_LOADS; i++) {
            const int byte = i * 1024 + lane * 16;
            if (byte < L::SX_BYTES) *reinterpret_cast<i32x4 *>(lds + sx_off + byte) = pre_sx[i];
        }
    };

    if (sb_begin < nsb) issue(sb_begin);
    for (int it = 0; it < iters; it++) {
        const int sb = sb_begin + it;
        const bool active = sb < nsb;
        __syncthreads();  // previous super-block's LDS reads are done
        if (active) commit();
        __syncthreads();  // staged bytes visible to the whole wave
        if (active && it + 1 < iters && sb + 1 < nsb) issue(sb + 1);
        if (!active) continue;

        // A operands for the 8 sub-blocks (K slice g of each), reused by all tiles.
        int64_t xa[NA][8];
        i32x4 sx[NA][8];
#pragma unroll
        for (int a = 0; a < NA; a++) {
#pragma unroll
            for (int s = 0; s < 8; s++) {
                xa[a][s] = *reinterpret_cast<const int64_t *>(lds + xa_off + a * 4096 + (s * 4 + g) * 128 + r * 8);
                if (DT == kQ4K)
                    sx[a][s] = *reinterpret_cast<const i32x4 *>(lds + sx_off + a * 512 + s * 64 + g * 16);
            }
        }

#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int row = 16 * t + r;
            int n = n_base + row;
            if (n >= N) n = N - 1;
            const uint32_t start = (uint32_t)n * row_bytes + (uint32_t)sb * BB;
            const int blk_off = (int)(wave_off + row * STRIDE + (start & 15u));
            const uint8_t *blk = lds + blk_off;
            if (DT == kQ4K) {
                const uint32_t *h32 = reinterpret_cast<const uint32_t *>(blk);
                const uint32_t h0 = h32[0], q0 = h32[1], q1 = h32[2], q2 = h32[3];
                const float d = half_bits_to_float(h0 & 0xffffu);
                const float dmin = half_bits_to_float(h0 >> 16);
                // 6-bit scales and mins of the eight sub-blocks (quant.go:96-103).
                int sc[8], mn[8];
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    sc[s] = (q0 >> (8 * s)) & 63;
                    mn[s] = (q1 >> (8 * s)) & 63;
                    sc[s + 4] = ((q2 >> (8 * s)) & 0x0f) | (((q0 >> (8 * s + 6)) & 3) << 4);
                    mn[s + 4] = ((q2 >> (8 * s + 4)) & 0x0f) | (((q1 >> (8 * s + 6)) & 3) << 4);
                }
                int acci[NA][4], accm[NA][4];
#pragma unroll
                for (int a = 0; a < NA; a++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acci[a][i] = accm[a][i] = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint64_t qs = *reinterpret_cast<const uint64_t *>(blk + 16 + 32 * j + 8 * g);
                    const int64_t blo = (int64_t)(qs & 0x0f0f0f0f0f0f0f0full);
                    const int64_t bhi = (int64_t)((qs >> 4) & 0x0f0f0f0f0f0f0f0full);
#pragma unroll
                    for (int a = 0; a < NA; a++) {
                        const i32x4 c0 = mfma_i8(xa[a][2 * j], blo);
                        const i32x4 c1 = mfma_i8(xa[a][2 * j + 1], bhi);
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            acci[a][i] = mad24(sc[2 * j], c0[i], acci[a][i]);
                            acci[a][i] = mad24(sc[2 * j + 1], c1[i], acci[a][i]);
                            accm[a][i] = mad24(mn[2 * j], sx[a][2 * j][i], accm[a][i]);
                            accm[a][i] = mad24(mn[2 * j + 1], sx[a][2 * j + 1][i], accm[a][i]);
                        }
                    }
                }
#pragma unroll
                for (int a = 0; a < NA; a++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        acc[t][a][i] += d * (float)acci[a][i] - dmin * (float)accm[a][i];
            } else {
                // Q6_K: ql[128] qh[64] sc[16] d (quant.go:261-285).
                const uint16_t dh = *reinterpret_cast<const uint16_t *>(blk + 208);
                const float d = half_bits_to_float(dh);
                int acci[NA][4];
#pragma unroll
                for (int a = 0; a < NA; a++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acci[a][i] = 0;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint64_t ql0 = lds_read8_a2(lds, blk_off + 64 * h + 8 * g);
                    const uint64_t ql1 = lds_read8_a2(lds, blk_off + 64 * h + 32 + 8 * g);
                    const uint64_t qh = lds_read8_a2(lds, blk_off + 128 + 32 * h + 8 * g);
                    const uint64_t sc8 = lds_read8_a2(lds, blk_off + 192 + 8 * h);
#pragma unroll
                    for (int qt = 0; qt < 4; qt++) {
                        const uint64_t ql = (qt & 1) ? ql1 : ql0;
                        const uint64_t nib = (qt >> 1) ? ((ql >> 4) & 0x0f0f0f0f0f0f0f0full)
                                                       : (ql & 0x0f0f0f0f0f0f0f0full);
                        const uint64_t hb = (qh >> (2 * qt)) & 0x0303030303030303ull;
                        const uint64_t v = q6_to_i8(nib | (hb << 4));
                        const int64_t ba = (int64_t)(g < 2 ? v : 0ull);
                        const int64_t bb = (int64_t)(g < 2 ? 0ull : v);
                        const int sa = (int)(int8_t)((sc8 >> (8 * (2 * qt))) & 0xff);
                        const int sbv = (int)(int8_t)((sc8 >> (8 * (2 * qt + 1))) & 0xff);
                        const int s = 4 * h + qt;
#pragma unroll
                        for (int a = 0; a < NA; a++) {
                            const i32x4 c0 = mfma_i8(xa[a][s], ba);
                            const i32x4 c1 = mfma_i8(xa[a][s], bb);
#pragma unroll
                            for (int i = 0; i < 4; i++) {
                                acci[a][i] = mad24(sa, c0[i], acci[a][i]);
                                acci[a][i] = mad24(sbv, c1[i], acci[a][i]);
                            }
                        }
                    }
                }
#pragma unroll
                for (int a = 0; a < NA; a++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[t][a][i] += d * (float)acci[a][i];
            }
        }
    }

    // Cross-wave reduction through LDS: red[w][rho][n_local].
    __syncthreads();
    float *red = reinterpret_cast<float *>(lds);
    constexpr int RHO = 16 * NA;
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int a = 0; a < NA; a++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                red[(wave * RHO + 16 * a + 4 * g + i) * 64 + 16 * t + r] = acc[t][a][i];
    __syncthreads();

    for (int idx = tid; idx < M * 64; idx += 256) {
        const int m = idx >> 6, nl = idx & 63;
        const int n = n_base + nl;
        float v = 0.0f;
#pragma unroll
        for (int wv = 0; wv < 4; wv++)
            v += 256.0f * red[(wv * RHO + m) * 64 + nl] + red[(wv * RHO + M + m) * 64 + nl];
        v *= xs[m];
        if (n < N) {
            if (splits == 1)
                out[(size_t)m * N + n] = residual ? v + residual[(size_t)m * N + n] : v;
            else
                partials[((size_t)split * M + m) * N + n] = v;
        }
    }
}

// --------------------------------------------------------------------------
// Q4_K verify GEMM. A workgroup of four waves owns 256 output rows (64 per
// wave, four 16-row MFMA tiles each) and a contiguous range of super-blocks;
// larger K is split across workgroups (partials summed by a second kernel).
// Per super-block the four waves share one staged copy of the activation
// planes; each wave stages its own rows:
//   hdr  [64 rows][32 B]   d f32, dmin f32, 8 scale bytes, 8 mins as int16
//                          (decoded once per row by the lane that loads it)
//   qs   [4 t][4 j][4 g][16 r][8 B], groups padded to 136 B (the MFMA read
//                          order; padding spreads the staging writes)
//   xa   [NA][32 slices][16 rho][8]  int8 activation planes (shared)
//   sx   [NA][16 rho][8]             int16 sub-block sums (shared)
// The min term uses v_dot2_i32_i16 over (min, sum) pairs; the scale term
// multiplies the int32 MFMA results by the 6-bit scales in int32.
// --------------------------------------------------------------------------
typedef short __attribute__((ext_vector_type(2))) s16x2;

template <int NA>
struct L4 {
    static constexpr int GS = 136;
    static constexpr int HDR = 0, QS = 2048, WAVE = QS + 64 * GS;
    static constexpr int XA = 4 * WAVE, SX = XA + NA * 4096, TOTAL = SX + NA * 256;
};

__device__ __forceinline__ int mad24i(int a, int b, int c) { return __mul24(a, b) + c; }

__device__ __forceinline__ int dot2(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s16x2, a), __builtin_bit_cast(s16x2, b), c, false);
}

template <int NA>
__global__ __launch_bounds__(256) void gemm_q4k_kernel(const uint8_t *__restrict__ w, uint32_t w_bytes,
                                                       uint32_t row_bytes, const uint8_t *__restrict__ xq,
                                                       float *out, int N, int K, int M,
                                                       int splits, int spw, float *__restrict__ partials,
                                                       const float *residual) {
    using L = L4<NA>;
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 15, g = lane >> 4;
    const int rg = blockIdx.x / splits, split = blockIdx.x % splits;
    const int n_base = rg * 256 + wave * 64;
    const int nsb = K / 256;
    const int sb_begin = split * spw;
    const int sb_end = min(sb_begin + spw, nsb);
    uint8_t *ws = lds + wave * L::WAVE;
    const float *xs = reinterpret_cast<const float *>(xq);
    const uint8_t *planes = xq + 64;
    const uint8_t *sums = xq + 64 + (size_t)NA * K * 16;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)w, (short)0, (int)((w_bytes + 15u) & ~15u), 0x00020000);

    float acc[4][NA][4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int a = 0; a < NA; a++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[t][a][i] = 0.0f;

    // Staging registers: super-block sb+1 is in flight while sb is computed.
    // (A second register stage was measured slower: the extra VGPRs cost a
    // wave per SIMD.)
    struct Stage {
        i32x4 hdr, qs[8], xa[NA], sx;
    };
    Stage st0;
    const int my_row = min(n_base + lane, N - 1);

    auto issue = [&](Stage &S, int sb) {
        const uint32_t base = (uint32_t)sb * 144u;
        S.hdr = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (uint32_t)my_row * row_bytes + base, 0, 0);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = lane + 64 * i;  // row c/8, 16-byte chunk c%8 of the quants
            const int n = min(n_base + (c >> 3), N - 1);
            S.qs[i] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, (uint32_t)n * row_bytes + base + 16 + (c & 7) * 16, 0, 0);
        }
#pragma unroll
        for (int a = 0; a < NA; a++)
            S.xa[a] = *reinterpret_cast<const i32x4 *>(planes + ((size_t)a * (K / 8) + (size_t)sb * 32) * 128 + tid * 16);
        if (tid < 16 * NA)
            S.sx = *reinterpret_cast<const i32x4 *>(sums + ((size_t)(tid >> 4) * nsb + sb) * 256 + (tid & 15) * 16);
    };
    auto commit = [&](const Stage &S) {
        {   // header of row `lane` (quant.go:96-103 packing, decoded once)
            const uint32_t h0 = (uint32_t)S.hdr[0], q0 = (uint32_t)S.hdr[1], q1 = (uint32_t)S.hdr[2],
                           q2 = (uint32_t)S.hdr[3];
            const float d = half_bits_to_float(h0 & 0xffffu);
            const float dmin = half_bits_to_float(h0 >> 16);
            const uint32_t sc_lo = q0 & 0x3f3f3f3fu;
            const uint32_t sc_hi = (q2 & 0x0f0f0f0fu) | ((q0 >> 2) & 0x30303030u);
            const uint32_t mn_lo = q1 & 0x3f3f3f3fu;
            const uint32_t mn_hi = ((q2 >> 4) & 0x0f0f0f0fu) | ((q1 >> 2) & 0x30303030u);
            const i32x4 r0 = {(int)__float_as_uint(d), (int)__float_as_uint(dmin), (int)sc_lo, (int)sc_hi};
            const i32x4 r1 = {(int)__builtin_amdgcn_perm(0u, mn_lo, 0x0c010c00u), (int)__builtin_amdgcn_perm(0u, mn_lo, 0x0c030c02u),
                              (int)__builtin_amdgcn_perm(0u, mn_hi, 0x0c010c00u), (int)__builtin_amdgcn_perm(0u, mn_hi, 0x0c030c02u)};
            *reinterpret_cast<i32x4 *>(ws + L::HDR + lane * 32) = r0;
            *reinterpret_cast<i32x4 *>(ws + L::HDR + lane * 32 + 16) = r1;
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = lane + 64 * i;
            const int row = c >> 3, ch = c & 7;
            const int t = row >> 4, rr = row & 15, j = ch >> 1, g0 = (ch & 1) * 2;
            uint8_t *dst = ws + L::QS + ((t * 4 + j) * 4 + g0) * L::GS + rr * 8;
            *reinterpret_cast<uint64_t *>(dst) = (uint64_t)(uint32_t)S.qs[i][0] | ((uint64_t)(uint32_t)S.qs[i][1] << 32);
            *reinterpret_cast<uint64_t *>(dst + L::GS) = (uint64_t)(uint32_t)S.qs[i][2] | ((uint64_t)(uint32_t)S.qs[i][3] << 32);
        }
#pragma unroll
        for (int a = 0; a < NA; a++) *reinterpret_cast<i32x4 *>(lds + L::XA + a * 4096 + tid * 16) = S.xa[a];
        if (tid < 16 * NA) *reinterpret_cast<i32x4 *>(lds + L::SX + tid * 16) = S.sx;
    };
    auto compute = [&]() {
        int64_t xa[NA][8];
        uint32_t sxp[NA][4][4];  // [a][i: rho = 4g+i][pair p: sub-blocks 2p, 2p+1]
#pragma unroll
        for (int a = 0; a < NA; a++) {
#pragma unroll
            for (int s = 0; s < 8; s++)
                xa[a][s] = *reinterpret_cast<const int64_t *>(lds + L::XA + a * 4096 + (s * 4 + g) * 128 + r * 8);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const i32x4 v = *reinterpret_cast<const i32x4 *>(lds + L::SX + a * 256 + (4 * g + i) * 16);
#pragma unroll
                for (int p = 0; p < 4; p++) sxp[a][i][p] = (uint32_t)v[p];
            }
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int row = 16 * t + r;
            const i32x4 h0 = *reinterpret_cast<const i32x4 *>(ws + L::HDR + row * 32);
            const i32x4 h1 = *reinterpret_cast<const i32x4 *>(ws + L::HDR + row * 32 + 16);
            const float d = __uint_as_float((uint32_t)h0[0]);
            const float dmin = __uint_as_float((uint32_t)h0[1]);
            int acci[NA][4], accm[NA][4];
#pragma unroll
            for (int a = 0; a < NA; a++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    int m = 0;
#pragma unroll
                    for (int p = 0; p < 4; p++) m = dot2((uint32_t)h1[p], sxp[a][i][p], m);
                    accm[a][i] = m;
                    acci[a][i] = 0;
                }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint64_t qs = *reinterpret_cast<const uint64_t *>(ws + L::QS + ((t * 4 + j) * 4 + g) * L::GS + r * 8);
                const int64_t blo = (int64_t)(qs & 0x0f0f0f0f0f0f0f0full);
                const int64_t bhi = (int64_t)((qs >> 4) & 0x0f0f0f0f0f0f0f0full);
                const uint32_t scw = (uint32_t)h0[2 + (j >> 1)];
                const int s0 = (int)__builtin_amdgcn_ubfe(scw, 16 * (j & 1), 8);
                const int s1 = (int)__builtin_amdgcn_ubfe(scw, 16 * (j & 1) + 8, 8);
#pragma unroll
                for (int a = 0; a < NA; a++) {
                    const i32x4 c0 = mfma_i8(xa[a][2 * j], blo);
                    const i32x4 c1 = mfma_i8(xa[a][2 * j + 1], bhi);
#pragma unroll
                    for (int i = 0; i < 4; i++) acci[a][i] = mad24i(s1, c1[i], mad24i(s0, c0[i], acci[a][i]));
                }
            }
#pragma unroll
            for (int a = 0; a < NA; a++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[t][a][i] += d * (float)acci[a][i] - dmin * (float)accm[a][i];
        }
    };

    if (sb_begin < sb_end) issue(st0, sb_begin);
    for (int sb = sb_begin; sb < sb_end; sb++) {
        __syncthreads();  // previous super-block's LDS reads are done
        commit(st0);
        __syncthreads();  // staged bytes visible to the workgroup
        if (sb + 1 < sb_end) issue(st0, sb + 1);
        compute();
    }

    // Epilogue per wave: combine the hi/lo planes through the wave's LDS area.
    __syncthreads();
    float *red = reinterpret_cast<float *>(ws);
    constexpr int RHO = 16 * NA;
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
        for (int a = 0; a < NA; a++)
#pragma unroll
            for (int i = 0; i < 4; i++) red[(16 * a + 4 * g + i) * 64 + 16 * t + r] = acc[t][a][i];
    __syncthreads();
    const int n = n_base + lane;
    if (n < N) {
        for (int m = 0; m < M; m++) {
            const float v = (256.0f * red[m * 64 + lane] + red[(M + m) * 64 + lane]) * xs[m];
            if (splits == 1) out[(size_t)m * N + n] = residual ? v + residual[(size_t)m * N + n] : v;
            else partials[((size_t)split * M + m) * N + n] = v;
        }
    }
    (void)RHO;
}

// Sums the split-K partials in a fixed order (deterministic).
__global__ __launch_bounds__(256) void reduce_splits_kernel(const float *__restrict__ partials,
                                                            float *out, int splits,
                                                            uint64_t count, const float *residual) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= count) return;
    float v = 0.0f;
    for (int s = 0; s < splits; s++) v += partials[(uint64_t)s * count + i];
    out[i] = residual ? v + residual[i] : v;
}

// --------------------------------------------------------------------------
// Bit-exact dequantization (tensor/quant.go:15-62). One thread per 256-block
// (K-quants) or per element (F32/F16/Q8_0). The FP32 expressions are written
// as separate multiply and subtract (no contraction) in the reference order.
// --------------------------------------------------------------------------
#pragma clang fp contract(off)

__device__ __forceinline__ uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

__device__ __forceinline__ float exact_mul(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float exact_sub(float a, float b) { return __fsub_rn(a, b); }

template <typename OutT>
__device__ __forceinline__ void put(OutT *dst, size_t i, float v);
template <> __device__ __forceinline__ void put<float>(float *dst, size_t i, float v) { dst[i] = v; }
template <> __device__ __forceinline__ void put<uint16_t>(uint16_t *dst, size_t i, float v) {
    dst[i] = __half_as_ushort(__float2half_rn(v));
}

template <typename OutT>
__global__ __launch_bounds__(256) void dequant_kquant_kernel(const uint8_t *__restrict__ src,
                                                             uint32_t dtype, uint64_t row_bytes,
                                                             uint64_t n_in, uint64_t n_out,
                                                             OutT *__restrict__ dst) {
    const uint64_t nblk = n_in / 256;
    const uint64_t id = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= nblk * n_out) return;
    const uint64_t row = id / nblk, b = id % nblk;
    const uint64_t out0 = row * n_in + b * 256;
    if (dtype == kQ4K || dtype == YUUKA_DTYPE_Q5_K) {
        const bool q5 = dtype == YUUKA_DTYPE_Q5_K;
        const uint8_t *p = src + row * row_bytes + b * (q5 ? 176 : 144);
        const float d = half_bits_to_float(rd16(p));
        const float dm = half_bits_to_float(rd16(p + 2));
        const uint8_t *q = p + 4;
        const uint8_t *qh = p + 16;
        const uint8_t *qs = p + (q5 ? 48 : 16);
        for (int j = 0, is = 0; j < 256; j += 64, is += 2) {
            uint32_t s0, m0, s1, m1;
            if (is < 4) { s0 = q[is] & 63; m0 = q[is + 4] & 63; }
            else { s0 = (q[is + 4] & 0x0f) | ((q[is - 4] >> 6) << 4); m0 = (q[is + 4] >> 4) | ((q[is] >> 6) << 4); }
            const int i1 = is + 1;
            if (i1 < 4) { s1 = q[i1] & 63; m1 = q[i1 + 4] & 63; }
            else { s1 = (q[i1 + 4] & 0x0f) | ((q[i1 - 4] >> 6) << 4); m1 = (q[i1 + 4] >> 4) | ((q[i1] >> 6) << 4); }
            const float d1 = exact_mul(d, (float)s0), min1 = exact_mul(dm, (float)m0);
            const float d2 = exact_mul(d, (float)s1), min2 = exact_mul(dm, (float)m1);
            const uint32_t bit0 = 1u << (2 * (j / 64)), bit1 = bit0 << 1;
            for (int l = 0; l < 32; l++) {
                uint32_t v0 = qs[l] & 0x0f, v1 = qs[l] >> 4;
                if (q5) {
                    if (qh[l] & bit0) v0 += 16;
                    if (qh[l] & bit1) v1 += 16;
                }
                put(dst, out0 + j + l, exact_sub(exact_mul(d1, (float)v0), min1));
                put(dst, out0 + j + 32 + l, exact_sub(exact_mul(d2, (float)v1), min2));
            }
            qs += 32;
        }
    } else {  // Q6_K
        const uint8_t *p = src + row * row_bytes + b * 210;
        const uint8_t *ql = p, *qh = p + 128, *sc = p + 192;
        const float d = half_bits_to_float(rd16(p + 208));
        for (int h = 0; h < 2; h++) {
            for (int l = 0; l < 32; l++) {
                const int is = l / 16;
                const int q1 = (int)((ql[64 * h + l] & 0x0f) | (((qh[32 * h + l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((ql[64 * h + l + 32] & 0x0f) | (((qh[32 * h + l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql[64 * h + l] >> 4) | (((qh[32 * h + l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql[64 * h + l + 32] >> 4) | (((qh[32 * h + l] >> 6) & 3) << 4)) - 32;
                const uint64_t base = out0 + 128 * h;
                put(dst, base + l, exact_mul(exact_mul(d, (float)(int8_t)sc[8 * h + is + 0]), (float)q1));
                put(dst, base + l + 32, exact_mul(exact_mul(d, (float)(int8_t)sc[8 * h + is + 2]), (float)q2));
                put(dst, base + l + 64, exact_mul(exact_mul(d, (float)(int8_t)sc[8 * h + is + 4]), (float)q3));
                put(dst, base + l + 96, exact_mul(exact_mul(d, (float)(int8_t)sc[8 * h + is + 6]), (float)q4));
            }
        }
    }
}

template <typename OutT>
__global__ __launch_bounds__(256) void dequant_flat_kernel(const uint8_t *__restrict__ src,
                                                           uint32_t dtype, uint64_t row_bytes,
                                                           uint64_t n_in, uint64_t n_out,
                                                           OutT *__restrict__ dst) {
    const uint64_t id = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (id >= n_in * n_out) return;
    const uint64_t row = id / n_in, col = id % n_in;
    const uint8_t *p = src + row * row_bytes;
    float v;
    if (dtype == YUUKA_DTYPE_F32) {
        v = reinterpret_cast<const float *>(p)[col];
    } else if (dtype == YUUKA_DTYPE_F16) {
        v = half_bits_to_float(rd16(p + col * 2));
    } else {  // Q8_0 (quant.go:86-93)
        const uint8_t *blk = p + (col / 32) * 34;
        v = exact_mul(half_bits_to_float(rd16(blk)), (float)(int8_t)blk[2 + col % 32]);
    }
    put(dst, id, v);
}

__global__ void cast_f16_kernel(const float *__restrict__ src, uint16_t *__restrict__ dst, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = __half_as_ushort(__float2half_rn(src[i]));
}

template <typename OutT>
hipError_t dequant_launch(const void *src, uint32_t dtype, OutT *dst, uint64_t n_in, uint64_t n_out,
                          hipStream_t stream) {
    const uint64_t rb = row_bytes(dtype, n_in);
    if (dtype == kQ4K || dtype == kQ6K || dtype == YUUKA_DTYPE_Q5_K) {
        const uint64_t total = n_in / 256 * n_out;
        dequant_kquant_kernel<OutT><<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(
            static_cast<const uint8_t *>(src), dtype, rb, n_in, n_out, dst);
    } else {
        const uint64_t total = n_in * n_out;
        dequant_flat_kernel<OutT><<<(unsigned)((total + 255) / 256), 256, 0, stream>>>(
            static_cast<const uint8_t *>(src), dtype, rb, n_in, n_out, dst);
    }
    return hipGetLastError();
}

}  // namespace

uint64_t row_bytes(uint32_t dtype, uint64_t cols) {
    uint64_t e, b;
    switch (dtype) {
    case YUUKA_DTYPE_F32: e = 1; b = 4; break;
    case YUUKA_DTYPE_F16: e = 1; b = 2; break;
    case YUUKA_DTYPE_Q8_0: e = 32; b = 34; break;
    case YUUKA_DTYPE_Q4_K: e = 256; b = 144; break;
    case YUUKA_DTYPE_Q5_K: e = 256; b = 176; break;
    case YUUKA_DTYPE_Q6_K: e = 256; b = 210; break;
    default: return 0;
    }
    if (cols == 0 || cols % e != 0) return 0;
    return cols / e * b;
}

GemmPlan gemm_plan(uint64_t n_in, uint64_t n_out, uint64_t rows, uint32_t dtype) {
    GemmPlan p;
    const int na = rows <= 8 ? 1 : 2;
    const int nsb = (int)(n_in / 256);
    int splits, spw;
    if (dtype == YUUKA_DTYPE_Q6_K) {
        // 64-row workgroups whose four waves split K.
        const int rowblocks = (int)((n_out + 63) / 64);
        const int waves_per_rb = std::max(4, (2048 + rowblocks - 1) / rowblocks);
        spw = std::max(1, (nsb + waves_per_rb - 1) / waves_per_rb);
        splits = (nsb + spw * 4 - 1) / (spw * 4);
    } else {
        // 256-row workgroups; K split across workgroups until ~2048 waves.
        const int groups = (int)((n_out + 255) / 256);
        splits = std::min(nsb, std::max(1, (512 + groups - 1) / groups));
        spw = (nsb + splits - 1) / splits;
        splits = (nsb + spw - 1) / spw;
    }
    p.splits = std::max(1, splits);
    p.sb_per_wave = std::max(1, spw);
    p.xq_bytes = 64 + (uint64_t)na * n_in * 17;
    p.part_bytes = p.splits > 1 ? (uint64_t)p.splits * rows * n_out * 4 : 0;
    p.tickets = 0;
    return p;
}

hipError_t launch_quantize_x(const float *x, uint64_t n_in, uint64_t rows, void *xq,
                             hipStream_t stream) {
    const int na = rows <= 8 ? 1 : 2;
    const dim3 grid((unsigned)rows, (unsigned)((n_in / 8 + 255) / 256));
    quantize_x_kernel<<<grid, 256, 0, stream>>>(x, (int)n_in, (int)rows, na, static_cast<uint8_t *>(xq));
    return hipGetLastError();
}

template <int DT, int NA>
static void launch_one(dim3 grid, hipStream_t stream, const uint8_t *wp, uint64_t wbytes, uint64_t rb,
                       const uint8_t *xp, float *dst, int N, int K, int M, const GemmPlan &plan, float *pp,
                       const float *res) {
    const size_t lds = 4 * Layout<DT, NA>::WAVE_BYTES + 16;
    gemm_kq_kernel<DT, NA><<<grid, 256, lds, stream>>>(wp, (uint32_t)wbytes, (uint32_t)rb, xp, dst, N, K, M,
                                                       plan.splits, plan.sb_per_wave, pp, res);
}

hipError_t launch_gemm_q(const void *w, uint32_t dtype, const void *xq, float *out, uint64_t n_in,
                         uint64_t n_out, uint64_t rows, const GemmPlan &plan, void *partials,
                         uint32_t *tickets, hipStream_t stream, const float *residual) {
    (void)tickets;
    const uint64_t rb = row_bytes(dtype, n_in);
    const uint64_t wbytes = rb * n_out;
    const int rowblocks = (int)((n_out + 63) / 64);
    const dim3 grid((unsigned)(rowblocks * plan.splits));
    const auto *wp = static_cast<const uint8_t *>(w);
    const auto *xp = static_cast<const uint8_t *>(xq);
    auto *pp = static_cast<float *>(partials);
    const int N = (int)n_out, K = (int)n_in, M = (int)rows;
    if (dtype == YUUKA_DTYPE_Q4_K) {
        const dim3 grid((unsigned)(((n_out + 255) / 256) * plan.splits));
        if (rows <= 8)
            gemm_q4k_kernel<1><<<grid, 256, L4<1>::TOTAL, stream>>>(wp, (uint32_t)wbytes, (uint32_t)rb, xp, out, N, K, M, plan.splits, plan.sb_per_wave, pp, residual);
        else
            gemm_q4k_kernel<2><<<grid, 256, L4<2>::TOTAL, stream>>>(wp, (uint32_t)wbytes, (uint32_t)rb, xp, out, N, K, M, plan.splits, plan.sb_per_wave, pp, residual);
    } else {
        if (rows <= 8) launch_one<kQ6K, 1>(grid, stream, wp, wbytes, rb, xp, out, N, K, M, plan, pp, residual);
        else launch_one<kQ6K, 2>(grid, stream, wp, wbytes, rb, xp, out, N, K, M, plan, pp, residual);
    }
    if (plan.splits > 1) {
        const uint64_t count = rows * n_out;
        reduce_splits_kernel<<<(unsigned)((count + 255) / 256), 256, 0, stream>>>(pp, out, plan.splits, count, residual);
    }
    return hipGetLastError();
}

hipError_t launch_dequant_f32(const void *src, uint32_t dtype, float *dst, uint64_t n_in,
                              uint64_t n_out, hipStream_t stream) {
    return dequant_launch<float>(src, dtype, dst, n_in, n_out, stream);
}

hipError_t launch_dequant_f16(const void *src, uint32_t dtype, uint16_t *dst, uint64_t n_in,
                              uint64_t n_out, hipStream_t stream) {
    return dequant_launch<uint16_t>(src, dtype, dst, n_in, n_out, stream);
}

hipError_t launch_cast_f16(const float *src, uint16_t *dst, uint64_t n, hipStream_t stream) {
    cast_f16_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(src, dst, n);
    return hipGetLastError();
}

}  // namespace yk
