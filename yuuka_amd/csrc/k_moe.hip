// k_moe.hip — mixture-of-experts FFN of the qwen35moe verify step
// (model/qwen35/forward.go:320-439 forwardMoEFFN / selectExperts) and the
// reference's MoE plan ops (backend/hip/bridge/yuuka_hip.h:457-470).
//
//  * router:   FP32 router logits (and the shared-expert gate logit) of the
//              verify rows, one workgroup per (4 expert rows, 8 rows), K
//              split over its waves.
//  * route:    top-`used` experts per row by repeated argmax (lower index
//              wins ties) and softmax over the selected logits, one wave per
//              row; then binning of the (row, slot) assignments by expert,
//              one workgroup per expert, in (row, slot) order, so the bins
//              are deterministic and every count is written (no memset,
//              graph-safe). Up to 16 rows, routing and binning run in one
//              workgroup (row masks per expert give the bin places).
//  * grouped GEMM: one launch over every expert's assigned rows. Workgroups
//              are (expert, part); a workgroup with no assignments exits.
//              The activation rows are quantized once per launch (int16
//              split into two int8 planes, one scale per row and
//              256-element super-block), staged in LDS per chunk of eight
//              assignments, and multiplied with v_mfma_i32_16x16x64_i8
//              against Q4_K weights decoded from HBM straight into MFMA
//              operand order, the sub-block scale and min in the B operands.
//              Eight assignments fill the high-plane half of one MFMA tile
//              and their low planes the other half.
//  * reduce / combine: weighted sum of the slots (and the sigmoid-gated
//              shared expert) into the residual stream, in the reference's
//              order of float32 operations.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <map>
#include <mutex>
#include <tuple>

#include "model_kernels.h"
#include "refmath.h"

namespace yk {
namespace {

typedef __attribute__((ext_vector_type(4))) int i32x4;

constexpr int kQMax = 32639;     // |q| bound that keeps the high plane in int8
constexpr int kMoeWaves = 8;
constexpr int kMoeThreads = 64 * kMoeWaves;
constexpr int kChunk = 8;        // assignments per MFMA tile (high planes in rows 0..7)
constexpr int kMoeMaxExperts = 1024;
constexpr int kMoeMaxRows = 512;     // rows of a grouped GEMM (an expert's chunks stay below 64)
constexpr int kMoeMaxList = 2048;    // work-list entries: experts + chunks past their first

// Wave reductions on the DPP path (a __shfl_xor is an LDS permute): within
// each 16-lane row (pairs, quads, half rows, rows), then the four rows'
// results through readlane (every lane gets the result).
template <int C>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), C, 0xf, 0xf, true));
}
__device__ __forceinline__ float rl_f(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xb1>(v);
    v += dpp_f<0x4e>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    return (rl_f(v, 0) + rl_f(v, 16)) + (rl_f(v, 32) + rl_f(v, 48));
}
__device__ __forceinline__ float wave_max_nonneg(float v) {  // values >= 0
    v = fmaxf(v, dpp_f<0xb1>(v));
    v = fmaxf(v, dpp_f<0x4e>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return fmaxf(fmaxf(rl_f(v, 0), rl_f(v, 16)), fmaxf(rl_f(v, 32), rl_f(v, 48)));
}

// ---------------------------------------------------------------- router
// logits[r][e] = W[e] . y[r] (FP32 weights, ffn_gate_inp) and, when `sv` is
// given, extra[r] = sv . y[r] (ffn_gate_inp_shexp, forward.go:385). One
// workgroup per (block of kRouterExperts expert rows, block of kRouterRows
// rows) (the shared gate vector is row E). Its four waves split K: lane l of
// wave w takes the float4 groups l + 64 (w + 4 j), so every wave issues its
// few loads at once; each lane's partial sums of the block's 32 dot products
// go to LDS, and 8 threads per product add them in a fixed order.
constexpr int kRouterWaves = 4;
constexpr int kRouterExperts = 4;
constexpr int kRouterRows = 8;
constexpr int kRouterDots = kRouterExperts * kRouterRows;
constexpr int kRouterPad = 264;  // LDS row stride (floats) of one dot product's 256 partials

__global__ __launch_bounds__(64 * kRouterWaves) void moe_router_kernel(const float *__restrict__ y, int H, int rows,
                                                                       const float *__restrict__ w, int E,
                                                                       float *__restrict__ logits,
                                                                       const float *__restrict__ sv,
                                                                       float *__restrict__ extra) {
    __shared__ float part[kRouterDots * kRouterPad];
    const int t = threadIdx.x;
    const int e0 = blockIdx.x * kRouterExperts, ne = E + (sv ? 1 : 0);
    const int r0 = blockIdx.y * kRouterRows;
    const float *wr[kRouterExperts];
    const float *yr[kRouterRows];
#pragma unroll
    for (int x = 0; x < kRouterExperts; x++) {
        const int e = min(e0 + x, ne - 1);
        wr[x] = e < E ? w + (uint64_t)e * H : sv;
    }
#pragma unroll
    for (int i = 0; i < kRouterRows; i++) yr[i] = y + (uint64_t)min(r0 + i, rows - 1) * H;
    float acc[kRouterExperts][kRouterRows];
#pragma unroll
    for (int x = 0; x < kRouterExperts; x++)
#pragma unroll
        for (int i = 0; i < kRouterRows; i++) acc[x][i] = 0.f;
#pragma unroll 2
    for (int k = 4 * t; k < H; k += 4 * 64 * kRouterWaves) {
        float4 wv[kRouterExperts], yv[kRouterRows];
#pragma unroll
        for (int x = 0; x < kRouterExperts; x++) wv[x] = *reinterpret_cast<const float4 *>(wr[x] + k);
#pragma unroll
        for (int i = 0; i < kRouterRows; i++) yv[i] = *reinterpret_cast<const float4 *>(yr[i] + k);
#pragma unroll
        for (int x = 0; x < kRouterExperts; x++)
#pragma unroll
            for (int i = 0; i < kRouterRows; i++)
                acc[x][i] += wv[x].x * yv[i].x + wv[x].y * yv[i].y + wv[x].z * yv[i].z + wv[x].w * yv[i].w;
    }
#pragma unroll
    for (int x = 0; x < kRouterExperts; x++)
#pragma unroll
        for (int i = 0; i < kRouterRows; i++) part[(x * kRouterRows + i) * kRouterPad + t] = acc[x][i];
    __syncthreads();
    // dot product d = t / 8; thread part p = t % 8 adds partials p, p + 8, ...
    const int d = t >> 3, p = t & 7;
    float s = 0.f;
#pragma unroll 8
    for (int j = 0; j < 64 * kRouterWaves / 8; j++) s += part[d * kRouterPad + p + 8 * j];
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    const int x = d / kRouterRows, r = r0 + d % kRouterRows, e = e0 + x;
    if (p == 0 && r < rows && e < ne) {
        if (e < E)
            logits[(uint64_t)r * E + e] = s;
        else
            extra[r] = s;
    }
}

// ---------------------------------------------------------------- route
// forward.go:393-439 selectExperts for every row (one wave per row, the
// row's logits held in registers, a taken mask per lane), then binning by
// expert (in a second launch above 16 rows) (the reference's assignment layout,
// yuuka_hip.h:457-460: bucket capacity rows*used). An assignment's place in
// its bin is the number of earlier (row, slot) assignments to the same
// expert, so the bins are in (row, slot) order.
constexpr int kRouteMaxPerLane = 16;  // experts <= 1024

// Monotone uint32 image of a float (larger value, larger key); -0 keys as +0
// because the reference compares values.
__device__ __forceinline__ uint32_t route_key(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u << 1) == 0u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

// Maximum over the wave: DPP inside each 16-lane row, then the four rows'
// results through readlane (wave-uniform).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0xb1>(v));
    v = max(v, dpp_u32<0x4e>(v));
    v = max(v, dpp_u32<0x124>(v));
    v = max(v, dpp_u32<0x128>(v));
    uint32_t best = 0;
#pragma unroll
    for (int r = 0; r < 4; r++) best = max(best, (uint32_t)__builtin_amdgcn_readlane((int)v, 16 * r));
    return best;
}

// selectExperts for one row by one wave. Expert e = lane + 64 i sits in
// lane `lane`, register i, so scanning i then lane visits experts in index
// order. The reference's scan (forward.go:403-418) starts each slot at the
// first untaken expert and replaces it only with a strictly greater logit:
// a NaN start keeps the slot, NaN elsewhere never wins, and equal maxima go
// to the lowest index. Per slot: the wave maximum of the order keys of the
// untaken non-NaN logits, then the lowest expert holding it from ballots;
// the untaken and NaN sets are wave-wide ballot masks.
template <int PL>
__device__ __forceinline__ void load_route_row(const float *__restrict__ l, int E, float (&v)[PL]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < PL; i++) v[i] = lane + 64 * i < E ? l[lane + 64 * i] : 0.f;
}

template <int PL>
__device__ __forceinline__ void route_row(const float (&v)[PL], int E, int used, int &my_id, float &my_w) {
    const int lane = threadIdx.x & 63;
    uint32_t key[PL];  // 0: taken, NaN or past E
    uint64_t live[PL], nan[PL];
#pragma unroll
    for (int i = 0; i < PL; i++) {
        const bool in = lane + 64 * i < E;
        key[i] = in && v[i] == v[i] ? route_key(v[i]) : 0u;
        live[i] = __ballot(in);
        nan[i] = __ballot(in && !(v[i] == v[i]));
    }
    my_id = 0;
    float my_pv = 0.f;
    for (int slot = 0; slot < used; slot++) {
        uint32_t m = key[0];
#pragma unroll
        for (int i = 1; i < PL; i++) m = max(m, key[i]);
        const uint32_t K = wave_max_u32(m);
        int first = -1;
        bool first_nan = false;
#pragma unroll
        for (int i = PL - 1; i >= 0; i--)
            if (live[i]) {
                const int bit = __builtin_ctzll(live[i]);
                first = 64 * i + bit;
                first_nan = (nan[i] >> bit) & 1ull;
            }
        int pick = 0;  // more slots than experts (forward.go:413-417)
        if (first >= 0) {
            if (K == 0u || first_nan) {
                pick = first;
            } else {
#pragma unroll
                for (int i = PL - 1; i >= 0; i--) {
                    const uint64_t hit = __ballot(key[i] == K);
                    if (hit) pick = 64 * i + __builtin_ctzll(hit);
                }
            }
#pragma unroll
            for (int i = 0; i < PL; i++)
                if (i == (pick >> 6)) {
                    live[i] &= ~(1ull << (pick & 63));
                    if (lane == (pick & 63)) key[i] = 0u;
                }
        }
        float pv = 0.f;
#pragma unroll
        for (int i = 0; i < PL; i++)
            if (i == (pick >> 6)) pv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[i]), pick & 63));
        if (lane == slot) {
            my_id = pick;
            my_pv = pv;
        }
    }
    // weights: float32(exp(float64(l - max))), float32 total in slot order,
    // then each divided by the total (forward.go:424-438); lane s computes
    // slot s's exponential, every lane the ordered total.
    float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_pv), 0));
    for (int sl = 1; sl < used; sl++) {
        const float o = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_pv), sl));
        if (o > mx) mx = o;
    }
    const float wt = lane < used ? (float)exp((double)__fsub_rn(my_pv, mx)) : 0.f;
    float total = 0.f;
    for (int sl = 0; sl < used; sl++)
        total = __fadd_rn(total, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wt), sl)));
    my_w = total > 0.f ? __fdiv_rn(wt, total) : wt;
}

// One wave per row (PL = experts per lane / 64, rounded up): the slots'
// picks and weights, kept by lane `slot`.
template <int PL>
__global__ __launch_bounds__(256) void moe_route_kernel(const float *__restrict__ logits, int rows, int E, int used,
                                                        int32_t *__restrict__ ids, float *__restrict__ weights) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    int id;
    float w;
    float v[PL];
    load_route_row<PL>(logits + (uint64_t)r * E, E, v);
    route_row<PL>(v, E, used, id, w);
    if (lane < used) {
        ids[(uint64_t)r * used + lane] = id;
        weights[(uint64_t)r * used + lane] = w;
    }
}

// Routing and binning in one workgroup of 16 waves, for at most 16 rows and
// used <= E (a row's experts are then distinct): wave w routes row w, and
// every pick sets its row's bit in its expert's row mask. (Routing a row is
// a few microseconds of dependent wave reductions, so more rows than waves
// are faster as one wave per row over many workgroups plus moe_bin_kernel.) An assignment's place in its expert's bin is the number of earlier
// rows in that mask, the order moe_bin_kernel gives.
constexpr int kRouteBinWaves = 16;
constexpr int kRouteBinRows = 16;
template <int PL>
__global__ __launch_bounds__(64 * kRouteBinWaves) void moe_route_bin_kernel(
    const float *__restrict__ logits, int rows, int E, int used, int32_t *__restrict__ ids,
    float *__restrict__ weights, int cap, int32_t *__restrict__ counts, int32_t *__restrict__ arows,
    int32_t *__restrict__ aslots, float *__restrict__ aweights) {
    __shared__ unsigned long long mask[64 * kRouteMaxPerLane];
    constexpr int kRounds = kRouteBinRows / kRouteBinWaves;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int e = threadIdx.x; e < E; e += 64 * kRouteBinWaves) mask[e] = 0ull;
    __syncthreads();
    int id[kRounds];
    float w[kRounds];
    float v[kRounds][PL];  // every row's logits requested before the first is routed
#pragma unroll
    for (int i = 0; i < kRounds; i++)
        if (wave + kRouteBinWaves * i < rows)
            load_route_row<PL>(logits + (uint64_t)(wave + kRouteBinWaves * i) * E, E, v[i]);
#pragma unroll
    for (int i = 0; i < kRounds; i++) {
        const int r = wave + kRouteBinWaves * i;
        id[i] = 0;
        w[i] = 0.f;
        if (r < rows) {
            route_row<PL>(v[i], E, used, id[i], w[i]);
            if (lane < used) {
                ids[(uint64_t)r * used + lane] = id[i];
                weights[(uint64_t)r * used + lane] = w[i];
                atomicOr(&mask[id[i]], 1ull << r);
            }
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += 64 * kRouteBinWaves) counts[e] = __popcll(mask[e]);
#pragma unroll
    for (int i = 0; i < kRounds; i++) {
        const int r = wave + kRouteBinWaves * i;
        if (r < rows && lane < used) {
            const uint64_t o = (uint64_t)id[i] * cap + __popcll(mask[id[i]] & ((1ull << r) - 1ull));
            arows[o] = r;
            aslots[o] = lane;
            aweights[o] = w[i];
        }
    }
}

// Workgroup e: expert e's assignments in (row, slot) order. Each pass tests
// 256 assignments; positions from a ballot prefix inside each wave plus the
// earlier waves' counts. Every count is written (no clearing needed).
__global__ __launch_bounds__(256) void moe_bin_kernel(const int32_t *__restrict__ ids,
                                                      const float *__restrict__ weights, int cap, int used,
                                                      int32_t *__restrict__ counts, int32_t *__restrict__ arows,
                                                      int32_t *__restrict__ aslots, float *__restrict__ aweights) {
    __shared__ int wcnt[2][4];
    const int e = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint64_t below = (1ull << lane) - 1ull;
    int base = 0, ph = 0;
    for (int a0 = 0; a0 < cap; a0 += 256, ph ^= 1) {
        const int a = a0 + (int)threadIdx.x;
        const bool hit = a < cap && ids[a] == e;
        const uint64_t b = __ballot(hit);
        if (lane == 0) wcnt[ph][wave] = __popcll(b);
        __syncthreads();  // alternating count buffers: one barrier per pass
        int off = base, tot = 0;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            off += w < wave ? wcnt[ph][w] : 0;
            tot += wcnt[ph][w];
        }
        if (hit) {
            const uint64_t o = (uint64_t)e * cap + off + __popcll(b & below);
            arows[o] = a / used;
            aslots[o] = a % used;
            aweights[o] = weights[a];
        }
        base += tot;
    }
    if (threadIdx.x == 0) counts[e] = base;
}

// ---------------------------------------------------------------- grouped GEMM
// Activation rows quantized once per launch into scratch (moe_quant_kernel):
//   planes [rows][2: high, low][K/64][4][16 B] (moe_quant_kernel's order)
//   scales [rows][K/256]  float (x ~= scale * q, q = 256 h + l)
struct MoeQuant {
    int8_t *planes;
    float *scales;
};

__host__ __device__ inline MoeQuant moe_quant_view(void *ws, int rows, int K) {
    uint8_t *p = static_cast<uint8_t *>(ws);
    MoeQuant q;
    q.planes = reinterpret_cast<int8_t *>(p);
    q.scales = reinterpret_cast<float *>(p + (uint64_t)rows * K * 2);
    return q;
}

// One wave per (row, super-block): lane l holds elements 4l .. 4l+3.
__global__ __launch_bounds__(256) void moe_quant_kernel(const float *__restrict__ x, int rows, int K, MoeQuant q) {
    const int nsb = K / 256;
    const int u = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (u >= rows * nsb) return;
    const int row = u / nsb, sb = u % nsb;
    const float4 v = *reinterpret_cast<const float4 *>(x + (uint64_t)row * K + sb * 256 + 4 * lane);
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    m = wave_max_nonneg(m);
    const float inv = m > 0.f ? (float)kQMax / m : 0.f;
    const int qv[4] = {(int)rintf(v.x * inv), (int)rintf(v.y * inv), (int)rintf(v.z * inv), (int)rintf(v.w * inv)};
    uint32_t hp = 0, lp = 0;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int h = (qv[t] + 128) >> 8;
        const int l = qv[t] - 256 * h;
        hp |= (uint32_t)(h & 0xff) << (8 * t);
        lp |= (uint32_t)(l & 0xff) << (8 * t);
    }
    // row layout: [plane][K/64 groups J][lane group gg][16 B], the 16 bytes
    // being bytes [8 gg, +8) of sub-blocks 2 J and 2 J + 1: the grouped
    // GEMM's LDS tile order, so it stages whole 16-byte pieces
    const int js = sb * 8 + (lane >> 3), o = 4 * (lane & 7);
    int8_t *dst = q.planes + (uint64_t)row * K * 2 + (uint64_t)(js >> 1) * 64 + (o >> 3) * 16 + (js & 1) * 8 + (o & 7);
    *reinterpret_cast<uint32_t *>(dst) = hp;
    *reinterpret_cast<uint32_t *>(dst + K) = lp;
    if (lane == 0) q.scales[(uint64_t)row * nsb + sb] = m > 0.f ? m / (float)kQMax : 0.f;
}

struct MoeGemmArgs {
    const uint8_t *w0;    // expert-stacked Q4_K rows: expert e, output n at row e*N + n
    const uint8_t *w1;    // second matrix of a gate/up pair (or null)
    uint64_t row_bytes;   // bytes of one packed row (K/256 * 144)
    const int32_t *counts, *arows, *aslots;
    MoeQuant xq;
    int rows, used, E, K, N;
    int tpw;              // 16-channel tiles per workgroup
    int by_slot;          // activation row = row*used + slot (down projection), else row
    int swiglu;           // out0 = SiLU(W0 y) * (W1 y)
    int packed;           // w0 / w1 packed (moe_pack_q4k_kernel)
    int shared;           // expert E is the shared expert: every row, output slot `used`
    int ostride;          // slots per row of the activation (down) and output rows: used + shared
    float *out0, *out1;   // [rows*used][N]
};

// Packed expert layout (launch_moe_pack_q4k): per (16-row tile T, super-block
// sb) 2304 contiguous bytes at (T * K/256 + sb) * 2304 — the grouped GEMM's
// 64 lanes' first 16-byte quant pieces (1 KB), their second pieces (1 KB),
// then the 16 rows' 16-byte headers (d, dmin, scales) — so that each of an
// item's three loads is one contiguous 1 KB (or 256 B) wave access.
constexpr int kPackItem = 2304;
// quant-byte offset in the Q4_K block of lane (c, g)'s piece qq (0, 1)
__host__ __device__ inline int moe_piece_off(int g, int qq) { return 16 + 32 * (2 * qq + (g >> 1)) + 16 * (g & 1); }

__global__ __launch_bounds__(256) void moe_pack_q4k_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                           uint64_t rows, int K) {
    // one thread per 16-byte piece: 144 pieces per (tile, super-block)
    const int nsb = K / 256;
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x, n = rows / 16 * nsb * (kPackItem / 16);
    if (i >= n) return;
    const uint64_t item = i / (kPackItem / 16);
    const int p = (int)(i % (kPackItem / 16));
    const uint64_t T = item / nsb;
    const int sb = (int)(item % nsb);
    int row, off;
    if (p < 128) {  // quant pieces: lane l = p & 63 (c = l & 15, g = l >> 4), piece p >> 6
        const int l = p & 63;
        row = l & 15;
        off = moe_piece_off(l >> 4, p >> 6);
    } else {  // header of row p - 128
        row = p - 128;
        off = 0;
    }
    const uint8_t *s = src + ((T * 16 + row) * nsb + sb) * 144 + off;
    *reinterpret_cast<uint4 *>(dst + item * kPackItem + 16 * p) = *reinterpret_cast<const uint4 *>(s);
}

typedef __attribute__((ext_vector_type(2))) unsigned short u16x2;

// Every byte of q times k, for byte products below 256: one packed 16-bit
// multiply (b0 + 256 b1) k = b0 k + 256 b1 k per half, no carry between bytes.
__device__ __forceinline__ uint32_t bytes_times(uint32_t q, uint32_t k) {
    const u16x2 b = {(unsigned short)k, (unsigned short)k};
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, q) * b);
}

// LDS byte offset of the 8 activation bytes of sub-block j, MFMA row r (high
// plane of assignment r for r < 8, low plane of r - 8), lane group gg:
// sub-blocks 2 jp and 2 jp + 1 side by side (one 16-byte read per K = 64).
__device__ __forceinline__ uint32_t moe_la_off(int j, int r, int gg) {
    return ((uint32_t)((((j >> 1) * 16 + r) * 4 + gg) * 2 + (j & 1))) * 8;
}

// tensor/quant.go:96-103 getScaleMinK4 for sub-block j of a Q4_K block
// whose scale bytes 0..11 are the words s1, s2, s3 (block bytes 4..15).
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

// Global -> LDS copies of one lane (lane l writes [m0 + 16 l, +16) or
// [m0 + 4 l, +4)), as inline assembly so that the compiler's wait counts
// do not see them (they would make every weight wait also wait for the
// copies); the kernel waits for them itself before a barrier.
__device__ __forceinline__ void lds_copy16(const void *src, const void *lds_dst) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_dst);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}
__device__ __forceinline__ void lds_copy4(const void *src, const void *lds_dst) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_dst);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}
__device__ __forceinline__ void vmem_wait_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Item (expert e, part): tiles [t0, t0 + tpw) of 16 output channels.
// Per chunk of up to eight assignments, each wave walks its (tile, matrix)
// pairs through the super-blocks in order (sums in registers, the next
// item's weights in flight; deterministic), one result per pair to LDS for
// the epilogue. Lane (c, g) of an item loads channel c's Q4_K bytes straight
// into MFMA B order and the activation planes of assignment c & 7 (high
// plane for c < 8) into A order.
template <bool PACKED>
__global__ __launch_bounds__(kMoeThreads) __attribute__((amdgpu_waves_per_eu(4))) void moe_gemm_kernel(MoeGemmArgs A) {
    // LDS: results [tpw][mats][8 rows][16 ch] floats, then the
    // chunk's activations: planes [K/64][16 r][4 g][2][8 B] (r < 8 high
    // plane of assignment r, r >= 8 low plane of assignment r - 8), scales
    // [K/256][8] float.
    extern __shared__ __attribute__((aligned(16))) float part[];
    const int nsb = A.K / 256;
    const int tiles = A.N / 16;
    const int parts = (tiles + A.tpw - 1) / A.tpw;
    const bool dual = A.w1 != nullptr;
    const int mats = dual ? 2 : 1;
    __shared__ uint16_t s_list[kMoeMaxList];
    __shared__ int s_wtot[kMoeWaves];
    // assignment metadata of three tasks (current, next, the one after):
    // [0, 8) rows, [8, 16) slots, [16] the expert's count
    __shared__ __attribute__((aligned(16))) int s_meta[3][32];
    const uint32_t la_bytes = (uint32_t)A.K * 16;  // one task's planes: K/64 groups of 1 KB
    uint8_t *la = reinterpret_cast<uint8_t *>(part + (uint64_t)A.tpw * mats * 128);
    float *lxs = reinterpret_cast<float *>(la + 2 * (uint64_t)la_bytes);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = lane & 15, g = lane >> 4;
    const uint64_t cap = (uint64_t)A.rows * A.used;

    // The work list: one entry (expert | chunk << 10) per chunk of up to
    // kChunk assignments of every expert some row selected, in expert and
    // chunk order (wave prefix sums of the chunk counts, wave totals added in
    // wave order); with A.shared, expert E is the shared expert and holds
    // every row. The work items are (entry, tile part) pairs dealt
    // round-robin over the grid, so every workgroup gets an equal share
    // wherever the assignments fall.
    const int nexp = A.E + (A.shared ? 1 : 0);
    int nlist = 0;
    for (int b0 = 0; b0 < nexp; b0 += kMoeThreads) {
        const int ex = b0 + (int)threadIdx.x;
        const int cnt = ex < A.E ? A.counts[ex] : (ex < nexp ? A.rows : 0);
        const int nch = (max(cnt, 0) + kChunk - 1) / kChunk;
        int incl = nch;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(incl, d);
            if (lane >= d) incl += o;
        }
        if (lane == 63) s_wtot[wave] = incl;
        __syncthreads();
        int base = nlist + incl - nch;
        for (int w = 0; w < wave; w++) base += s_wtot[w];
        for (int j = 0; j < nch; j++) s_list[base + j] = (uint16_t)(ex | (j << 10));
        for (int w = 0; w < kMoeWaves; w++) nlist += s_wtot[w];
        __syncthreads();
    }
    const int items = nlist * parts;
    if ((int)blockIdx.x >= items) return;  // workgroup-uniform

    // Task k is this workgroup's item k, blockIdx.x + k * gridDim.x. Task
    // k's planes and scales sit in LDS buffer k & 1, its metadata in slot
    // k % 3; task k + 1's planes and task k + 2's metadata are copied into
    // LDS (global_load_lds, outside the compiler's wait counts) while task k
    // streams its weights, and every wave waits for its own copies (vmcnt 0)
    // before the barrier that ends task k.
    auto item_of = [&](int k) { return (int)blockIdx.x + k * (int)gridDim.x; };
    auto entry_of = [&](int k) { return (int)s_list[item_of(k) / parts]; };
    auto meta_issue = [&](int k, int slot) __attribute__((always_inline)) {
        const int en = entry_of(k), e = en & 1023, c0 = (en >> 10) * kChunk;
        if (wave == 0 && lane < 17) {
            if (e == A.E) {  // the shared expert: rows c0.., slot `used`, count rows
                s_meta[slot][lane] = lane < 8 ? min(c0 + lane, A.rows - 1) : lane < 16 ? A.used : A.rows;
            } else {
                const uint64_t b = (uint64_t)e * cap;
                const int32_t *src = lane < 8    ? A.arows + b + min((uint64_t)(c0 + lane), cap - 1)
                                     : lane < 16 ? A.aslots + b + min((uint64_t)(c0 + lane - 8), cap - 1)
                                                 : A.counts + e;
                lds_copy4(src, &s_meta[slot][0]);
            }
        }
    };
    // activation row of assignment i of a task (padding rows repeat the
    // chunk's first assignment and are never stored)
    auto act_row = [&](const int *mt, int c0, int i) __attribute__((always_inline)) {
        const int j = c0 + i < mt[16] ? i : 0;
        return A.by_slot ? mt[j] * A.ostride + mt[8 + j] : mt[j];
    };
    auto stage_issue = [&](int c0, int slot, int buf) __attribute__((always_inline)) {
        const int *mt = s_meta[slot];
        uint8_t *dst = la + (uint64_t)buf * la_bytes;
        {   // planes: lane l of group J copies MFMA row l >> 2, lane group l & 3
            const int r = lane >> 2, gg = lane & 3;
            const int8_t *src = A.xq.planes + (uint64_t)act_row(mt, c0, r & 7) * A.K * 2 + (r >= 8 ? A.K : 0) + gg * 16;
            for (int J = wave; J < A.K / 64; J += kMoeWaves) lds_copy16(src + J * 64, dst + J * 1024);
        }
        float *xd = lxs + (uint64_t)buf * nsb * 8;  // scales [K/256][8]
        for (int b = wave; b * 64 < nsb * 8; b += kMoeWaves) {
            const int idx = b * 64 + lane;
            if (idx < nsb * 8) lds_copy4(A.xq.scales + (uint64_t)act_row(mt, c0, idx & 7) * nsb + (idx >> 3), xd + b * 64);
        }
    };

    // task 0: metadata, then its planes with task 1's metadata
    meta_issue(0, 0);
    vmem_wait_all();
    __syncthreads();
    if (item_of(1) < items) meta_issue(1, 1);
    stage_issue((entry_of(0) >> 10) * kChunk, 0, 0);
    vmem_wait_all();
    __syncthreads();
    for (int k = 0;; k++) {
        const int slot = k % 3, buf = k & 1;
        const int *mt = s_meta[slot];
        const int en = entry_of(k), e = en & 1023, c0 = (en >> 10) * kChunk;
        const int count = mt[16], nr = min(kChunk, count - c0);
        const int t0 = (item_of(k) % parts) * A.tpw, ntl = min(A.tpw, tiles - t0);
        // the next task's planes, and the metadata of the one after it
        if (item_of(k + 1) < items) {
            stage_issue((entry_of(k + 1) >> 10) * kChunk, (k + 1) % 3, buf ^ 1);
            if (item_of(k + 2) < items) meta_issue(k + 2, (k + 2) % 3);
        }
        const uint8_t *lat = la + (uint64_t)buf * la_bytes;
        const float *lxt = lxs + (uint64_t)buf * nsb * 8;
        // items (tile, matrix, super-block): wave w walks the pairs (tile,
        // matrix) w, w + 8, ... through their super-blocks in order with the
        // next item's weights in flight, sums in registers in super-block
        // order, one result per pair to LDS
        const int pairs = ntl * mats;
        const int npw = wave < pairs ? (pairs - wave + kMoeWaves - 1) / kMoeWaves : 0;
        const int total = npw * nsb;
        const int rbase = 4 * (g & 1);
        // quant bytes of an item: lane (c, g) loads 16 contiguous bytes per
        // half of the block, [32 jp + 16 (g & 1), +16) with jp = 2 qq + (g >> 1),
        // so each load covers 64 contiguous bytes of every channel; the
        // activation operands below follow the same (sub-block, element)
        // assignment (the MFMA sums over K in any order)
        auto load_item = [&](int q, uint4 &H, uint4 (&Q)[2]) __attribute__((always_inline)) {
            int oz;  // opaque zero: the lane's row address is rebuilt per item, not held (and spilled)
            asm volatile("s_mov_b32 %0, 0" : "=s"(oz));
            const int lc = c + oz, lg = g + oz;
            const int tm = wave + kMoeWaves * (q / nsb), sb = q % nsb, m = tm % mats, tl = tm / mats;
            const uint8_t *w = m ? A.w1 : A.w0;
            if constexpr (PACKED) {
                const uint8_t *it = w + ((uint64_t)(e * (A.N / 16) + t0 + tl) * nsb + sb) * kPackItem;
                Q[0] = *reinterpret_cast<const uint4 *>(it + 16 * (lc + 16 * lg));
                Q[1] = *reinterpret_cast<const uint4 *>(it + 1024 + 16 * (lc + 16 * lg));
                H = *reinterpret_cast<const uint4 *>(it + 2048 + 16 * lc);
            } else {
                const uint8_t *blk = w + ((uint64_t)e * A.N + (t0 + tl) * 16 + lc) * A.row_bytes + (uint64_t)sb * 144;
                H = *reinterpret_cast<const uint4 *>(blk);
#pragma unroll
                for (int qq = 0; qq < 2; qq++) Q[qq] = *reinterpret_cast<const uint4 *>(blk + moe_piece_off(lg, qq));
            }
        };
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        auto compute_item = [&](int q, const uint4 &H, const uint4 (&Q)[2]) __attribute__((always_inline)) {
            const int sb = q % nsb;
            const float4 xs4 = *reinterpret_cast<const float4 *>(lxt + sb * 8 + rbase);
            const float xs[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
            // sub-block scale (two 3-bit digits) and min in the B operands
            // of three K = 64 MFMAs per pair of sub-blocks: exact int32
            i32x4 alo = {0, 0, 0, 0}, ahi = {0, 0, 0, 0}, amn = {0, 0, 0, 0};
            // this lane's scale bytes: sub-blocks 2 jp, 2 jp + 1 of jp = 2 qq + b
            // sit in bytes 2 b, 2 b + 1 of each scale word (getScaleMinK4 layout)
            int oz;  // opaque zero: lane-derived offsets are rebuilt per item
            asm volatile("s_mov_b32 %0, 0" : "=s"(oz));
            const int lc = c + oz, lg = g + oz, b = lg >> 1;
            const uint32_t y1 = H.y >> (16 * b), z1 = H.z >> (16 * b), w1 = H.w >> (16 * b);
#pragma unroll
            for (int mi = 0; mi < 4; mi++) {
                const int qq = mi >> 1, hh = mi & 1, jp = 2 * qq + b;
                const uint64_t raw = hh ? ((uint64_t)Q[qq].z | ((uint64_t)Q[qq].w << 32))
                                        : ((uint64_t)Q[qq].x | ((uint64_t)Q[qq].y << 32));
                const uint64_t qe = raw & 0x0F0F0F0F0F0F0F0Full, qo = (raw >> 4) & 0x0F0F0F0F0F0F0F0Full;
                int sce, mne, sco, mno;
                if (qq == 0) {  // sub-blocks 0..3: low six bits of scale / min bytes
                    sce = (int)(y1 & 63);
                    sco = (int)((y1 >> 8) & 63);
                    mne = (int)(z1 & 63);
                    mno = (int)((z1 >> 8) & 63);
                } else {  // sub-blocks 4..7: nibbles of bytes 8..11, high bits of 0..7
                    sce = (int)((w1 & 0xF) | (((y1 >> 6) & 3) << 4));
                    sco = (int)(((w1 >> 8) & 0xF) | (((y1 >> 14) & 3) << 4));
                    mne = (int)(((w1 >> 4) & 0xF) | (((z1 >> 6) & 3) << 4));
                    mno = (int)(((w1 >> 12) & 0xF) | (((z1 >> 14) & 3) << 4));
                }
                const uint32_t qw[4] = {(uint32_t)qe, (uint32_t)(qe >> 32), (uint32_t)qo, (uint32_t)(qo >> 32)};
                const uint32_t lo[2] = {(uint32_t)(sce & 7), (uint32_t)(sco & 7)};
                const uint32_t hi[2] = {(uint32_t)(sce >> 3), (uint32_t)(sco >> 3)};
                const i32x4 b_lo = {(int)bytes_times(qw[0], lo[0]), (int)bytes_times(qw[1], lo[0]),
                                    (int)bytes_times(qw[2], lo[1]), (int)bytes_times(qw[3], lo[1])};
                const i32x4 b_hi = {(int)bytes_times(qw[0], hi[0]), (int)bytes_times(qw[1], hi[0]),
                                    (int)bytes_times(qw[2], hi[1]), (int)bytes_times(qw[3], hi[1])};
                const int me = (int)__builtin_amdgcn_perm((uint32_t)mne, (uint32_t)mne, 0u);
                const int mo = (int)__builtin_amdgcn_perm((uint32_t)mno, (uint32_t)mno, 0u);
                const i32x4 b_mn = {me, me, mo, mo};
                const i32x4 av =
                    *reinterpret_cast<const i32x4 *>(lat + moe_la_off(sb * 8 + 2 * jp, lc, 2 * (lg & 1) + hh));
                alo = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b_lo, alo, 0, 0, 0);
                ahi = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b_hi, ahi, 0, 0, 0);
                amn = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, b_mn, amn, 0, 0, 0);
            }
            const float d = h2f((uint16_t)(H.x & 0xffffu)), dmin = h2f((uint16_t)(H.x >> 16));
#pragma unroll
            for (int i = 0; i < 4; i++) {
                // this lane's plane (rows 0..7 high, 8..15 low); the planes
                // are combined once per pair
                const float v = d * (float)(alo[i] + 8 * ahi[i]) - dmin * (float)amn[i];
                acc[i] += xs[i] * v;
            }
            if (sb == nsb - 1) {  // the pair's last super-block: its result to LDS
                const int tm = wave + kMoeWaves * (q / nsb);
                float *dst = part + (uint64_t)tm * 128;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float lo = __shfl_xor(acc[i], 32);
                    if (g < 2) dst[(4 * g + i) * 16 + c] = fmaf(256.f, acc[i], lo);
                    acc[i] = 0.f;
                }
            }
        };
        // Every load past the first is issued unconditionally (the item index
        // clamped to the wave's last item, which is then read again): loads
        // under a branch make the compiler's wait counts merge conservatively,
        // and the multiply of one stage would wait for the other stage's
        // loads too. Each stage keeps its own code path (two items per
        // iteration).
        uint4 h0, h1;
        uint4 q0[2], q1[2];
        if (total > 0) {  // wave-uniform
            load_item(0, h0, q0);
            load_item(min(1, total - 1), h1, q1);
            for (int q = 0; q < total; q += 2) {
                compute_item(q, h0, q0);
                __builtin_amdgcn_sched_barrier(0);
                load_item(min(q + 2, total - 1), h0, q0);
                if (q + 1 < total) compute_item(q + 1, h1, q1);
                __builtin_amdgcn_sched_barrier(0);
                load_item(min(q + 3, total - 1), h1, q1);
            }
        }
        __syncthreads();
        // the epilogue
        for (int o = threadIdx.x; o < ntl * nr * 16; o += kMoeThreads) {
            const int tl = o / (nr * 16), rem = o % (nr * 16), i = rem / 16, cc = rem % 16;
            float y[2] = {0.f, 0.f};
            for (int m = 0; m < mats; m++) y[m] = part[(uint64_t)(tl * mats + m) * 128 + i * 16 + cc];
            const uint64_t dst = (uint64_t)(mt[i] * A.ostride + mt[8 + i]) * A.N + (t0 + tl) * 16 + cc;
            if (A.swiglu) {
                A.out0[dst] = __fmul_rn(silu_ref(y[0]), y[1]);
            } else {
                A.out0[dst] = y[0];
                if (dual) A.out1[dst] = y[1];
            }
        }
        vmem_wait_all();
        __syncthreads();
        if (item_of(k + 1) >= items) break;
    }
}

// ---------------------------------------------------------------- reduce
// x[r] += sum_slot w[r][slot] * out[r*used + slot] (yuuka_hip.h:468-469),
// and with `so`: + sigmoid(sg[r]) * so[r] (forward.go:381-388). float32
// operations in the reference's order, no contraction (written as plain
// operators under the pragma: the __fmul_rn / __fadd_rn helpers are defined
// in a contractable context and would still be fused after inlining).
// With `shared_slot` the shared expert's output is slot `used` of eo (rows
// of used + 1 slots) instead of `so`.
__global__ __launch_bounds__(256) void moe_combine_kernel(float *__restrict__ x, const float *__restrict__ eo,
                                                          const float *__restrict__ w, int rows, int used, int H,
                                                          const float *__restrict__ so,
                                                          const float *__restrict__ sg, int shared_slot) {
#pragma clang fp contract(off)  // the reference rounds every product and sum
    const int r = blockIdx.x;
    const int ostride = used + (shared_slot ? 1 : 0);
    const float *er = eo + (uint64_t)r * ostride * H;
    const float *wr = w + (uint64_t)r * used;
    const float *sr = shared_slot ? er + (uint64_t)used * H : (so ? so + (uint64_t)r * H : nullptr);
    const float gate = sr ? sigmoid_ref(sg[r]) : 0.f;
    const int i = blockIdx.y * blockDim.x + threadIdx.x;  // grid (rows, H / 256): one element per thread
    if (i < H) {
        float t = 0.f;
#pragma unroll 8
        for (int s = 0; s < used; s++) t = t + wr[s] * er[(uint64_t)s * H + i];
        if (sr) t = t + gate * sr[i];
        x[(uint64_t)r * H + i] = x[(uint64_t)r * H + i] + t;
    }
}

}  // namespace

uint64_t moe_gemm_ws(int act_rows, int K) { return (uint64_t)act_rows * K * 2 + (uint64_t)act_rows * (K / 256) * 4 + 256; }

hipError_t launch_moe_router(const float *y, int H, int rows, const float *w, int E, float *logits, const float *sv,
                             float *extra, hipStream_t s) {
    const int n = E + (sv ? 1 : 0);
    moe_router_kernel<<<dim3((unsigned)((n + kRouterExperts - 1) / kRouterExperts),
                             (unsigned)((rows + kRouterRows - 1) / kRouterRows)),
                        64 * kRouterWaves, 0, s>>>(y, H, rows, w, E, logits, sv, extra);
    return hipGetLastError();
}

hipError_t launch_moe_route(const float *logits, int rows, int E, int used, int32_t *ids, float *weights,
                            int32_t *counts, int32_t *arows, int32_t *aslots, float *aweights, hipStream_t s) {
    if (E > 64 * kRouteMaxPerLane || used > 64) return hipErrorInvalidValue;
    if (rows <= kRouteBinRows && used <= E) {
        if (E <= 256)
            moe_route_bin_kernel<4><<<1, 64 * kRouteBinWaves, 0, s>>>(logits, rows, E, used, ids, weights, rows * used,
                                                                      counts, arows, aslots, aweights);
        else if (E <= 512)
            moe_route_bin_kernel<8><<<1, 64 * kRouteBinWaves, 0, s>>>(logits, rows, E, used, ids, weights, rows * used,
                                                                      counts, arows, aslots, aweights);
        else
            moe_route_bin_kernel<16><<<1, 64 * kRouteBinWaves, 0, s>>>(logits, rows, E, used, ids, weights,
                                                                       rows * used, counts, arows, aslots, aweights);
        return hipGetLastError();
    }
    const unsigned g = (unsigned)((rows + 3) / 4);
    if (E <= 256) moe_route_kernel<4><<<g, 256, 0, s>>>(logits, rows, E, used, ids, weights);
    else if (E <= 512) moe_route_kernel<8><<<g, 256, 0, s>>>(logits, rows, E, used, ids, weights);
    else moe_route_kernel<16><<<g, 256, 0, s>>>(logits, rows, E, used, ids, weights);
    moe_bin_kernel<<<(unsigned)E, 256, 0, s>>>(ids, weights, rows * used, used, counts, arows, aslots, aweights);
    return hipGetLastError();
}

// Resident workgroups of the grouped GEMM variant at this LDS size on the
// current device: measured once per (device, variant, LDS size) under a lock
// (gate/up and down launches differ in LDS, so a single cached entry would be
// recomputed on nearly every launch).
static unsigned moe_resident_wgs(bool packed, uint32_t lds) {
    static std::mutex mu;
    static std::map<std::tuple<int, bool, uint32_t>, unsigned> cache;
    int dev = 0;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_tuple(dev, packed, lds);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 1;
    const void *fn = packed ? reinterpret_cast<const void *>(moe_gemm_kernel<true>)
                            : reinterpret_cast<const void *>(moe_gemm_kernel<false>);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kMoeThreads, lds) != hipSuccess || per_cu <= 0)
        per_cu = 1;
    const unsigned r = (unsigned)(per_cu * cus);
    cache.emplace(key, r);
    return r;
}

hipError_t launch_moe_gemm(const MoeGemm &g, void *ws, hipStream_t s) {
    const int ostride = g.used + (g.shared ? 1 : 0);
    const int act_rows = g.by_slot ? g.rows * ostride : g.rows;
    // work-list bounds: expert | chunk << 10 in 16 bits, at most kMoeMaxList entries
    if (g.experts + (g.shared ? 1 : 0) > kMoeMaxExperts || g.rows > kMoeMaxRows ||
        g.experts + 1 + (g.rows * ostride) / kChunk > kMoeMaxList)
        return hipErrorInvalidValue;
    MoeGemmArgs a{};
    a.w0 = static_cast<const uint8_t *>(g.w0);
    a.w1 = static_cast<const uint8_t *>(g.w1);
    a.row_bytes = g.row_bytes;
    a.counts = g.counts;
    a.arows = g.arows;
    a.aslots = g.aslots;
    a.xq = moe_quant_view(ws, act_rows, g.K);
    a.rows = g.rows;
    a.used = g.used;
    a.E = g.experts;
    a.K = g.K;
    a.N = g.N;
    a.by_slot = g.by_slot;
    a.swiglu = g.swiglu;
    a.packed = g.packed;
    a.shared = g.shared ? 1 : 0;
    a.ostride = ostride;
    a.out0 = g.out0;
    a.out1 = g.out1;
    const int nsb = g.K / 256, mats = g.w1 ? 2 : 1, tiles = g.N / 16;
    // tiles per workgroup: as many as keep nsb * mats * tpw items near 64
    // (enough workgroups in flight; each wave walks a few pairs)
    int tpw = (32 * 1024) / (nsb * mats * 512);
    tpw = std::max(1, std::min(tpw, 16));
    tpw = std::min(tpw, tiles);
    a.tpw = tpw;
    // results, two buffers of planes (K/64 groups of 1 KB) and of scales
    const uint32_t lds = (uint32_t)tpw * mats * 512 + 2 * (uint32_t)g.K * 16 + 2 * (uint32_t)nsb * 32;
    const int units = act_rows * nsb;
    moe_quant_kernel<<<(units + 3) / 4, 256, 0, s>>>(g.x, act_rows, g.K, a.xq);
    // a persistent grid of the resident workgroups (the kernel deals the
    // active experts' items over it)
    const int parts = (tiles + tpw - 1) / tpw;
    const unsigned grid = (unsigned)std::min<int64_t>((int64_t)g.experts * parts, moe_resident_wgs(g.packed != 0, lds));
    if (g.packed) moe_gemm_kernel<true><<<grid, kMoeThreads, lds, s>>>(a);
    else moe_gemm_kernel<false><<<grid, kMoeThreads, lds, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_moe_pack_q4k(const void *src, void *dst, uint64_t rows, int K, hipStream_t s) {
    if (rows % 16 || K % 256 || K <= 0) return hipErrorInvalidValue;
    const uint64_t n = rows / 16 * (uint64_t)(K / 256) * (kPackItem / 16);
    if (n == 0) return hipSuccess;
    moe_pack_q4k_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(static_cast<const uint8_t *>(src),
                                                                     static_cast<uint8_t *>(dst), rows, K);
    return hipGetLastError();
}

hipError_t launch_moe_combine(float *x, const float *eo, const float *w, int rows, int used, int H, const float *so,
                              const float *sg, hipStream_t s, bool shared_slot) {
    moe_combine_kernel<<<dim3((unsigned)rows, (unsigned)((H + 255) / 256)), 256, 0, s>>>(x, eo, w, rows, used, H, so, sg,
                                                                                         shared_slot ? 1 : 0);
    return hipGetLastError();
}

}  // namespace yk
