// k_attn.hip — paged attention of the verify rows for one gated-attention
// layer, with the per-head q/k RMSNorm, RoPE and the KV-cache write folded in.
//
// The reference runs this as separate ops (model/qwen35/forward.go:418-458
// through engine/gpu/plan.go: k norm, k RoPE, KV write, q norm, q RoPE,
// attention). Here one kernel does all of them:
//  * grid = (key chunks, kv heads); a workgroup owns CK consecutive key
//    positions of one kv head and every query row of that head's group
//    (heads / kv_heads query heads x rows);
//  * every workgroup normalises and rotates its query rows itself (they are
//    tiny), so no kernel has to finish first;
//  * keys before the verify rows come from the paged pool; the verify rows'
//    own keys and values are computed by the workgroup whose chunk holds
//    their positions, rounded exactly as the pool stores them (F16: the
//    reference's round-half-up Float32ToFloat16), used from LDS and written
//    to the pool once;
//  * scores, softmax partials and the value product run from LDS; the
//    per-chunk partials {sum p*v, max, sum p} are merged (and gated) by
//    attn_merge, as flash-decoding does.
// RoPE angles come from rope_table_kernel, computed once per step in float64
// (forward.go:495-514).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>

#include "model_kernels.h"
#include "refmath.h"

namespace yk {
namespace {


__device__ __forceinline__ int cur_pos_a(const ModelDyn &dyn) { return dyn.pos_dev ? *dyn.pos_dev : dyn.pos; }

// exp(x) for finite x <= 0 (a score minus its row's running maximum), in
// float32 as the reference's GPU attention kernels compute it
// (kernels/hip/attention: expf of score - max). 2^(x log2 e) on the hardware
// exp2 (v_exp_f32), with the rounding error of the product x * L1 (an FMA
// residual) and the low part L2 of log2 e carried as a factor 2^r ~ 1 + r ln 2
// (|r| < 2^-17, so r^2 is below float precision): relative error ~1e-7
// against the float64 exp, instead of ~|x| 2^-24 for exp2(x * log2 e).
__device__ __forceinline__ float exp_nonpos(float x) {
    constexpr float L1 = 1.44269502162933349609375f;  // log2(e) rounded to float
    constexpr float L2 = 1.92596298909e-8f;            // log2(e) - L1
    // exp(-128) is 0 in float; the clamp keeps x * L1 and its residual
    // finite. A NaN score stays NaN (fmaxf would turn it into -128), as the
    // reference's expf lets it through to the output.
    x = x == x ? fmaxf(x, -128.0f) : x;
    const float p = x * L1;
    const float r = fmaf(x, L1, -p) + x * L2;
    return __builtin_amdgcn_exp2f(p) * fmaf(r, 0.693147180559945309f, 1.0f);
}

__device__ __forceinline__ double wave_sum_d(double v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}
__device__ __forceinline__ float wave_sum_f(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// cos / sin of every (row, rotation pair): theta = pos * base^(-2i/rot).
__global__ void rope_table_kernel(float2 *__restrict__ tab, int rows, int rot_dim, double base, ModelDyn dyn,
                                  int displacement, int rq_rows) {
    const int half = rot_dim / 2;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * half) return;
    if (blockIdx.y) {  // request blockIdx.y: its rows and {token, position} pair
        tab += (uint64_t)blockIdx.y * rq_rows * half;
        if (dyn.pos_dev) dyn.pos_dev += 2 * blockIdx.y;
    }
    const int r = idx / half, i = idx % half;
    const int pos = cur_pos_a(dyn) + displacement + r;
    const double theta = (double)pos * pow(base, -2.0 * (double)i / (double)rot_dim);
    tab[idx] = make_float2((float)cos(theta), (float)sin(theta));
}

// Request blockIdx.z of a batched launch: offsets of its query rows (q),
// key / value rows (kv), block table, rope rows, partial-result slab and
// {token, position} pair.
struct AttnReqOff {
    uint64_t q, kv, table, rope, part;
    int pos;
};

__device__ __forceinline__ AttnReqOff attn_request(const AttnVArgs &a, int ck) {
    const uint64_t rq = blockIdx.z;
    const uint64_t rows = rq * a.rq_rows;
    AttnReqOff o;
    o.q = rows * a.heads * (a.gated ? 2 * a.head_dim : a.head_dim);
    o.kv = rows * a.kv_dim;
    o.table = rq * (uint64_t)((a.capacity + a.block_size - 1) / a.block_size);
    o.rope = rows * (a.rope_dim / 2);
    o.part = rq * (uint64_t)((a.capacity + ck - 1) / ck) * a.rows * a.heads * (a.head_dim + 2);
    o.pos = 2 * (int)rq;
    return o;
}

#define YK_ATTN_REQUEST(CK)                                  \
    {                                                        \
        const AttnReqOff ro_ = attn_request(a, CK);          \
        q += ro_.q;                                          \
        k += ro_.kv;                                         \
        v += ro_.kv;                                         \
        table += ro_.table;                                  \
        rope += ro_.rope;                                    \
        part += ro_.part;                                    \
        if (dyn.pos_dev) dyn.pos_dev += ro_.pos;             \
    }

template <int FMT> struct KvT;
// CK keys per workgroup; rows of K / V in LDS are padded by PAD elements
// (16-byte aligned rows, spread over the banks).
template <> struct KvT<0> { using T = float; static constexpr int CK = 32, PAD = 4; };
template <> struct KvT<1> { using T = uint16_t; static constexpr int CK = 64, PAD = 8; };

// Four consecutive K / V elements of an LDS row as floats.
__device__ __forceinline__ float4 kv4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ float4 kv4(const uint16_t *p) {
    const uint2 u = *reinterpret_cast<const uint2 *>(p);
    return make_float4(h2f((uint16_t)(u.x & 0xffffu)), h2f((uint16_t)(u.x >> 16)), h2f((uint16_t)(u.y & 0xffffu)),
                       h2f((uint16_t)(u.y >> 16)));
}

template <int FMT>
__device__ __forceinline__ float kv_val(typename KvT<FMT>::T v) {
    if constexpr (FMT == 1) return h2f(v);
    else return v;
}
template <int FMT>
__device__ __forceinline__ typename KvT<FMT>::T kv_store(float v) {
    if constexpr (FMT == 1) return ref_f32_to_f16(v);
    else return v;
}

// Per-head RMSNorm (x * (scale * w), forward.go:472-482) and RoPE of one
// D-vector by one wave, written to dst (LDS). Returns nothing; lanes hold
// elements l, l + 64, ...
__device__ __forceinline__ void norm_rope_wave(const float *__restrict__ src, const float *__restrict__ w,
                                               float *dst, int D, float eps, const float2 *__restrict__ cs,
                                               int half) {
    const int lane = threadIdx.x & 63;
    float x[4];
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int d = lane + 64 * i;
        x[i] = d < D ? src[d] : 0.0f;
        ss += (double)x[i] * (double)x[i];
    }
    ss = wave_sum_d(ss);
    const float mean = (float)(ss / (double)D);
    const float scale = (float)(1.0 / sqrt((double)(mean + eps)));
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int d = lane + 64 * i;
        if (d < D) dst[d] = __fmul_rn(x[i], __fmul_rn(scale, w[d]));
    }
    // rotation pairs (i, i + half), i < half <= 64: one lane each
    float y0 = 0.0f, y1 = 0.0f;
    if (lane < half) {
        y0 = dst[lane];
        y1 = dst[lane + half];
    }
    if (lane < half) {
#pragma clang fp contract(off)  // float32 products and sums rounded separately, as the reference
        const float c = cs[lane].x, s = cs[lane].y;
        dst[lane] = y0 * c - y1 * s;
        dst[lane + half] = y0 * s + y1 * c;
    }
}

template <int FMT>
__global__ __launch_bounds__(256) void attn_verify_kernel(const float *__restrict__ q, const float *__restrict__ k,
                                                          const float *__restrict__ v, uint8_t *kpool_b,
                                                          uint8_t *vpool_b, const int32_t *__restrict__ table,
                                                          const float *__restrict__ q_norm,
                                                          const float *__restrict__ k_norm,
                                                          const float2 *__restrict__ rope, AttnVArgs a,
                                                          float *__restrict__ part, ModelDyn dyn) {
    using T = typename KvT<FMT>::T;
    constexpr int CK = KvT<FMT>::CK, PAD = KvT<FMT>::PAD;
    extern __shared__ __align__(16) uint8_t lds[];
    T *kpool = reinterpret_cast<T *>(kpool_b);
    T *vpool = reinterpret_cast<T *>(vpool_b);
    YK_ATTN_REQUEST(CK);
    const int kvh = blockIdx.y, chunk = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int D = a.head_dim, R = a.rows;
    const int G = a.heads / a.kv_heads, nq = G * R;
    const int p0 = cur_pos_a(dyn) + a.displacement;  // position of verify row 0
    const int last = p0 + R - 1;
    const int key0 = chunk * CK;
    if (key0 > last) return;  // no row sees this chunk; the merge skips it
    const int half = a.rope_dim / 2;
    const int qstride = a.gated ? 2 * D : D;
    const int ks = D + PAD;  // LDS row stride of K and V (elements)
    float *Qs = reinterpret_cast<float *>(lds);                       // [nq][D]
    T *Ks = reinterpret_cast<T *>(Qs + nq * D);                       // [CK][ks]
    T *Vs = Ks + CK * ks;                                             // [CK][ks]
    float *S = reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(Vs + CK * ks) + 0);  // [nq][CK]
    // 16-byte align S
    S = reinterpret_cast<float *>((reinterpret_cast<uintptr_t>(S) + 15) & ~uintptr_t(15));

    // ---- cached keys / values of this chunk (positions < p0), coalesced
    {
        constexpr int PER = 256 / CK;  // threads per key row
        const int kk = threadIdx.x / PER, part_i = threadIdx.x % PER;
        const int p = key0 + kk;
        const int span = D / PER;  // elements per thread
        T *kd = Ks + kk * ks + part_i * span;
        T *vd = Vs + kk * ks + part_i * span;
        const int n16 = span * (int)sizeof(T) / 16;  // 16-byte pieces per thread
        if (p < p0) {
            const int64_t slot = (int64_t)table[p / a.block_size] * a.block_size + p % a.block_size;
            const uint4 *kr = reinterpret_cast<const uint4 *>(kpool + slot * a.kv_dim + (int64_t)kvh * D + part_i * span);
            const uint4 *vr = reinterpret_cast<const uint4 *>(vpool + slot * a.kv_dim + (int64_t)kvh * D + part_i * span);
            for (int e = 0; e < n16; e++) {
                reinterpret_cast<uint4 *>(kd)[e] = kr[e];
                reinterpret_cast<uint4 *>(vd)[e] = vr[e];
            }
        } else if (p > last) {
            for (int e = 0; e < n16; e++) {
                reinterpret_cast<uint4 *>(kd)[e] = make_uint4(0, 0, 0, 0);
                reinterpret_cast<uint4 *>(vd)[e] = make_uint4(0, 0, 0, 0);
            }
        }
    }
    // ---- query rows (normalised and rotated) and this chunk's new keys
    for (int vec = wave; vec < nq; vec += 4) {
        const int g = vec / R, r = vec % R;
        const int head = kvh * G + g;
        norm_rope_wave(q + ((int64_t)r * a.heads + head) * qstride, q_norm, Qs + vec * D, D, a.eps,
                       rope + r * half, half);
    }
    float *kbuf = S;  // scratch for one new key row per wave (S is free until the scores)
    for (int r = wave; r < R; r += 4) {
        const int p = p0 + r;
        if (p < key0 || p >= key0 + CK) continue;
        const int kk = p - key0;
        float *kw = kbuf + wave * D;
        norm_rope_wave(k + (int64_t)r * a.kv_dim + (int64_t)kvh * D, k_norm, kw, D, a.eps, rope + r * half, half);
        const int64_t slot = (int64_t)table[p / a.block_size] * a.block_size + p % a.block_size;
        for (int d = lane; d < D; d += 64) {
            const T kq = kv_store<FMT>(kw[d]);
            const T vq = kv_store<FMT>(v[(int64_t)r * a.kv_dim + (int64_t)kvh * D + d]);
            Ks[kk * ks + d] = kq;
            Vs[kk * ks + d] = vq;
            kpool[slot * a.kv_dim + (int64_t)kvh * D + d] = kq;
            vpool[slot * a.kv_dim + (int64_t)kvh * D + d] = vq;
        }
    }
    __syncthreads();

    // ---- scores: thread = (key kk, query group), full D, 8 queries a pass
    {
        constexpr int QG = 256 / CK;  // query groups
        const int kk = threadIdx.x % CK, qg = threadIdx.x / CK;
        const int p = key0 + kk;
        const T *kr = Ks + kk * ks;
        for (int j0 = qg; j0 < nq; j0 += QG * 8) {
            float acc[8];
#pragma unroll
            for (int u = 0; u < 8; u++) acc[u] = 0.0f;
            for (int d = 0; d < D; d += 4) {
                const float4 kd = kv4(kr + d);
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int j = min(j0 + u * QG, nq - 1);
                    const float4 qd = *reinterpret_cast<const float4 *>(Qs + j * D + d);
                    acc[u] = fmaf(qd.x, kd.x, acc[u]);
                    acc[u] = fmaf(qd.y, kd.y, acc[u]);
                    acc[u] = fmaf(qd.z, kd.z, acc[u]);
                    acc[u] = fmaf(qd.w, kd.w, acc[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int j = j0 + u * QG;
                if (j < nq) {
                    const int r = j % R;
                    S[j * CK + kk] = p <= p0 + r ? acc[u] * a.scale : -INFINITY;
                }
            }
        }
    }
    __syncthreads();
    // ---- softmax partials: one wave per query row of the chunk
    for (int j = wave; j < nq; j += 4) {
        const float sc = lane < CK ? S[j * CK + lane] : -INFINITY;
        const float m = wave_max_f(sc);
        const float e = (sc == -INFINITY) ? 0.0f : exp_nonpos(sc - m);
        const float l = wave_sum_f(e);
        if (lane < CK) S[j * CK + lane] = e;
        if (lane == 0) {
            const int g = j / R, r = j % R;
            float *rec = part + (((int64_t)chunk * R + r) * a.heads + kvh * G + g) * (D + 2);
            rec[D] = m;
            rec[D + 1] = l;
        }
    }
    __syncthreads();
    // ---- value product: thread = dimension d, 16 query rows a pass
    for (int d = threadIdx.x; d < D; d += 256) {
        for (int j0 = 0; j0 < nq; j0 += 16) {
            float acc[16];
#pragma unroll
            for (int u = 0; u < 16; u++) acc[u] = 0.0f;
            for (int kk = 0; kk < CK; kk += 4) {
                const float v0 = kv_val<FMT>(Vs[(kk + 0) * ks + d]), v1 = kv_val<FMT>(Vs[(kk + 1) * ks + d]);
                const float v2 = kv_val<FMT>(Vs[(kk + 2) * ks + d]), v3 = kv_val<FMT>(Vs[(kk + 3) * ks + d]);
#pragma unroll
                for (int u = 0; u < 16; u++) {
                    const int j = min(j0 + u, nq - 1);
                    const float4 pj = *reinterpret_cast<const float4 *>(S + j * CK + kk);
                    acc[u] = fmaf(pj.x, v0, acc[u]);
                    acc[u] = fmaf(pj.y, v1, acc[u]);
                    acc[u] = fmaf(pj.z, v2, acc[u]);
                    acc[u] = fmaf(pj.w, v3, acc[u]);
                }
            }
#pragma unroll
            for (int u = 0; u < 16; u++) {
                const int j = j0 + u;
                if (j < nq) {
                    const int g = j / R, r = j % R;
                    part[(((int64_t)chunk * R + r) * a.heads + kvh * G + g) * (D + 2) + d] = acc[u];
                }
            }
        }
    }
}

// ---- MFMA path (F16 KV, head_dim 256, rope_dim 64, at most 32 query rows
// per kv head): scores and the value product run on v_mfma_f32_16x16x32_f16.
// K and V are exact in F16; query rows and probabilities are split into an
// F16 high part and an F16 remainder (two MFMAs), which keeps every product
// to ~2^-22 relative with FP32 accumulation.
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMD = 256;            // head dim
constexpr int kMK = 64;             // keys per workgroup
constexpr int kMQ = 32;             // query rows (two 16-row MFMA tiles)
constexpr int kAW = 8;              // waves of the MFMA kernel
constexpr int kVt = kMK + 8;        // halves per transposed V row (bank spread)
constexpr uint32_t kOffVt = 0;                              // [256][72] f16 (V transposed)
constexpr uint32_t kOffQh = kOffVt + kMD * kVt * 2;         // [32][256] f16, blocks XOR (row & 15)
constexpr uint32_t kOffQl = kOffQh + kMQ * kMD * 2;
constexpr uint32_t kOffS = kOffQl + kMQ * kMD * 2;          // [32][64] f32 scores, then P in place:
                                                            // [32][2: high, low][64] f16, blocks XOR (row & 7)
constexpr uint32_t kOffML = kOffS + kMQ * kMK * 4;         // [3][32] f32: running max, sum, rescale
constexpr uint32_t kMfmaLds = kOffML + 3 * kMQ * 4;         // 76 KB: two workgroups per CU

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xf, 0xf, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xf, 0xf, true);
    return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}
__device__ __forceinline__ float rl_f(float v, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); }
__device__ __forceinline__ double rl_dd(double v, int l) {
    const uint64_t b = __double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// wave-wide sum / max (DPP inside 16-lane rows, then the four row results)
__device__ __forceinline__ double wave_sum_dpp_d(double v) {
    v += dpp_d<0xb1>(v);
    v += dpp_d<0x4e>(v);
    v += dpp_d<0x124>(v);
    v += dpp_d<0x128>(v);
    return (rl_dd(v, 15) + rl_dd(v, 31)) + (rl_dd(v, 47) + rl_dd(v, 63));
}
__device__ __forceinline__ float wave_sum_dpp_f(float v) {
    v += dpp_f<0xb1>(v);
    v += dpp_f<0x4e>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x128>(v);
    return (rl_f(v, 15) + rl_f(v, 31)) + (rl_f(v, 47) + rl_f(v, 63));
}
__device__ __forceinline__ float wave_max_dpp_f(float v) {
    v = fmaxf(v, dpp_f<0xb1>(v));
    v = fmaxf(v, dpp_f<0x4e>(v));
    v = fmaxf(v, dpp_f<0x124>(v));
    v = fmaxf(v, dpp_f<0x128>(v));
    return fmaxf(fmaxf(rl_f(v, 15), rl_f(v, 31)), fmaxf(rl_f(v, 47), rl_f(v, 63)));
}

// Per-head RMSNorm and RoPE (rope_dim 64) of one 256-vector by one wave; lane
// l holds elements 4l .. 4l + 3, so rotation pair (i, i + 32) sits in lanes
// (l, l + 8) of the first DPP row and one row rotation exchanges them.
__device__ __forceinline__ void norm_rope4(const float *__restrict__ src, const float *__restrict__ w, float eps,
                                           const float2 *__restrict__ cs, float (&y)[4]) {
    const int lane = threadIdx.x & 63;
    const float4 x = *reinterpret_cast<const float4 *>(src + 4 * lane);
    const float4 w4 = *reinterpret_cast<const float4 *>(w + 4 * lane);
    double ss = (double)x.x * (double)x.x;
    ss += (double)x.y * (double)x.y;
    ss += (double)x.z * (double)x.z;
    ss += (double)x.w * (double)x.w;
    ss = wave_sum_dpp_d(ss);
    const float mean = (float)(ss / (double)kMD);
    const float scale = (float)(1.0 / sqrt((double)(mean + eps)));
    y[0] = __fmul_rn(x.x, __fmul_rn(scale, w4.x));
    y[1] = __fmul_rn(x.y, __fmul_rn(scale, w4.y));
    y[2] = __fmul_rn(x.z, __fmul_rn(scale, w4.z));
    y[3] = __fmul_rn(x.w, __fmul_rn(scale, w4.w));
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) pr[i] = dpp_f<0x128>(y[i]);  // partner lane (l + 8) % 16 of the row
    if (lane < 16) {
#pragma clang fp contract(off)  // float32 products and sums rounded separately, as the reference
        const bool first = lane < 8;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = 4 * lane + i, pi = first ? e : e - 32;
            const float c = cs[pi].x, sn = cs[pi].y;
            // first half: y0 c - y1 s; second half: y0 s + y1 c (y0 = element pi)
            y[i] = first ? y[i] * c - pr[i] * sn : pr[i] * sn + y[i] * c;
        }
    }
}

// norm_rope4 on operands already in registers: x = elements 4l .. 4l + 3,
// w4 the norm weights, cs the rotation pairs lane l < 16 uses.
__device__ __forceinline__ void norm_rope_regs(const float4 x, const float4 w4, float eps, const float2 (&cs)[4],
                                               float (&y)[4]) {
    const int lane = threadIdx.x & 63;
    double ss = (double)x.x * (double)x.x;
    ss += (double)x.y * (double)x.y;
    ss += (double)x.z * (double)x.z;
    ss += (double)x.w * (double)x.w;
    ss = wave_sum_dpp_d(ss);
    const float mean = (float)(ss / (double)kMD);
    const float scale = (float)(1.0 / sqrt((double)(mean + eps)));
    y[0] = __fmul_rn(x.x, __fmul_rn(scale, w4.x));
    y[1] = __fmul_rn(x.y, __fmul_rn(scale, w4.y));
    y[2] = __fmul_rn(x.z, __fmul_rn(scale, w4.z));
    y[3] = __fmul_rn(x.w, __fmul_rn(scale, w4.w));
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) pr[i] = dpp_f<0x128>(y[i]);  // partner lane (l + 8) % 16 of the row
    if (lane < 16) {
#pragma clang fp contract(off)  // float32 products and sums rounded separately, as the reference
        const bool first = lane < 8;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float c = cs[i].x, sn = cs[i].y;
            y[i] = first ? y[i] * c - pr[i] * sn : pr[i] * sn + y[i] * c;
        }
    }
}

__device__ __forceinline__ uint32_t pack_h2(_Float16 a, _Float16 b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// 16-byte global -> LDS copy of one lane (lane l writes [m0 + 16 l, +16)),
// issued as inline assembly so the compiler does not wait on it (the kernel
// waits with s_waitcnt vmcnt(0) before its first barrier).
__device__ __forceinline__ void lds_copy16_at(const void *src, uint32_t m0) {
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}

__device__ __forceinline__ void lds_only_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One workgroup per (64-key chunk, KV head, request): launches of at most
// ~1024 chunk workgroups (short contexts). The chunk's keys and values load
// while the queries are prepared; the verify rows walk the LDS-resident
// chunk in blocks of kMQ / G rows.
__global__ __launch_bounds__(64 * kAW) __attribute__((amdgpu_waves_per_eu(4))) void attn_verify_mfma_kernel(const float *__restrict__ q, const float *__restrict__ k,
                                                               const float *__restrict__ v, uint16_t *kpool,
                                                               uint16_t *vpool, const int32_t *__restrict__ table,
                                                               const float *__restrict__ q_norm,
                                                               const float *__restrict__ k_norm,
                                                               const float2 *__restrict__ rope, AttnVArgs a,
                                                               float *__restrict__ part, ModelDyn dyn) {
    extern __shared__ __align__(16) uint8_t lds[];
    YK_ATTN_REQUEST(kMK);
    const int kvh = blockIdx.y, chunk = blockIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int r16 = lane & 15, g4 = lane >> 4;
    const int R = a.rows;
    const int G = a.heads / a.kv_heads;
    const int p0 = cur_pos_a(dyn) + a.displacement;  // position of verify row 0
    const int last = p0 + R - 1;
    const int key0 = chunk * kMK;
    if (key0 > last) return;  // no row sees this chunk; the merge skips it
    const int half = a.rope_dim / 2;
    const int qstride = a.gated ? 2 * kMD : kMD;

    // ---- cached keys straight into MFMA B order: the scores lane (key kk,
    //      group g4) holds dims [32 ks + 8 g4, +8) of key kk for every ks.
    //      Keys at or past p0 (this step's rows) are read after they are
    //      written below.
    const int kk_s = (wave & 3) * 16 + r16;
    const bool scorer = 16 * (wave >> 2) < G * min(kMQ / G, R);  // row tile of this wave in use
    half8 kreg[kMD / 32];
    auto load_keys = [&](bool fresh) __attribute__((always_inline)) {
        const int p = key0 + kk_s;
        const bool want = scorer && (fresh ? (p >= p0 && p <= last) : p < p0);
        if (want) {
            const int64_t slot = (int64_t)table[p / a.block_size] * a.block_size + p % a.block_size;
            const half8 *src = reinterpret_cast<const half8 *>(kpool + slot * a.kv_dim + (int64_t)kvh * kMD + g4 * 8);
#pragma unroll
            for (int ks = 0; ks < kMD / 32; ks++) kreg[ks] = src[4 * ks];
        } else if (!fresh) {
#pragma unroll
            for (int ks = 0; ks < kMD / 32; ks++) kreg[ks] = half8{};
        }
    };
    load_keys(false);
    // ---- cached values: wave w loads dims [32w, 32w + 32) of every key
    //      (lane = key) and stores them transposed
    constexpr int kVE = kMD / kAW / 8;  // 16-byte pieces per lane
    uint4 vreg[kVE];
    const int vkey = lane, vp = key0 + vkey;
    {
        if (vp < p0) {
            const int64_t slot = (int64_t)table[vp / a.block_size] * a.block_size + vp % a.block_size;
            const uint4 *src =
                reinterpret_cast<const uint4 *>(vpool + slot * a.kv_dim + (int64_t)kvh * kMD + wave * (kMD / kAW));
#pragma unroll
            for (int e = 0; e < kVE; e++) vreg[e] = src[e];
        } else {
#pragma unroll
            for (int e = 0; e < kVE; e++) vreg[e] = make_uint4(0, 0, 0, 0);
        }
    }
    // ---- query rows in blocks of RB verify rows (G * RB <= kMQ MFMA rows):
    //      normalised, rotated, split into F16 high + remainder. A wave's
    //      rows are loaded first, then computed (no load waits in the loop).
    const int RB = kMQ / G;
    auto prep_q = [&](int r0, int Rb) __attribute__((always_inline)) {
        int oz;  // opaque zero: keeps the per-vector offsets below from being hoisted and spilled
        asm volatile("s_mov_b32 %0, 0" : "=s"(oz));
        const int plane = lane + oz;
        constexpr int kQV = kMQ / kAW;
        const int nqb = G * Rb;
        const float4 w4 = *reinterpret_cast<const float4 *>(q_norm + 4 * plane);
        float4 xq[kQV];
#pragma unroll
        for (int t = 0; t < kQV; t++) {
            const int vec = wave + kAW * t;
            if (vec < nqb) {
                const int gq = vec / Rb, r = r0 + vec % Rb;
                xq[t] = *reinterpret_cast<const float4 *>(q + ((int64_t)r * a.heads + kvh * G + gq) * qstride + 4 * plane);
            }
        }
#pragma unroll
        for (int t = 0; t < kQV; t++) {
            const int vec = wave + kAW * t;
            if (vec >= nqb) break;
            const int r = r0 + vec % Rb;
            float2 cq[4] = {};
            if (plane < 16) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int e = 4 * plane + i;
                    cq[i] = rope[r * half + (plane < 8 ? e : e - 32)];
                }
            }
            float y[4];
            norm_rope_regs(xq[t], w4, a.eps, cq, y);
            _Float16 hi[4], lo[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                hi[i] = (_Float16)y[i];
                lo[i] = (_Float16)(y[i] - (float)hi[i]);
            }
            const uint32_t off = (uint32_t)vec * kMD * 2 + (uint32_t)(((plane >> 1) ^ (vec & 15)) * 16 + (plane & 1) * 8);
            *reinterpret_cast<uint2 *>(lds + kOffQh + off) = make_uint2(pack_h2(hi[0], hi[1]), pack_h2(hi[2], hi[3]));
            *reinterpret_cast<uint2 *>(lds + kOffQl + off) = make_uint2(pack_h2(lo[0], lo[1]), pack_h2(lo[2], lo[3]));
        }
    };
    // ---- values of this chunk, transposed (keys past the verify rows: zero)
    {
        uint16_t *vt = reinterpret_cast<uint16_t *>(lds + kOffVt);
        if (vp < p0 || vp > last) {
#pragma unroll
            for (int e = 0; e < kVE; e++) {
                const uint32_t w4[4] = {vreg[e].x, vreg[e].y, vreg[e].z, vreg[e].w};
#pragma unroll
                for (int i = 0; i < 8; i++)
                    vt[(wave * (kMD / kAW) + e * 8 + i) * kVt + vkey] = (uint16_t)(w4[i >> 1] >> (16 * (i & 1)));
            }
        }
    }
    prep_q(0, min(RB, R));
    // ---- the verify rows' own keys and values (rows whose position falls in
    //      this chunk): rounded as the pool stores them, into the pool (keys)
    //      and LDS (values)
    for (int r = wave; r < R; r += kAW) {
        const int p = p0 + r;
        if (p < key0 || p >= key0 + kMK) continue;
        const int kk = p - key0;
        const int64_t slot = (int64_t)table[p / a.block_size] * a.block_size + p % a.block_size;
        float y[4];
        norm_rope4(k + (int64_t)r * a.kv_dim + (int64_t)kvh * kMD, k_norm, a.eps, rope + r * half, y);
        uint16_t kq[4], vq[4];
        const float4 vv = *reinterpret_cast<const float4 *>(v + (int64_t)r * a.kv_dim + (int64_t)kvh * kMD + 4 * lane);
        const float vf[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            kq[i] = ref_f32_to_f16(y[i]);
            vq[i] = ref_f32_to_f16(vf[i]);
        }
        const uint2 kw = make_uint2((uint32_t)kq[0] | ((uint32_t)kq[1] << 16), (uint32_t)kq[2] | ((uint32_t)kq[3] << 16));
        const uint2 vw = make_uint2((uint32_t)vq[0] | ((uint32_t)vq[1] << 16), (uint32_t)vq[2] | ((uint32_t)vq[3] << 16));
        *reinterpret_cast<uint2 *>(kpool + slot * a.kv_dim + (int64_t)kvh * kMD + 4 * lane) = kw;
        *reinterpret_cast<uint2 *>(vpool + slot * a.kv_dim + (int64_t)kvh * kMD + 4 * lane) = vw;
        uint16_t *vt = reinterpret_cast<uint16_t *>(lds + kOffVt);
#pragma unroll
        for (int i = 0; i < 4; i++) vt[(4 * lane + i) * kVt + kk] = vq[i];
    }
    if (key0 + kMK - 1 >= p0) {
        __syncthreads();  // the new keys are in the pool (global and LDS fence)
        load_keys(true);
    } else {
        lds_only_barrier();
    }

    for (int r0 = 0; r0 < R; r0 += RB) {
    const int Rb = min(RB, R - r0), nq = G * Rb;  // this block's verify rows and MFMA rows
    if (r0) {  // every wave is past the previous block's scores and softmax
        lds_only_barrier();
        prep_q(r0, Rb);
        lds_only_barrier();
    }
    // ---- scores: wave w owns keys [16 (w & 3), +16) of row tile w >> 2
    if (16 * (wave >> 2) < nq) {
        const int rt = wave >> 2;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const int kk = (wave & 3) * 16 + r16;
#pragma unroll
        for (int ks = 0; ks < kMD / 32; ks++) {
            const int blk = ks * 4 + g4;
            const half8 b = kreg[ks];
            const uint32_t qo = (uint32_t)(rt * 16 + r16) * kMD * 2 + (uint32_t)((blk ^ r16) * 16);
            const half8 ah = *reinterpret_cast<const half8 *>(lds + kOffQh + qo);
            const half8 al = *reinterpret_cast<const half8 *>(lds + kOffQl + qo);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, b, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, b, acc, 0, 0, 0);
        }
        float *S = reinterpret_cast<float *>(lds + kOffS);
        const int p = key0 + kk;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int qi = rt * 16 + g4 * 4 + e;
            if (qi < nq) S[qi * kMK + kk] = p <= p0 + r0 + qi % Rb ? acc[e] * a.scale : -INFINITY;
        }
    }
    lds_only_barrier();
    // ---- softmax partials: four query rows per wave at a time, one 16-lane
    //      DPP row per query row, lane s holding keys [4 s, 4 s + 4)
    {
        const float *S = reinterpret_cast<const float *>(lds + kOffS);
        const int sub = lane >> 4, s16 = lane & 15;
        for (int q0 = 4 * wave; q0 < nq; q0 += 4 * kAW) {
            const int qi = q0 + sub;
            const bool live = qi < nq;
            const int qc = live ? qi : q0;
            const float4 sv = *reinterpret_cast<const float4 *>(S + qc * kMK + 4 * s16);
            const float sc[4] = {sv.x, sv.y, sv.z, sv.w};
            float m = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
            m = fmaxf(m, dpp_f<0xb1>(m));
            m = fmaxf(m, dpp_f<0x4e>(m));
            m = fmaxf(m, dpp_f<0x124>(m));
            m = fmaxf(m, dpp_f<0x128>(m));
            float e[4];
#pragma unroll
            for (int i = 0; i < 4; i++) e[i] = (sc[i] == -INFINITY) ? 0.0f : exp_nonpos(sc[i] - m);
            float l = (e[0] + e[1]) + (e[2] + e[3]);
            l += dpp_f<0xb1>(l);
            l += dpp_f<0x4e>(l);
            l += dpp_f<0x124>(l);
            l += dpp_f<0x128>(l);
            _Float16 hi[4], lo[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                hi[i] = (_Float16)e[i];
                lo[i] = (_Float16)(e[i] - (float)hi[i]);
            }
            if (live) {
                // P replaces the row's scores: high halves in bytes [0, 128), low in [128, 256);
                // keys 4 s16 .. + 3 sit in one 8-key block
                const int key = 4 * s16;
                const uint32_t off = (uint32_t)qi * kMK * 4 + (uint32_t)((((key >> 3) ^ (qi & 7)) * 16) + (key & 7) * 2);
                *reinterpret_cast<uint2 *>(lds + kOffS + off) = make_uint2(pack_h2(hi[0], hi[1]), pack_h2(hi[2], hi[3]));
                *reinterpret_cast<uint2 *>(lds + kOffS + kMK * 2 + off) =
                    make_uint2(pack_h2(lo[0], lo[1]), pack_h2(lo[2], lo[3]));
                if (s16 == 0) {
                    const int gq = qi / Rb, r = r0 + qi % Rb;
                    float *rec = part + (((int64_t)chunk * R + r) * a.heads + kvh * G + gq) * (kMD + 2);
                    rec[kMD] = m;
                    rec[kMD + 1] = l;
                }
            }
        }
    }
    lds_only_barrier();
    // ---- value product: wave w owns dims [32w, 32w + 32) (two 16-wide tiles)
    {
        constexpr int kJ = kMD / kAW / 16;
        f32x4 o[kJ][2];
#pragma unroll
        for (int j = 0; j < kJ; j++)
#pragma unroll
            for (int rt = 0; rt < 2; rt++) o[j][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
        const bool two = nq > 16;
#pragma unroll
        for (int ks = 0; ks < kMK / 32; ks++) {
            const int blk = ks * 4 + g4;
            half8 ah[2], al[2];
#pragma unroll
            for (int rt = 0; rt < 2; rt++) {
                const uint32_t po = (uint32_t)(rt * 16 + r16) * kMK * 4 + (uint32_t)((blk ^ (r16 & 7)) * 16);
                ah[rt] = *reinterpret_cast<const half8 *>(lds + kOffS + po);
                al[rt] = *reinterpret_cast<const half8 *>(lds + kOffS + kMK * 2 + po);
            }
#pragma unroll
            for (int j = 0; j < kJ; j++) {
                const int dcol = wave * (kMD / kAW) + j * 16 + r16;
                const half8 b = *reinterpret_cast<const half8 *>(lds + kOffVt + (uint32_t)dcol * kVt * 2 + (uint32_t)(ks * 32 + g4 * 8) * 2);
                o[j][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[0], b, o[j][0], 0, 0, 0);
                o[j][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[0], b, o[j][0], 0, 0, 0);
                if (two) {
                    o[j][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[1], b, o[j][1], 0, 0, 0);
                    o[j][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[1], b, o[j][1], 0, 0, 0);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < kJ; j++)
#pragma unroll
            for (int rt = 0; rt < 2; rt++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int qi = rt * 16 + g4 * 4 + e;
                    if (qi < nq) {
                        const int gq = qi / Rb, r = r0 + qi % Rb, d = wave * (kMD / kAW) + j * 16 + r16;
                        part[(((int64_t)chunk * R + r) * a.heads + kvh * G + gq) * (kMD + 2) + d] = o[j][rt][e];
                    }
                }
    }
    }
}

// LDS layout of the grouped kernel with NT 16-row query tiles: the
// transposed V chunk, the query tiles (F16 high, remainder), the scores /
// probabilities and the running (max, sum, rescale) of every query row.
// Page-table entries of a group's keys held in LDS by the PF kernels
// (three to six tiles; the launcher caps the group so that they fit).
constexpr int kPtCap = 256;
template <int NT> struct GroupLds {
    static constexpr int kQ = 16 * NT;
    static constexpr uint32_t Vt = 0;
    static constexpr uint32_t Qh = Vt + kMD * kVt * 2;
    static constexpr uint32_t Ql = Qh + kQ * kMD * 2;
    static constexpr uint32_t S = Ql + kQ * kMD * 2;
    static constexpr uint32_t ML = S + kQ * kMK * 4;
    static constexpr uint32_t PT = ML + 3 * kQ * 4;
    static constexpr uint32_t total = PT + (NT > 2 ? kPtCap * 4 : 0);
};
static_assert(GroupLds<2>::total == kMfmaLds, "two-tile layout");
static_assert(GroupLds<6>::total <= 160 * 1024, "six-tile layout fits LDS");
static_assert(GroupLds<5>::total <= 160 * 1024 && GroupLds<3>::total <= 160 * 1024, "PF layouts fit LDS");

// One workgroup per (group of `cpw` 64-key chunks, KV head, request). The
// verify rows' own keys and values in the group's range go to the pool
// first; then, per block of 16 NT / G verify rows, the group's chunks are
// walked in order with an online softmax (running max m, sum l and the
// rescale of the P.V accumulators in registers). One partial record
// (o, m, l) per (group, row, head) for the merge.
// NT = 2: 76 KB of LDS and at most 128 VGPRs, two workgroups per CU.
// NT = 3, 5, 6 (PF): 48, 80 or 96 MFMA rows in one block (config 3's 36
// rows of 4 heads x 9 verify rows, config 4's 68 of 4 x 17, so each chunk
// is read once per step), 99 / 137 / 157 KB of LDS and one workgroup per
// CU; with the register budget of two waves per SIMD the next chunk's keys
// and values load into a second register set while the current chunk is
// computed.
template <int NT, bool PF>
__global__ __launch_bounds__(64 * kAW) __attribute__((amdgpu_waves_per_eu(NT > 2 ? 2 : 4))) void attn_verify_mfma_group_kernel(
    const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ v, uint16_t *kpool,
    uint16_t *vpool, const int32_t *__restrict__ table, const float *__restrict__ q_norm,
    const float *__restrict__ k_norm, const float2 *__restrict__ rope, AttnVArgs a, float *__restrict__ part,
    ModelDyn dyn, int cpw) {
    extern __shared__ __align__(16) uint8_t lds[];
    YK_ATTN_REQUEST(kMK * cpw);
    const int kvh = blockIdx.y, grp = blockIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int r16 = lane & 15, g4 = lane >> 4;
    const int R = a.rows;
    const int G = a.heads / a.kv_heads;
    const int p0 = cur_pos_a(dyn) + a.displacement;  // position of verify row 0
    const int last = p0 + R - 1;
    const int c_lo = grp * cpw;
    if (c_lo * kMK > last) return;  // no row sees this group; the merge skips it
    const int c_hi = min(c_lo + cpw, last / kMK + 1);
    const int half = a.rope_dim / 2;
    const int qstride = a.gated ? 2 * kMD : kMD;
    using LY = GroupLds<NT>;
    constexpr int kQ = LY::kQ;
    float *Mrow = reinterpret_cast<float *>(lds + LY::ML);  // running max per MFMA row
    float *Lrow = Mrow + kQ;                                // running sum
    float *Arow = Lrow + kQ;                                // this chunk's rescale of the accumulators

    // ---- the verify rows' own keys and values (rows whose position falls in
    //      this group): rounded as the pool stores them, into the pool
    for (int r = wave; r < R; r += kAW) {
        const int p = p0 + r;
        if (p < c_lo * kMK || p >= c_hi * kMK) continue;
        const int64_t slot = (int64_t)table[p / a.block_size] * a.block_size + p % a.block_size;
        float y[4];
        norm_rope4(k + (int64_t)r * a.kv_dim + (int64_t)kvh * kMD, k_norm, a.eps, rope + r * half, y);
        uint16_t kq[4], vq[4];
        const float4 vv = *reinterpret_cast<const float4 *>(v + (int64_t)r * a.kv_dim + (int64_t)kvh * kMD + 4 * lane);
        const float vf[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            kq[i] = ref_f32_to_f16(y[i]);
            vq[i] = ref_f32_to_f16(vf[i]);
        }
        const uint2 kw = make_uint2((uint32_t)kq[0] | ((uint32_t)kq[1] << 16), (uint32_t)kq[2] | ((uint32_t)kq[3] << 16));
        const uint2 vw = make_uint2((uint32_t)vq[0] | ((uint32_t)vq[1] << 16), (uint32_t)vq[2] | ((uint32_t)vq[3] << 16));
        *reinterpret_cast<uint2 *>(kpool + slot * a.kv_dim + (int64_t)kvh * kMD + 4 * lane) = kw;
        *reinterpret_cast<uint2 *>(vpool + slot * a.kv_dim + (int64_t)kvh * kMD + 4 * lane) = vw;
    }
    if (p0 < c_hi * kMK) __syncthreads();  // the new rows are in the pool (global fence)

    // keys straight into MFMA B order: the scores lane (key kk, group g4)
    // holds dims [32 ks + 8 g4, +8) of key kk for every ks
    const int kk_s = (wave & 3) * 16 + r16;
    constexpr int kVE = kMD / kAW / 8;                          // 16-byte V pieces per lane
    static_assert(kVE == 4, "four value pieces per lane: two keys x two 8-dim blocks");
    constexpr int kJ = kMD / kAW / 16;                          // 16-wide output tiles per wave
    const int RB = kQ / G;
    // ---- query rows of one block: normalised, rotated, split into F16 high +
    //      remainder. A wave's rows are loaded first, then computed.
    auto prep_q = [&](int r0, int Rb) __attribute__((always_inline)) {
        int oz;  // opaque zero: keeps the per-vector offsets below from being hoisted and spilled
        asm volatile("s_mov_b32 %0, 0" : "=s"(oz));
        const int plane = lane + oz;
        constexpr int kQV = kQ / kAW;
        const int nqb = G * Rb;
        const float4 w4 = *reinterpret_cast<const float4 *>(q_norm + 4 * plane);
        float4 xq[kQV];
#pragma unroll
        for (int t = 0; t < kQV; t++) {
            const int vec = wave + kAW * t;
            if (vec < nqb) {
                const int gq = vec / Rb, r = r0 + vec % Rb;
                xq[t] = *reinterpret_cast<const float4 *>(q + ((int64_t)r * a.heads + kvh * G + gq) * qstride + 4 * plane);
            }
        }
#pragma unroll
        for (int t = 0; t < kQV; t++) {
            const int vec = wave + kAW * t;
            if (vec >= nqb) break;
            const int r = r0 + vec % Rb;
            float2 cq[4] = {};
            if (plane < 16) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int e = 4 * plane + i;
                    cq[i] = rope[r * half + (plane < 8 ? e : e - 32)];
                }
            }
            float y[4];
            norm_rope_regs(xq[t], w4, a.eps, cq, y);
            _Float16 hi[4], lo[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                hi[i] = (_Float16)y[i];
                lo[i] = (_Float16)(y[i] - (float)hi[i]);
            }
            // [tile][dims / 32][group of 8 dims][row of the tile][8 FP16]
            const uint32_t off = (uint32_t)(vec >> 4) * 8192 + (uint32_t)(plane >> 3) * 1024 +
                                 (uint32_t)((plane >> 1) & 3) * 256 + (uint32_t)(vec & 15) * 16 + (uint32_t)(plane & 1) * 8;
            *reinterpret_cast<uint2 *>(lds + LY::Qh + off) = make_uint2(pack_h2(hi[0], hi[1]), pack_h2(hi[2], hi[3]));
            *reinterpret_cast<uint2 *>(lds + LY::Ql + off) = make_uint2(pack_h2(lo[0], lo[1]), pack_h2(lo[2], lo[3]));
        }
    };

    // keys (scorer waves) and values (wave w: dims [32w, +32) of key `plane`)
    // of chunk ci, from positions clamped to the last verify row: keys past
    // it are masked out of the scores, and their values get probability 0
    struct KvRegs {
        half8 k[kMD / 32];
        uint4 v[kVE];
    };
    // Page-table entries of this lane's key (scores) and value row of chunk
    // ci, then the chunk's loads from them. The entries are requested one
    // chunk ahead of the loads that use them: waiting for them then also
    // waits only for loads that are due anyway.
    struct Pages {
        int32_t k, v0, v1;
    };
    // PF: the group's page-table entries sit in LDS (loaded once below), so
    // waiting for an entry never waits for the vector loads issued before it
    // PF (six tiles): the launcher only takes power-of-two page sizes, so
    // page and slot of a position are a shift and a mask
    const int bsh = PF ? __builtin_ctz((unsigned)a.block_size) : 0, bsm = a.block_size - 1;
    auto page_of = [&](int pos) __attribute__((always_inline)) { return PF ? pos >> bsh : pos / a.block_size; };
    auto slot_in = [&](int pos) __attribute__((always_inline)) { return PF ? pos & bsm : pos % a.block_size; };
    const int pg0 = page_of(c_lo * kMK);
    if constexpr (PF) {
        int *pt = reinterpret_cast<int *>(lds + LY::PT);
        const int pg1 = page_of(min(c_hi * kMK - 1, last));
        for (int i = (int)threadIdx.x; i <= pg1 - pg0; i += (int)blockDim.x) pt[i] = table[pg0 + i];
        __syncthreads();
    }
    auto fetch_pages = [&](Pages &P, int ci) __attribute__((always_inline)) {
        const int key0 = ci * kMK;
        if constexpr (PF) {
            const int *pt = reinterpret_cast<const int *>(lds + LY::PT);
            P.k = pt[page_of(min(key0 + kk_s, last)) - pg0];
            P.v0 = pt[page_of(min(key0 + (lane & 31), last)) - pg0];
            P.v1 = pt[page_of(min(key0 + 32 + (lane & 31), last)) - pg0];
            return;
        }
        P.k = table[page_of(min(key0 + kk_s, last))];
        P.v0 = table[page_of(min(key0 + (lane & 31), last))];
        P.v1 = table[page_of(min(key0 + 32 + (lane & 31), last))];
    };
    auto load_kv = [&](KvRegs &X, const Pages &P, int ci) __attribute__((always_inline)) {
        const int key0 = ci * kMK;
        const int p = min(key0 + kk_s, last);
        const int64_t ks_ = (int64_t)P.k * a.block_size + slot_in(p);
        const half8 *ksrc = reinterpret_cast<const half8 *>(kpool + ks_ * a.kv_dim + (int64_t)kvh * kMD + g4 * 8);
#pragma unroll
        for (int ks = 0; ks < kMD / 32; ks++) X.k[ks] = ksrc[4 * ks];
        // values: piece e of the lane is key 32 (e & 1) + lane % 32, dims
        // [32 wave + 8 b, +8) with b = 2 (e >> 1) + lane / 32 — 32 keys x 32
        // bytes per load instruction
        const int vp0 = min(key0 + (lane & 31), last), vp1 = min(key0 + 32 + (lane & 31), last);
        const int64_t vcol = (int64_t)kvh * kMD + wave * (kMD / kAW) + (lane >> 5) * 8;
        const uint4 *v0 = reinterpret_cast<const uint4 *>(vpool + ((int64_t)P.v0 * a.block_size + slot_in(vp0)) * a.kv_dim + vcol);
        const uint4 *v1 = reinterpret_cast<const uint4 *>(vpool + ((int64_t)P.v1 * a.block_size + slot_in(vp1)) * a.kv_dim + vcol);
        X.v[0] = v0[0];
        X.v[1] = v1[0];
        X.v[2] = v0[2];
        X.v[3] = v1[2];
    };

    for (int r0 = 0; r0 < R; r0 += RB) {
        const int Rb = min(RB, R - r0), nq = G * Rb;  // this block's verify rows and MFMA rows
        const int ntl = (nq + 15) / 16;               // row tiles in use
        if (r0) lds_only_barrier();                   // the previous block's reads of Q, M, L are done
        prep_q(r0, Rb);
        if (threadIdx.x < kQ) {
            Mrow[threadIdx.x] = -INFINITY;
            Lrow[threadIdx.x] = 0.0f;
            Arow[threadIdx.x] = 1.0f;  // rows past the block's own keep their (unused) accumulators
        }
        f32x4 o[kJ][NT];
#pragma unroll
        for (int j = 0; j < kJ; j++)
#pragma unroll
            for (int rt = 0; rt < NT; rt++) o[j][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
        // one chunk of the group from the registers X
        auto chunk = [&](const KvRegs &X, int ci, auto &&mid) __attribute__((always_inline)) {
            const int key0 = ci * kMK;
            // Lane constants re-derived per chunk from an opaque zero: hoisted
            // out of the chunk loop, the per-tile offsets they feed would be
            // spilled for the whole loop.
            int oz;
            asm volatile("s_mov_b32 %0, 0" : "=s"(oz));
            const int lr16 = r16 + oz, lg4 = g4 + oz, lkk = kk_s + oz, llane = lane + oz;
            lds_only_barrier();  // the previous chunk's P.V reads of Vt are done; Q, M, L are written
            {
                uint16_t *vt = reinterpret_cast<uint16_t *>(lds + LY::Vt);
#pragma unroll
                for (int e = 0; e < kVE; e++) {
                    const uint4 vv = X.v[e];  // past the last key: the last key's (finite, probability 0)
                    const uint32_t w4[4] = {vv.x, vv.y, vv.z, vv.w};
                    const int key = (e & 1) * 32 + (llane & 31), d0 = wave * (kMD / kAW) + (2 * (e >> 1) + (llane >> 5)) * 8;
                    // lanes 32..63 write 8 dims further: 32 banks away (kVt = 72)
#pragma unroll
                    for (int i = 0; i < 8; i++) vt[(d0 + i) * kVt + key] = (uint16_t)(w4[i >> 1] >> (16 * (i & 1)));
                }
            }
            // ---- scores: wave w owns keys [16 (w & 3), +16) of row tiles
            //      w >> 2, (w >> 2) + 2, ... Every row of a tile is stored (rows
            //      past the block's own are never read); the causal mask is the
            //      softmax's. With every tile in use (one block of rows, the
            //      usual case) the tiles run without a branch between them, so
            //      their LDS reads can be issued ahead of the MFMAs.
            auto score_tile = [&](int rt) __attribute__((always_inline)) {
                // A operands at lane base + immediates; two accumulators so
                // that consecutive MFMAs do not wait for each other
                const uint8_t *qa = lds + LY::Qh + (uint32_t)rt * 8192 + (uint32_t)lg4 * 256 + (uint32_t)lr16 * 16;
                f32x4 acc = {0.f, 0.f, 0.f, 0.f}, acc2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < kMD / 32; ks++) {
                    const half8 ah = *reinterpret_cast<const half8 *>(qa + ks * 1024);
                    const half8 al = *reinterpret_cast<const half8 *>(qa + (LY::Ql - LY::Qh) + ks * 1024);
                    // keys past the last are the last key again (clamped loads):
                    // finite, and masked by the softmax
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, X.k[ks], acc, 0, 0, 0);
                    acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, X.k[ks], acc2, 0, 0, 0);
                }
                acc += acc2;
                float *S = reinterpret_cast<float *>(lds + LY::S) + (rt * 16 + lg4 * 4) * kMK + lkk;
#pragma unroll
                for (int e = 0; e < 4; e++) S[e * kMK] = acc[e] * a.scale;
            };
            const bool odd = (wave >> 2) != 0;
            if (ntl == NT) {
                if (odd) {
#pragma unroll
                    for (int rt = 1; rt < NT; rt += 2) score_tile(rt);
                } else {
#pragma unroll
                    for (int rt = 0; rt < NT; rt += 2) score_tile(rt);
                }
            } else {
#pragma unroll
                for (int rt = 0; rt < NT; rt++)
                    if (rt % 2 == (int)odd && rt < ntl) score_tile(rt);
            }
            lds_only_barrier();
            mid();  // the next chunk's loads, issued while the waves are spread over the chunk
            // ---- online softmax: four query rows per wave at a time, one
            //      16-lane DPP row per query row, lane s holding keys
            //      [4 s, 4 s + 4) (the row's reductions never leave the DPP
            //      row, and the four exponentials of a lane overlap)
            {
                const float *S = reinterpret_cast<const float *>(lds + LY::S);
                const int sub = llane >> 4, s16 = llane & 15;
                for (int q0 = 4 * wave; q0 < nq; q0 += 4 * kAW) {
                    const int qi = q0 + sub;
                    const bool live = qi < nq;
                    const int qc = live ? qi : q0;
                    const float4 sv = *reinterpret_cast<const float4 *>(S + qc * kMK + 4 * s16);
                    float sc[4] = {sv.x, sv.y, sv.z, sv.w};
                    if (key0 + kMK - 1 > p0 + r0) {  // the chunk reaches the block's rows: causal mask
                        const int rowpos = p0 + r0 + qc % Rb;
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            if (key0 + 4 * s16 + i > rowpos) sc[i] = -INFINITY;
                    }
                    float mc = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
                    mc = fmaxf(mc, dpp_f<0xb1>(mc));
                    mc = fmaxf(mc, dpp_f<0x4e>(mc));
                    mc = fmaxf(mc, dpp_f<0x124>(mc));
                    mc = fmaxf(mc, dpp_f<0x128>(mc));
                    const float m_old = Mrow[qc];
                    const float m_new = fmaxf(m_old, mc);
                    float e[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                    float alpha = 1.0f;
                    if (m_new != -INFINITY) {
#pragma unroll
                        for (int i = 0; i < 4; i++) e[i] = (sc[i] == -INFINITY) ? 0.0f : exp_nonpos(sc[i] - m_new);
                        alpha = m_old == -INFINITY ? 0.0f : exp_nonpos(m_old - m_new);
                    }
                    float lc = (e[0] + e[1]) + (e[2] + e[3]);
                    lc += dpp_f<0xb1>(lc);
                    lc += dpp_f<0x4e>(lc);
                    lc += dpp_f<0x124>(lc);
                    lc += dpp_f<0x128>(lc);
                    _Float16 hi[4], lo[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        hi[i] = (_Float16)e[i];
                        lo[i] = (_Float16)(e[i] - (float)hi[i]);
                    }
                    if (live) {
                        // P replaces the row's scores: high halves in bytes [0, 128), low in
                        // [128, 256); keys 4 s16 .. + 3 sit in one 8-key block
                        const int key = 4 * s16;
                        const uint32_t off = (uint32_t)qi * kMK * 4 + (uint32_t)((((key >> 3) ^ (qi & 7)) * 16) + (key & 7) * 2);
                        *reinterpret_cast<uint2 *>(lds + LY::S + off) = make_uint2(pack_h2(hi[0], hi[1]), pack_h2(hi[2], hi[3]));
                        *reinterpret_cast<uint2 *>(lds + LY::S + kMK * 2 + off) =
                            make_uint2(pack_h2(lo[0], lo[1]), pack_h2(lo[2], lo[3]));
                        if (s16 == 0) {
                            Lrow[qi] = Lrow[qi] * alpha + lc;
                            Mrow[qi] = m_new;
                            Arow[qi] = alpha;
                        }
                    }
                }
            }
            lds_only_barrier();
            // ---- value product: wave w owns dims [32w, 32w + 32). This
            //      wave's V operands for both key halves, then one row tile at
            //      a time: its accumulators rescaled by this chunk's alpha, then
            //      its probabilities (2 x kJ x 2 MFMAs). Without a branch between
            //      the tiles when every tile is in use.
            half8 vb[kMK / 32][kJ];
#pragma unroll
            for (int ks = 0; ks < kMK / 32; ks++)
#pragma unroll
                for (int j = 0; j < kJ; j++) {
                    const int dcol = wave * (kMD / kAW) + j * 16 + lr16;
                    vb[ks][j] = *reinterpret_cast<const half8 *>(lds + LY::Vt + (uint32_t)dcol * kVt * 2 +
                                                                 (uint32_t)(ks * 32 + lg4 * 8) * 2);
                }
            auto pv_tile = [&](int rt) __attribute__((always_inline)) {
                const float4 al = *reinterpret_cast<const float4 *>(Arow + rt * 16 + lg4 * 4);
#pragma unroll
                for (int j = 0; j < kJ; j++) {
                    o[j][rt][0] *= al.x;
                    o[j][rt][1] *= al.y;
                    o[j][rt][2] *= al.z;
                    o[j][rt][3] *= al.w;
                }
#pragma unroll
                for (int ks = 0; ks < kMK / 32; ks++) {
                    const int blk = ks * 4 + lg4;
                    const uint32_t po = (uint32_t)(rt * 16 + lr16) * kMK * 4 + (uint32_t)((blk ^ (lr16 & 7)) * 16);
                    const half8 ah = *reinterpret_cast<const half8 *>(lds + LY::S + po);
                    const half8 al = *reinterpret_cast<const half8 *>(lds + LY::S + kMK * 2 + po);
#pragma unroll
                    for (int j = 0; j < kJ; j++) {
                        o[j][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, vb[ks][j], o[j][rt], 0, 0, 0);
                        o[j][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, vb[ks][j], o[j][rt], 0, 0, 0);
                    }
                }
            };
            if (ntl == NT) {
#pragma unroll
                for (int rt = 0; rt < NT; rt++) pv_tile(rt);
            } else {
#pragma unroll
                for (int rt = 0; rt < NT; rt++)
                    if (rt < ntl) pv_tile(rt);
            }
        };
        if constexpr (PF) {
            // two register sets: chunk ci + 1 loads while chunk ci is computed,
            // and the page entries of chunk ci + 2 are requested meanwhile.
            // The loads go out after chunk ci's scores, when the waves are
            // spread over the chunk (issued together at the chunk's start,
            // the eight waves' loads queue behind each other: config 3 100
            // -> 91 us per layer).
            // Every load is issued unconditionally (indices clamped to the last
            // chunk): under a branch the compiler's wait counts merge
            // conservatively and the current chunk would wait for the next
            // one's loads.
            KvRegs XA, XB;
            Pages PA, PB;
            fetch_pages(PA, c_lo);
            load_kv(XA, PA, c_lo);
            fetch_pages(PB, min(c_lo + 1, c_hi - 1));
            for (int ci = c_lo; ci < c_hi; ci += 2) {
                chunk(XA, ci, [&]() __attribute__((always_inline)) {
                    load_kv(XB, PB, min(ci + 1, c_hi - 1));
                    fetch_pages(PA, min(ci + 2, c_hi - 1));
                });
                if (ci + 1 >= c_hi) break;
                chunk(XB, ci + 1, [&]() __attribute__((always_inline)) {
                    load_kv(XA, PA, min(ci + 2, c_hi - 1));
                    fetch_pages(PB, min(ci + 3, c_hi - 1));
                });
            }
        } else {
            KvRegs X;
            Pages P;
            for (int ci = c_lo; ci < c_hi; ci++) {
                fetch_pages(P, ci);
                load_kv(X, P, ci);
                chunk(X, ci, []() {});
            }
        }
        // ---- this block's partial records: o, and (m, l) of every row
        int oz;  // opaque zero: the per-row indices below stay inside the block loop
        asm volatile("s_mov_b32 %0, 0" : "=s"(oz));
        const int rg4 = g4 + oz, rr16 = r16 + oz;
#pragma unroll
        for (int j = 0; j < kJ; j++)
#pragma unroll
            for (int rt = 0; rt < NT; rt++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int qi = rt * 16 + rg4 * 4 + e;
                    if (qi < nq) {
                        const int gq = qi / Rb, r = r0 + qi % Rb, d = wave * (kMD / kAW) + j * 16 + rr16;
                        part[(((int64_t)grp * R + r) * a.heads + kvh * G + gq) * (kMD + 2) + d] = o[j][rt][e];
                    }
                }
        if (threadIdx.x < nq) {
            const int qi = threadIdx.x, gq = qi / Rb, r = r0 + qi % Rb;
            float *rec = part + (((int64_t)grp * R + r) * a.heads + kvh * G + gq) * (kMD + 2);
            rec[kMD] = Mrow[qi];
            rec[kMD + 1] = Lrow[qi];
        }
    }
}

// Merges the chunk partials of one (query head, row) and applies the output
// gate sigmoid(gate) (forward.go:452-456). The chunk weights exp(m_c - max)
// are computed once per workgroup into LDS.
__device__ __forceinline__ int chunks_total(const AttnVArgs &a, int ck) { return (a.capacity + ck - 1) / ck; }

// Merge of the chunk records of one (head, verify row): softmax weights
// exp(m_c - max) of the chunks' maxima, o = sum_c o_c w_c / sum_c l_c w_c in
// chunk order, times the output gate. Every record field a thread needs is
// requested before the first is used (the chunk maxima and sums, the gate
// and up to kMergeBatch values of the thread's column), so the merge waits
// for one memory round trip instead of one per loop over the chunks.
constexpr int kMergeBatch = 32;
__global__ __launch_bounds__(256) void attn_merge_v_kernel(const float *__restrict__ q, const float *__restrict__ part,
                                                           AttnVArgs a, int ck, int chunks, float *__restrict__ out,
                                                           ModelDyn dyn) {
    extern __shared__ float wsh[];  // [3][chunks]: maxima, sums, weights
    if (blockIdx.z) {  // request blockIdx.z
        const uint64_t rq = blockIdx.z, rows = rq * a.rq_rows;
        q += rows * a.heads * (a.gated ? 2 * a.head_dim : a.head_dim);
        out += rows * a.heads * a.head_dim;
        part += rq * (uint64_t)chunks_total(a, ck) * a.rows * a.heads * (a.head_dim + 2);
        if (dyn.pos_dev) dyn.pos_dev += 2 * rq;
    }
    const int r = blockIdx.y, h = blockIdx.x;
    const int D = a.head_dim;  // <= 256 (launcher)
    const int p0 = cur_pos_a(dyn) + a.displacement;
    const int nchunk = min((p0 + r) / ck + 1, chunks);
    float *ms = wsh, *ls = wsh + chunks, *ws = wsh + 2 * chunks;
    auto rec_of = [&](int c) { return part + (((int64_t)c * a.rows + r) * a.heads + h) * (D + 2); };
    const int d = min((int)threadIdx.x, D - 1);
    const int qstride = a.gated ? 2 * D : D;
    const float gq = a.gated ? q[((int64_t)r * a.heads + h) * qstride + D + d] : 0.0f;
    float v[kMergeBatch];
#pragma unroll
    for (int i = 0; i < kMergeBatch; i++) v[i] = i < nchunk ? rec_of(i)[d] : 0.0f;  // nchunk: workgroup-uniform
    float mx = -INFINITY;
    for (int c = threadIdx.x; c < nchunk; c += 256) {
        const float *rc = rec_of(c);
        ms[c] = rc[D];
        ls[c] = rc[D + 1];
        mx = fmaxf(mx, ms[c]);
    }
    __shared__ float red[4];
    mx = wave_max_f(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int c = threadIdx.x; c < nchunk; c += 256) ws[c] = ms[c] == -INFINITY ? 0.0f : exp_nonpos(ms[c] - mx);
    __syncthreads();
    float lsum = 0.0f;
#pragma unroll 8
    for (int c = 0; c < nchunk; c++) lsum += ls[c] * ws[c];
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kMergeBatch; i++)
        if (i < nchunk) acc += v[i] * ws[i];
    for (int c0 = kMergeBatch; c0 < nchunk; c0 += kMergeBatch) {
#pragma unroll
        for (int i = 0; i < kMergeBatch; i++) v[i] = c0 + i < nchunk ? rec_of(c0 + i)[d] : 0.0f;
#pragma unroll
        for (int i = 0; i < kMergeBatch; i++)
            if (c0 + i < nchunk) acc += v[i] * ws[c0 + i];
    }
    if ((int)threadIdx.x >= D) return;
    float o = acc * (1.0f / lsum);
    if (a.gated) o *= sigmoid_ref(gq);
    out[((int64_t)r * a.heads + h) * D + d] = o;
}

}  // namespace

int attn_verify_chunk(uint32_t fmt) { return fmt == 1 ? KvT<1>::CK : KvT<0>::CK; }

uint64_t attn_verify_scratch_bytes(const AttnVArgs &a) {
    const int ck = attn_verify_chunk(a.fmt);
    const uint64_t chunks = (uint64_t)(a.capacity + ck - 1) / ck;
    return chunks * a.rows * a.heads * (a.head_dim + 2) * 4;
}

uint32_t attn_verify_lds_bytes(const AttnVArgs &a) {
    const int ck = attn_verify_chunk(a.fmt);
    const int esz = a.fmt == 1 ? 2 : 4, pad = a.fmt == 1 ? KvT<1>::PAD : KvT<0>::PAD;
    const int nq = a.heads / a.kv_heads * a.rows;
    const uint32_t kv = (uint32_t)(2 * ck * (a.head_dim + pad) * esz);
    const uint32_t s = (uint32_t)std::max(nq * ck, 4 * a.head_dim) * 4;
    return (uint32_t)(nq * a.head_dim * 4) + kv + 16 + s;
}

hipError_t launch_rope_table(float2 *tab, int rows, int rot_dim, double base, const ModelDyn &dyn, int displacement,
                             hipStream_t s, int nreq, int rq_rows) {
    const int n = rows * (rot_dim / 2);
    rope_table_kernel<<<dim3((unsigned)((n + 255) / 256), (unsigned)(nreq > 0 ? nreq : 1)), 256, 0, s>>>(
        tab, rows, rot_dim, base, dyn, displacement, rq_rows > rows ? rq_rows : rows);
    return hipGetLastError();
}

// The MFMA kernel serves F16 pools with 256-dim heads and 64-dim rotation;
// it walks the verify rows in blocks of kMQ / G, so up to 32 rows a launch.
bool attn_verify_mfma(int fmt, int heads, int kv_heads, int head_dim, int rope_dim, int kv_dim) {
    return fmt == 1 && head_dim == kMD && rope_dim == 64 && kv_heads > 0 && heads / kv_heads <= kMQ &&
           kv_dim % 8 == 0;
}

int attn_verify_max_rows(const AttnVArgs &a) {
    return attn_verify_mfma((int)a.fmt, a.heads, a.kv_heads, a.head_dim, a.rope_dim, a.kv_dim) ? 32 : 16;
}

static int64_t attn_device_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 1;
    }
    return cus;
}

static bool use_mfma_path(const AttnVArgs &a) {
    return attn_verify_mfma((int)a.fmt, a.heads, a.kv_heads, a.head_dim, a.rope_dim, a.kv_dim) && a.rows <= 32;
}

hipError_t launch_attn_verify(const float *q, const float *k, const float *v, void *kpool, void *vpool,
                              const int32_t *table, const float *q_norm, const float *k_norm, const float2 *rope,
                              float *out, const AttnVArgs &a, void *scratch, const ModelDyn &dyn, int max_pos_hint,
                              hipStream_t s) {
    const bool mfma = use_mfma_path(a);
    const unsigned nz = (unsigned)(a.nreq > 0 ? a.nreq : 1);
    // MFMA kernel: groups of cpw chunks per workgroup once a launch has more
    // than ~512 chunk workgroups (fewer partial records, query preparation
    // amortized; config 5's 1056 chunk workgroups: attention + merge 581 ->
    // 464 us per step with pairs, 481 us with fours); short contexts keep
    // one chunk per workgroup
    // Blocks of more than 32 MFMA rows (G x rows) take the PF grouped kernel
    // (3, 5 or 6 row tiles): one workgroup per CU, so its groups are sized
    // for about one round of workgroups over the CUs.
    const bool wide = mfma && (a.heads / a.kv_heads) * a.rows > 32 && a.block_size > 0 &&
                      (a.block_size & (a.block_size - 1)) == 0;
    int cpw = 1;
    if (mfma) {
        const int c1 = (a.capacity + kMK - 1) / kMK;
        const int l1 = max_pos_hint >= 0 ? std::min(c1, max_pos_hint / kMK + 1) : c1;
        const int64_t wgs = (int64_t)l1 * a.kv_heads * nz;
        cpw = (int)std::max<int64_t>(1, std::min<int64_t>(8, wgs / 512));
        if (wide && cpw > 1) {
            // groups per (KV head, request) that fit one workgroup per CU
            const int64_t per = std::max<int64_t>(1, attn_device_cus() / ((int64_t)a.kv_heads * nz));
            cpw = (int)std::max<int64_t>(2, std::min<int64_t>(32, (l1 + per - 1) / per));
        }
        if (const char *e = getenv("YUUKA_ATTN_CPW")) {  // tests and tuning: a fixed group size
            const int v = atoi(e);
            if (v >= 1 && v <= 32) cpw = v;
        }
        // the PF kernels keep the group's page entries in LDS
        if (wide) cpw = std::max(1, std::min(cpw, (kPtCap - 2) * std::max(1, a.block_size) / kMK));
    }
    const int ck = mfma ? kMK * cpw : attn_verify_chunk(a.fmt);
    const int chunks = (a.capacity + ck - 1) / ck;
    const int launch_chunks = max_pos_hint >= 0 ? std::min(chunks, max_pos_hint / ck + 1) : chunks;
    auto *part = static_cast<float *>(scratch);
    static bool attr0 = false, attr1 = false, attr2 = false;
    if (mfma) {
        if (!attr2) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_verify_mfma_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_verify_mfma_group_kernel<2, false>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_verify_mfma_group_kernel<3, true>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_verify_mfma_group_kernel<5, true>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_verify_mfma_group_kernel<6, true>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            attr2 = true;
        }
        const dim3 grid((unsigned)launch_chunks, (unsigned)a.kv_heads, nz);
        if (cpw == 1)
            attn_verify_mfma_kernel<<<grid, 64 * kAW, kMfmaLds, s>>>(q, k, v, static_cast<uint16_t *>(kpool),
                                                                      static_cast<uint16_t *>(vpool), table, q_norm,
                                                                      k_norm, rope, a, part, dyn);
        else if (wide) {
            // row tiles: the launch's MFMA rows in one block where they fit
            const int nq = (a.heads / a.kv_heads) * a.rows;
            if (nq <= 48)
                attn_verify_mfma_group_kernel<3, true><<<grid, 64 * kAW, GroupLds<3>::total, s>>>(
                    q, k, v, static_cast<uint16_t *>(kpool), static_cast<uint16_t *>(vpool), table, q_norm, k_norm,
                    rope, a, part, dyn, cpw);
            else if (nq <= 80)
                attn_verify_mfma_group_kernel<5, true><<<grid, 64 * kAW, GroupLds<5>::total, s>>>(
                    q, k, v, static_cast<uint16_t *>(kpool), static_cast<uint16_t *>(vpool), table, q_norm, k_norm,
                    rope, a, part, dyn, cpw);
            else
                attn_verify_mfma_group_kernel<6, true><<<grid, 64 * kAW, GroupLds<6>::total, s>>>(
                    q, k, v, static_cast<uint16_t *>(kpool), static_cast<uint16_t *>(vpool), table, q_norm, k_norm,
                    rope, a, part, dyn, cpw);
        }
        else
            attn_verify_mfma_group_kernel<2, false><<<grid, 64 * kAW, kMfmaLds, s>>>(
                q, k, v, static_cast<uint16_t *>(kpool), static_cast<uint16_t *>(vpool), table, q_norm, k_norm, rope,
                a, part, dyn, cpw);
    } else if (a.fmt == 1) {
        const uint32_t lds = attn_verify_lds_bytes(a);
        if (!attr1) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_verify_kernel<1>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            attr1 = true;
        }
        attn_verify_kernel<1><<<dim3((unsigned)launch_chunks, (unsigned)a.kv_heads, nz), 256, lds, s>>>(
            q, k, v, static_cast<uint8_t *>(kpool), static_cast<uint8_t *>(vpool), table, q_norm, k_norm, rope, a,
            part, dyn);
    } else {
        const uint32_t lds = attn_verify_lds_bytes(a);
        if (!attr0) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_verify_kernel<0>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            attr0 = true;
        }
        attn_verify_kernel<0><<<dim3((unsigned)launch_chunks, (unsigned)a.kv_heads, nz), 256, lds, s>>>(
            q, k, v, static_cast<uint8_t *>(kpool), static_cast<uint8_t *>(vpool), table, q_norm, k_norm, rope, a,
            part, dyn);
    }
    if (a.head_dim > 256) return hipErrorInvalidValue;  // the merge holds one column per thread
    attn_merge_v_kernel<<<dim3((unsigned)a.heads, (unsigned)a.rows, nz), 256, (size_t)launch_chunks * 12, s>>>(
        q, part, a, ck, launch_chunks, out, dyn);
    return hipGetLastError();
}

}  // namespace yk
