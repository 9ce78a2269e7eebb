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

#include "model_kernels.h"
#include "refmath.h"

namespace yk {
namespace {

__device__ __forceinline__ int cur_pos_a(const ModelDyn &dyn) { return dyn.pos_dev ? *dyn.pos_dev : dyn.pos; }

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
                                  int displacement) {
    const int half = rot_dim / 2;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= rows * half) return;
    const int r = idx / half, i = idx % half;
    const int pos = cur_pos_a(dyn) + displacement + r;
    const double theta = (double)pos * pow(base, -2.0 * (double)i / (double)rot_dim);
    tab[idx] = make_float2((float)cos(theta), (float)sin(theta));
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
        const float c = cs[lane].x, s = cs[lane].y;
        dst[lane] = __fsub_rn(__fmul_rn(y0, c), __fmul_rn(y1, s));
        dst[lane + half] = __fadd_rn(__fmul_rn(y0, s), __fmul_rn(y1, c));
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
        const float e = (sc == -INFINITY) ? 0.0f : (float)exp((double)(sc - m));
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

// Merges the chunk partials of one (query head, row) and applies the output
// gate sigmoid(gate) (forward.go:452-456).
__global__ __launch_bounds__(256) void attn_merge_v_kernel(const float *__restrict__ q, const float *__restrict__ part,
                                                           AttnVArgs a, int ck, int chunks, float *__restrict__ out,
                                                           ModelDyn dyn) {
    const int r = blockIdx.y, h = blockIdx.x;
    const int D = a.head_dim;
    const int p0 = cur_pos_a(dyn) + a.displacement;
    const int nchunk = min((p0 + r) / ck + 1, chunks);
    float mx = -INFINITY;
    for (int c = 0; c < nchunk; c++) mx = fmaxf(mx, part[(((int64_t)c * a.rows + r) * a.heads + h) * (D + 2) + D]);
    float lsum = 0.0f;
    for (int c = 0; c < nchunk; c++) {
        const float *rec = part + (((int64_t)c * a.rows + r) * a.heads + h) * (D + 2);
        if (rec[D] != -INFINITY) lsum += rec[D + 1] * (float)exp((double)(rec[D] - mx));
    }
    const float inv = 1.0f / lsum;
    const int qstride = a.gated ? 2 * D : D;
    for (int d = threadIdx.x; d < D; d += 256) {
        float acc = 0.0f;
        for (int c = 0; c < nchunk; c++) {
            const float *rec = part + (((int64_t)c * a.rows + r) * a.heads + h) * (D + 2);
            if (rec[D] != -INFINITY) acc += rec[d] * (float)exp((double)(rec[D] - mx));
        }
        float o = acc * inv;
        if (a.gated) o *= sigmoid_ref(q[((int64_t)r * a.heads + h) * qstride + D + d]);
        out[((int64_t)r * a.heads + h) * D + d] = o;
    }
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
                             hipStream_t s) {
    const int n = rows * (rot_dim / 2);
    rope_table_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(tab, rows, rot_dim, base, dyn, displacement);
    return hipGetLastError();
}

hipError_t launch_attn_verify(const float *q, const float *k, const float *v, void *kpool, void *vpool,
                              const int32_t *table, const float *q_norm, const float *k_norm, const float2 *rope,
                              float *out, const AttnVArgs &a, void *scratch, const ModelDyn &dyn, int max_pos_hint,
                              hipStream_t s) {
    const int ck = attn_verify_chunk(a.fmt);
    const int chunks = (a.capacity + ck - 1) / ck;
    const int launch_chunks = max_pos_hint >= 0 ? std::min(chunks, max_pos_hint / ck + 1) : chunks;
    const uint32_t lds = attn_verify_lds_bytes(a);
    auto *part = static_cast<float *>(scratch);
    static bool attr0 = false, attr1 = false;
    if (a.fmt == 1) {
        if (!attr1) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_verify_kernel<1>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            attr1 = true;
        }
        attn_verify_kernel<1><<<dim3((unsigned)launch_chunks, (unsigned)a.kv_heads), 256, lds, s>>>(
            q, k, v, static_cast<uint8_t *>(kpool), static_cast<uint8_t *>(vpool), table, q_norm, k_norm, rope, a,
            part, dyn);
    } else {
        if (!attr0) {
            (void)hipFuncSetAttribute(reinterpret_cast<const void *>(attn_verify_kernel<0>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            attr0 = true;
        }
        attn_verify_kernel<0><<<dim3((unsigned)launch_chunks, (unsigned)a.kv_heads), 256, lds, s>>>(
            q, k, v, static_cast<uint8_t *>(kpool), static_cast<uint8_t *>(vpool), table, q_norm, k_norm, rope, a,
            part, dyn);
    }
    attn_merge_v_kernel<<<dim3((unsigned)a.heads, (unsigned)a.rows), 256, 0, s>>>(q, part, a, ck, launch_chunks, out,
                                                                                  dyn);
    return hipGetLastError();
}

}  // namespace yk
