// k_moe.hip — mixture-of-experts FFN of the qwen35moe verify step
// (model/qwen35/forward.go:320-439 forwardMoEFFN / selectExperts) and the
// reference's MoE plan ops (backend/hip/bridge/yuuka_hip.h:457-470).
//
//  * router:   FP32 router logits (and the shared-expert gate logit) of the
//              verify rows, one wave per expert row.
//  * route:    top-`used` experts per row by repeated argmax (lower index
//              wins ties), softmax over the selected logits, and binning of
//              the (row, slot) assignments by expert. One workgroup; the
//              bins are filled in (row, slot) order by one thread per
//              expert, so they are deterministic and every count is written
//              (no memset, graph-safe).
//  * grouped GEMM: one launch over every expert's assigned rows. Workgroups
//              are (expert, part); a workgroup with no assignments exits.
//              The assigned rows are quantized into LDS once per workgroup
//              (int16 split into two int8 planes, one scale per row and
//              256-element super-block, exact sub-block sums for the Q4_K
//              min term) and multiplied with v_mfma_i32_16x16x32_i8 against
//              Q4_K weights decoded from HBM straight into MFMA operand
//              order. Eight assignments fill the high-plane half of one MFMA
//              tile and their low planes the other half.
//  * reduce / combine: weighted sum of the slots (and the sigmoid-gated
//              shared expert) into the residual stream, in the reference's
//              order of float32 operations.
#include <hip/hip_runtime.h>

#include <climits>

#include "model_kernels.h"
#include "refmath.h"

namespace yk {
namespace {

typedef __attribute__((ext_vector_type(4))) int i32x4;

constexpr int kQMax = 32639;     // |q| bound that keeps the high plane in int8
constexpr int kMoeWaves = 8;
constexpr int kMoeThreads = 64 * kMoeWaves;
constexpr int kChunk = 8;        // assignments per MFMA tile (high planes in rows 0..7)

__device__ __forceinline__ float wave_sum(float v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// ---------------------------------------------------------------- router
// logits[r][e] = W[e] . y[r] (FP32 weights, ffn_gate_inp) and, when `sv` is
// given, extra[r] = sv . y[r] (ffn_gate_inp_shexp, forward.go:385).
__global__ __launch_bounds__(kMoeThreads) void moe_router_kernel(const float *__restrict__ y, int H, int rows,
                                                                 const float *__restrict__ w, int E,
                                                                 float *__restrict__ logits,
                                                                 const float *__restrict__ sv,
                                                                 float *__restrict__ extra) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e = blockIdx.x * kMoeWaves + wave;
    if (e > E || (e == E && !sv)) return;
    const float *wr = e < E ? w + (uint64_t)e * H : sv;
    for (int r = 0; r < rows; r++) {
        const float *yr = y + (uint64_t)r * H;
        float acc = 0.f;
        for (int k = 4 * lane; k < H; k += 256) {
            const float4 a = *reinterpret_cast<const float4 *>(wr + k);
            const float4 b = *reinterpret_cast<const float4 *>(yr + k);
            acc += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
        }
        acc = wave_sum(acc);
        if (lane == 0) {
            if (e < E)
                logits[(uint64_t)r * E + e] = acc;
            else
                extra[r] = acc;
        }
    }
}

// ---------------------------------------------------------------- route
// forward.go:393-439 selectExperts for every row, then binning by expert
// (the reference's assignment layout, yuuka_hip.h:457-460: bucket capacity
// rows*used). LDS: ids [rows*used].
__global__ __launch_bounds__(1024) void moe_route_kernel(const float *__restrict__ logits, int rows, int E,
                                                         int used, int32_t *__restrict__ ids,
                                                         float *__restrict__ weights, int32_t *__restrict__ counts,
                                                         int32_t *__restrict__ arows, int32_t *__restrict__ aslots,
                                                         float *__restrict__ aweights) {
    extern __shared__ int32_t sid[];  // ids [rows*used], then weights [rows*used]
    float *sw = reinterpret_cast<float *>(sid + rows * used);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    for (int r = wave; r < rows; r += nw) {
        const float *l = logits + (uint64_t)r * E;
        int32_t *rid = sid + r * used;
        for (int slot = 0; slot < used; slot++) {
            // Reference scan: the first untaken expert starts as best and a
            // later one replaces it only when strictly greater. So a NaN
            // start keeps the slot, NaN elsewhere never wins, and equal
            // maxima resolve to the lowest index.
            int first = INT_MAX, bi = INT_MAX;
            float bv = 0.f;
            for (int e = lane; e < E; e += 64) {
                bool taken = false;
                for (int p = 0; p < slot; p++) taken |= rid[p] == e;
                if (taken) continue;
                first = min(first, e);
                const float v = l[e];
                if (v == v && (bi == INT_MAX || v > bv)) {
                    bv = v;
                    bi = e;
                }
            }
            for (int off = 32; off > 0; off >>= 1) {
                first = min(first, __shfl_xor(first, off));
                const float ov = __shfl_xor(bv, off);
                const int oi = __shfl_xor(bi, off);
                if (oi != INT_MAX && (bi == INT_MAX || ov > bv || (ov == bv && oi < bi))) {
                    bv = ov;
                    bi = oi;
                }
            }
            int pick;
            if (first == INT_MAX)
                pick = 0;  // more slots than experts (forward.go:413-417)
            else if (!(l[first] == l[first]) || bi == INT_MAX)
                pick = first;
            else
                pick = bi;
            if (lane == 0) rid[slot] = pick;
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
        }
        if (lane == 0) {
            // weights: float32(exp(float64(l - max))), float32 total in slot
            // order, then each divided by the total (forward.go:424-438).
            float mx = l[rid[0]];
            for (int s = 1; s < used; s++)
                if (l[rid[s]] > mx) mx = l[rid[s]];
            float total = 0.f;
            for (int s = 0; s < used; s++) total = __fadd_rn(total, (float)exp((double)__fsub_rn(l[rid[s]], mx)));
            for (int s = 0; s < used; s++) {
                const float wt = (float)exp((double)__fsub_rn(l[rid[s]], mx));
                const float v = total > 0.f ? __fdiv_rn(wt, total) : wt;
                sw[r * used + s] = v;
                ids[(uint64_t)r * used + s] = rid[s];
                weights[(uint64_t)r * used + s] = v;
            }
        }
    }
    __syncthreads();
    const int cap = rows * used;
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        int n = 0;
        for (int a = 0; a < cap; a++) {
            if (sid[a] != e) continue;
            const uint64_t o = (uint64_t)e * cap + n;
            arows[o] = a / used;
            aslots[o] = a % used;
            aweights[o] = sw[a];
            n++;
        }
        counts[e] = n;
    }
}

// ---------------------------------------------------------------- grouped GEMM
struct MoeGemmArgs {
    const float *x;       // activation rows [.][K]
    const uint8_t *w0;    // expert-stacked Q4_K rows: expert e, output n at row e*N + n
    const uint8_t *w1;    // second matrix of a gate/up pair (or null)
    uint64_t row_bytes;   // bytes of one packed row (K/256 * 144)
    const int32_t *counts, *arows, *aslots;
    int rows, used, E, K, N, parts;
    int by_slot;          // activation row = row*used + slot (down projection), else row
    int swiglu;           // out0 = SiLU(W0 y) * (W1 y)
    float *out0, *out1;   // [rows*used][N]
};

__device__ __forceinline__ i32x4 mfma_i8(int64_t a, int64_t b) {
    const i32x4 zero = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, zero, 0, 0, 0);
}

// tensor/quant.go:96-103 getScaleMinK4 for the eight sub-blocks of a Q4_K
// block whose scale bytes are s[0..11].
__device__ __forceinline__ void scales_k4(const uint8_t *s, int sc[8], int mn[8]) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
        sc[j] = s[j] & 63;
        mn[j] = s[j + 4] & 63;
        sc[j + 4] = (s[j + 8] & 0xF) | ((s[j] >> 6) << 4);
        mn[j + 4] = (s[j + 8] >> 4) | ((s[j + 4] >> 6) << 4);
    }
}

// LDS layout of one chunk of activations:
//   xa   [K/32 sub-blocks][4 g][16 r][8 B]  r < 8: high plane of row r,
//                                           r >= 8: low plane of row r - 8
//   sums [K/32][8]  int32 sub-block sums of q per row
//   xs   [K/256][8] float scales
__host__ __device__ constexpr uint32_t moe_lds_bytes(int K) {
    return (uint32_t)K * 16 + (uint32_t)(K / 32) * 8 * 4 + (uint32_t)(K / 256) * 8 * 4;
}

__global__ __launch_bounds__(kMoeThreads) void moe_gemm_kernel(MoeGemmArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int e = blockIdx.x, part = blockIdx.y;
    const int count = A.counts[e];
    if (count <= 0) return;
    const int nsb = A.K / 256, nsub = A.K / 32;
    uint8_t *xa = lds;
    int32_t *sums = reinterpret_cast<int32_t *>(lds + (uint32_t)A.K * 16);
    float *xs = reinterpret_cast<float *>(lds + (uint32_t)A.K * 16 + (uint32_t)nsub * 32);
    __shared__ int s_row[kChunk], s_out[kChunk];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int tiles = A.N / 16;
    const int t_begin = (int)((int64_t)tiles * part / A.parts);
    const int t_end = (int)((int64_t)tiles * (part + 1) / A.parts);
    const uint64_t cap = (uint64_t)A.rows * A.used;
    const bool dual = A.w1 != nullptr;

    for (int c0 = 0; c0 < count; c0 += kChunk) {
        const int nr = min(kChunk, count - c0);
        __syncthreads();  // the previous chunk's readers are done with LDS
        if (threadIdx.x < kChunk) {
            const int i = threadIdx.x;
            if (i < nr) {
                const uint64_t o = (uint64_t)e * cap + c0 + i;
                const int row = A.arows[o], slot = A.aslots[o];
                s_out[i] = row * A.used + slot;
                s_row[i] = A.by_slot ? row * A.used + slot : row;
            } else {
                s_out[i] = -1;
                s_row[i] = -1;
            }
        }
        __syncthreads();
        // Quantize: wave per (row, super-block) unit; lane holds 4 elements.
        for (int u = wave; u < kChunk * nsb; u += kMoeWaves) {
            const int i = u / nsb, sb = u % nsb;
            const int j = lane >> 3, g = (lane >> 1) & 3, e0 = (lane & 1) * 4;
            int q[4] = {0, 0, 0, 0};
            float scale = 0.f;
            if (i < nr) {
                const float4 v = *reinterpret_cast<const float4 *>(A.x + (uint64_t)s_row[i] * A.K + sb * 256 + 4 * lane);
                float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
                for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
                const float inv = m > 0.f ? (float)kQMax / m : 0.f;
                scale = m > 0.f ? m / (float)kQMax : 0.f;
                q[0] = (int)rintf(v.x * inv);
                q[1] = (int)rintf(v.y * inv);
                q[2] = (int)rintf(v.z * inv);
                q[3] = (int)rintf(v.w * inv);
            }
            uint32_t hp = 0, lp = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int h = (q[t] + 128) >> 8;
                const int l = q[t] - 256 * h;
                hp |= (uint32_t)(h & 0xff) << (8 * t);
                lp |= (uint32_t)(l & 0xff) << (8 * t);
            }
            uint8_t *dst = xa + ((uint32_t)((sb * 8 + j) * 4 + g)) * 128 + e0;
            *reinterpret_cast<uint32_t *>(dst + i * 8) = hp;
            *reinterpret_cast<uint32_t *>(dst + (8 + i) * 8) = lp;
            int s = q[0] + q[1] + q[2] + q[3];
            s += __shfl_xor(s, 1);
            s += __shfl_xor(s, 2);
            s += __shfl_xor(s, 4);
            if ((lane & 7) == 0) sums[(sb * 8 + j) * 8 + i] = s;
            if (lane == 0) xs[sb * 8 + i] = scale;
        }
        __syncthreads();

        const int c = lane & 15, g = lane >> 4;
        for (int t = t_begin + wave; t < t_end; t += kMoeWaves) {
            const int n0 = t * 16;
            float y[2][4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
            for (int sb = 0; sb < nsb; sb++) {
#pragma unroll
                for (int m = 0; m < 2; m++) {
                    if (m == 1 && !dual) break;
                    const uint8_t *blk =
                        (m ? A.w1 : A.w0) + ((uint64_t)e * A.N + n0 + c) * A.row_bytes + (uint64_t)sb * 144;
                    const uint4 hdr = *reinterpret_cast<const uint4 *>(blk);
                    uint64_t qv[4];
#pragma unroll
                    for (int p = 0; p < 4; p++) qv[p] = *reinterpret_cast<const uint64_t *>(blk + 16 + 32 * p + 8 * g);
                    int sc[8], mn[8];
                    {
                        uint8_t sb12[12];
#pragma unroll
                        for (int p = 0; p < 4; p++) {
                            sb12[p] = (hdr.y >> (8 * p)) & 0xff;
                            sb12[4 + p] = (hdr.z >> (8 * p)) & 0xff;
                            sb12[8 + p] = (hdr.w >> (8 * p)) & 0xff;
                        }
                        scales_k4(sb12, sc, mn);
                    }
                    int acc[4] = {0, 0, 0, 0}, ms[4] = {0, 0, 0, 0};
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        const uint64_t raw = qv[j >> 1];
                        const uint64_t b = (j & 1) ? (raw >> 4) & 0x0F0F0F0F0F0F0F0Full : raw & 0x0F0F0F0F0F0F0F0Full;
                        const int64_t a =
                            *reinterpret_cast<const int64_t *>(xa + ((uint32_t)((sb * 8 + j) * 4 + g)) * 128 + c * 8);
                        const i32x4 r = mfma_i8(a, (int64_t)b);
                        const int4 sm = *reinterpret_cast<const int4 *>(sums + (sb * 8 + j) * 8 + 4 * (g & 1));
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[i] += r[i] * sc[j];
                        ms[0] += mn[j] * sm.x;
                        ms[1] += mn[j] * sm.y;
                        ms[2] += mn[j] * sm.z;
                        ms[3] += mn[j] * sm.w;
                    }
                    const float d = h2f((uint16_t)(hdr.x & 0xffffu)), dmin = h2f((uint16_t)(hdr.x >> 16));
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int lo = __shfl_xor(acc[i], 32);
                        const float v = d * (256.f * (float)acc[i] + (float)lo) - dmin * (float)ms[i];
                        y[m][i] += xs[sb * 8 + ((4 * g + i) & 7)] * v;
                    }
                }
            }
            if (g < 2) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int rr = 4 * g + i;
                    if (rr >= nr) continue;
                    const uint64_t o = (uint64_t)s_out[rr] * A.N + n0 + c;
                    if (A.swiglu) {
                        A.out0[o] = __fmul_rn(silu_ref(y[0][i]), y[1][i]);
                    } else {
                        A.out0[o] = y[0][i];
                        if (dual) A.out1[o] = y[1][i];
                    }
                }
            }
        }
    }
}

// ---------------------------------------------------------------- reduce
// x[r] += sum_slot w[r][slot] * out[r*used + slot] (yuuka_hip.h:468-469),
// and with `so`: + sigmoid(sg[r]) * so[r] (forward.go:381-388). float32
// operations in the reference's order, no contraction (written as plain
// operators under the pragma: the __fmul_rn / __fadd_rn helpers are defined
// in a contractable context and would still be fused after inlining).
__global__ __launch_bounds__(256) void moe_combine_kernel(float *__restrict__ x, const float *__restrict__ eo,
                                                          const float *__restrict__ w, int rows, int used, int H,
                                                          const float *__restrict__ so,
                                                          const float *__restrict__ sg) {
#pragma clang fp contract(off)  // the reference rounds every product and sum
    const int r = blockIdx.x;
    const float *er = eo + (uint64_t)r * used * H;
    const float *wr = w + (uint64_t)r * used;
    const float gate = so ? sigmoid_ref(sg[r]) : 0.f;
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        float t = 0.f;
        for (int s = 0; s < used; s++) t = t + wr[s] * er[(uint64_t)s * H + i];
        if (so) t = t + gate * so[(uint64_t)r * H + i];
        x[(uint64_t)r * H + i] = x[(uint64_t)r * H + i] + t;
    }
}

}  // namespace

uint32_t moe_gemm_lds(int K) { return moe_lds_bytes(K); }

hipError_t launch_moe_router(const float *y, int H, int rows, const float *w, int E, float *logits, const float *sv,
                             float *extra, hipStream_t s) {
    const int n = E + (sv ? 1 : 0);
    moe_router_kernel<<<(n + kMoeWaves - 1) / kMoeWaves, kMoeThreads, 0, s>>>(y, H, rows, w, E, logits, sv, extra);
    return hipGetLastError();
}

hipError_t launch_moe_route(const float *logits, int rows, int E, int used, int32_t *ids, float *weights,
                            int32_t *counts, int32_t *arows, int32_t *aslots, float *aweights, hipStream_t s) {
    const uint32_t lds = (uint32_t)rows * used * 8;
    moe_route_kernel<<<1, 1024, lds, s>>>(logits, rows, E, used, ids, weights, counts, arows, aslots, aweights);
    return hipGetLastError();
}

hipError_t launch_moe_gemm(const MoeGemm &g, hipStream_t s) {
    MoeGemmArgs a{};
    a.x = g.x;
    a.w0 = static_cast<const uint8_t *>(g.w0);
    a.w1 = static_cast<const uint8_t *>(g.w1);
    a.row_bytes = g.row_bytes;
    a.counts = g.counts;
    a.arows = g.arows;
    a.aslots = g.aslots;
    a.rows = g.rows;
    a.used = g.used;
    a.E = g.experts;
    a.K = g.K;
    a.N = g.N;
    a.by_slot = g.by_slot;
    a.swiglu = g.swiglu;
    a.out0 = g.out0;
    a.out1 = g.out1;
    const int tiles = g.N / 16;
    // Enough workgroups per expert that the active experts cover the chip,
    // at least two tiles per wave.
    int parts = tiles / (2 * kMoeWaves);
    parts = parts < 1 ? 1 : (parts > 16 ? 16 : parts);
    a.parts = parts;
    moe_gemm_kernel<<<dim3((unsigned)g.experts, (unsigned)parts), kMoeThreads, moe_lds_bytes(g.K), s>>>(a);
    return hipGetLastError();
}

hipError_t launch_moe_combine(float *x, const float *eo, const float *w, int rows, int used, int H, const float *so,
                              const float *sg, hipStream_t s) {
    moe_combine_kernel<<<rows, 256, 0, s>>>(x, eo, w, rows, used, H, so, sg);
    return hipGetLastError();
}

}  // namespace yk
