// k_model.hip — kernels of the qwen35 verify step other than the GEMM and the
// acceptance: embedding gather, RMSNorm (rows / per head), RoPE, paged KV
// write, paged attention over the verify rows, and the Gated DeltaNet block
// (causal conv + SiLU + L2 norm, delta-rule scan, gated RMSNorm) including
// the commit pass that advances the recurrent state by the accepted rows.
//
// Arithmetic follows model/qwen35/forward.go and recurrent.go: float32 values,
// float64 where the reference converts (norm sums, exp, log1p, RoPE angles).
// Reductions run in parallel, so sums differ from the serial reference order
// by rounding only.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include "model_kernels.h"
#include "refmath.h"

namespace yk {
namespace {



__device__ __forceinline__ int cur_pos(const ModelDyn &dyn) { return dyn.pos_dev ? *dyn.pos_dev : dyn.pos; }

// Wave sums on the DPP path (a __shfl_xor is an LDS permute): pairs, quads,
// half rows and rows of 16 lanes, then the four rows through readlane.
template <int C>
__device__ __forceinline__ double dpp_sum_step(double v) {
    const uint64_t b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, C, 0xf, 0xf, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), C, 0xf, 0xf, true);
    return v + __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}
__device__ __forceinline__ double rl_dbl(double v, int l) {
    const uint64_t b = __double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double wave_sum_dpp(double v) {
    v = dpp_sum_step<0x140>(dpp_sum_step<0x141>(dpp_sum_step<0x4e>(dpp_sum_step<0xb1>(v))));
    return (rl_dbl(v, 0) + rl_dbl(v, 16)) + (rl_dbl(v, 32) + rl_dbl(v, 48));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, true));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, true));
    const auto rl = [](float x, int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), l)); };
    return (rl(v, 0) + rl(v, 16)) + (rl(v, 32) + rl(v, 48));
}

template <typename T>
__device__ __forceinline__ T block_sum256(T v, T *red) {
    v = wave_sum_dpp(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    T s = red[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) s += red[w];
    __syncthreads();
    return s;
}

// ----------------------------------------------------------- embedding
// forward.go:120-130: dequantize the token's table row (bit-exact decoders).
#pragma clang fp contract(off)
__device__ float dequant_one(const uint8_t *row, uint32_t dtype, int col) {
    if (dtype == YUUKA_DTYPE_F32) return reinterpret_cast<const float *>(row)[col];
    if (dtype == YUUKA_DTYPE_F16) return h2f(reinterpret_cast<const uint16_t *>(row)[col]);
    if (dtype == YUUKA_DTYPE_Q8_0) {
        const uint8_t *b = row + (col / 32) * 34;
        return __fmul_rn(h2f((uint16_t)(b[0] | (b[1] << 8))), (float)(int8_t)b[2 + col % 32]);
    }
    if (dtype == YUUKA_DTYPE_Q4_K) {
        const uint8_t *p = row + (col / 256) * 144;
        const int e = col % 256, j = e / 64, l = e % 64, s = 2 * j + (l >= 32);
        const uint8_t *q = p + 4;
        uint32_t sc, mn;
        if (s < 4) { sc = q[s] & 63; mn = q[s + 4] & 63; }
        else { sc = (q[s + 4] & 0x0f) | ((q[s - 4] >> 6) << 4); mn = (q[s + 4] >> 4) | ((q[s] >> 6) << 4); }
        const uint8_t qb = p[16 + 32 * j + (l % 32)];
        const uint32_t v = l < 32 ? (qb & 0x0f) : (qb >> 4);
        const float d = h2f((uint16_t)(p[0] | (p[1] << 8))), dm = h2f((uint16_t)(p[2] | (p[3] << 8)));
        return __fsub_rn(__fmul_rn(__fmul_rn(d, (float)sc), (float)v), __fmul_rn(dm, (float)mn));
    }
    // Q6_K
    const uint8_t *p = row + (col / 256) * 210;
    const int e = col % 256, n = e / 128, t = (e % 128) / 32, l = e % 32;
    const uint8_t qlb = p[64 * n + 32 * (t & 1) + l];
    const uint32_t lo = t < 2 ? (qlb & 0x0f) : (qlb >> 4);
    const uint32_t hi = (p[128 + 32 * n + l] >> (2 * t)) & 3;
    const int q6 = (int)(lo | (hi << 4)) - 32;
    const int sc = (int)(int8_t)p[192 + 8 * n + 2 * t + l / 16];
    const float d = h2f((uint16_t)(p[208] | (p[209] << 8)));
    return __fmul_rn(__fmul_rn(d, (float)sc), (float)q6);
}
#pragma clang fp contract(on)

__global__ __launch_bounds__(256) void embedding_kernel(const uint8_t *__restrict__ table, uint32_t dtype,
                                                        uint64_t row_bytes, const int32_t *__restrict__ tokens,
                                                        int host_token, int vocab, int cols, float *__restrict__ out) {
    const int r = blockIdx.y;
    int tok = tokens ? tokens[r] : host_token;
    tok = tok < 0 ? 0 : (tok >= vocab ? vocab - 1 : tok);  // ids are validated on the host
    const uint8_t *row = table + (uint64_t)tok * row_bytes;
    for (int c = blockIdx.x * 256 + threadIdx.x; c < cols; c += gridDim.x * 256)
        out[(uint64_t)r * cols + c] = dequant_one(row, dtype, c);
}

// ------------------------------------------------------------- RMSNorm
// forward.go:460-470: dst = src * scale * weight, scale from a float64 sum.
__global__ __launch_bounds__(256) void rmsnorm_rows_kernel(const float *__restrict__ src, const float *__restrict__ w,
                                                           float *__restrict__ dst, int cols, uint64_t src_stride,
                                                           uint64_t dst_stride, float eps) {
    __shared__ double red[4];
    const float *x = src + blockIdx.x * src_stride;
    double s = 0.0;
#pragma unroll 8
    for (int c = threadIdx.x; c < cols; c += 256) s += (double)x[c] * (double)x[c];
    s = block_sum256(s, red);
    const float mean = (float)(s / (double)cols);
    const float scale = (float)(1.0 / sqrt((double)(mean + eps)));
    float *y = dst + blockIdx.x * dst_stride;
#pragma unroll 8
    for (int c = threadIdx.x; c < cols; c += 256) y[c] = __fmul_rn(__fmul_rn(x[c], scale), w[c]);
}

// A split-K residual GEMM's reduction (partials summed in split order, then
// + residual, stored to out: bg_reduce_kernel's arithmetic) and the RMSNorm
// of the result (rmsnorm_rows_kernel's arithmetic and summation order) in
// one launch, bit-identical to the two kernels in turn.
template <int P>
__global__ __launch_bounds__(256) void reduce_rmsnorm_rows_kernel(const float *__restrict__ part, uint64_t sstride,
                                                                  int splits, const float *res, float *out,
                                                                  const float *__restrict__ w, float *__restrict__ dst,
                                                                  int cols, uint64_t dst_stride, float eps) {
    // thread t holds elements t + 256 i (i < P, cols = 256 P) in registers;
    // each element sums its partials in split order, SG splits' loads in
    // flight at a time, and the squares add in element order as
    // rmsnorm_rows_kernel adds them
    constexpr int SG = P >= 16 ? 2 : 32 / P;
    __shared__ double red[4];
    const uint64_t r = blockIdx.x, base = r * (uint64_t)cols;
    float v[P];
#pragma unroll
    for (int i = 0; i < P; i++) v[i] = 0.f;
    for (int s0 = 0; s0 < splits; s0 += SG) {
        float t[SG][P];
#pragma unroll
        for (int j = 0; j < SG; j++)
#pragma unroll
            for (int i = 0; i < P; i++)
                if (s0 + j < splits) t[j][i] = part[(uint64_t)(s0 + j) * sstride + base + threadIdx.x + 256 * i];
#pragma unroll
        for (int j = 0; j < SG; j++)
#pragma unroll
            for (int i = 0; i < P; i++)
                if (s0 + j < splits) v[i] += t[j][i];
    }
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < P; i++) {
        const uint64_t o = base + threadIdx.x + 256 * i;
        v[i] = __fadd_rn(v[i], res[o]);
        out[o] = v[i];
        s += (double)v[i] * (double)v[i];
    }
    s = block_sum256(s, red);
    const float mean = (float)(s / (double)cols);
    const float scale = (float)(1.0 / sqrt((double)(mean + eps)));
    float *y = dst + r * dst_stride;
#pragma unroll
    for (int i = 0; i < P; i++) {
        const int c = threadIdx.x + 256 * i;
        y[c] = __fmul_rn(__fmul_rn(v[i], scale), w[c]);
    }
}

// forward.go:472-482 per head: x *= scale * weight.
__global__ __launch_bounds__(256) void rmsnorm_heads_kernel(const float *__restrict__ src, const float *__restrict__ w,
                                                            float *__restrict__ dst, int size, int heads, int stride,
                                                            float eps) {
    __shared__ double red[4];
    const int r = blockIdx.y, h = blockIdx.x;
    const float *x = src + ((uint64_t)r * heads + h) * stride;
    float *y = dst + ((uint64_t)r * heads + h) * stride;
    double s = 0.0;
    for (int c = threadIdx.x; c < size; c += 256) s += (double)x[c] * (double)x[c];
    s = block_sum256(s, red);
    const float mean = (float)(s / (double)size);
    const float scale = (float)(1.0 / sqrt((double)(mean + eps)));
    for (int c = threadIdx.x; c < size; c += 256) y[c] = __fmul_rn(x[c], __fmul_rn(scale, w[c]));
}

// ---------------------------------------------------------------- RoPE
// forward.go:495-514 with position = base position + displacement + row.
__global__ __launch_bounds__(128) void rope_kernel(float *__restrict__ data, int heads, int stride, int rot_dim,
                                                   uint64_t row_stride, double base, ModelDyn dyn, int displacement) {
    const int r = blockIdx.y, i = blockIdx.x * 128 + threadIdx.x;
    const int half = rot_dim / 2;
    if (i >= half) return;
    const int pos = cur_pos(dyn) + displacement + r;
    const double theta = (double)pos * pow(base, -2.0 * (double)i / (double)rot_dim);
    const float c = (float)cos(theta), s = (float)sin(theta);
    float *row = data + (uint64_t)r * row_stride;
    for (int h = 0; h < heads; h++) {
        float *v = row + (uint64_t)h * stride;
        const float x0 = v[i], x1 = v[i + half];
        v[i] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s));
        v[i + half] = __fadd_rn(__fmul_rn(x0, s), __fmul_rn(x1, c));
    }
}

// ----------------------------------------------------------- KV write
// kv_pool.go:131-146 + kv_format.go:93-137 (F32 / F16 rows), positions
// pos + row mapped through the block table (memory.go:254-266).
__global__ __launch_bounds__(256) void kv_write_kernel(const float *__restrict__ k, const float *__restrict__ v,
                                                       uint8_t *__restrict__ kpool, uint8_t *__restrict__ vpool,
                                                       const int32_t *__restrict__ table, int kv_dim, int block_size,
                                                       uint32_t fmt, ModelDyn dyn, int displacement) {
    const int r = blockIdx.y;
    const int p = cur_pos(dyn) + displacement + r;
    const int64_t slot = (int64_t)table[p / block_size] * block_size + p % block_size;
    for (int c = blockIdx.x * 256 + threadIdx.x; c < kv_dim; c += gridDim.x * 256) {
        const float kv0 = k[(uint64_t)r * kv_dim + c], kv1 = v[(uint64_t)r * kv_dim + c];
        if (fmt == 1) {
            reinterpret_cast<uint16_t *>(kpool)[slot * kv_dim + c] = ref_f32_to_f16(kv0);
            reinterpret_cast<uint16_t *>(vpool)[slot * kv_dim + c] = ref_f32_to_f16(kv1);
        } else {
            reinterpret_cast<float *>(kpool)[slot * kv_dim + c] = kv0;
            reinterpret_cast<float *>(vpool)[slot * kv_dim + c] = kv1;
        }
    }
}

// ----------------------------------------------------------- attention
// forward.go:190-218 for `rows` queries at positions pos+disp+r over keys
// 0..pos+disp+r (causal), GQA kvh = h / group, softmax(q.k * scale), then
// out *= sigmoid(gate) for the gated layout (q row = [q | gate] per head).
// Pass 1: workgroup per (kv head, chunk of 64 keys); lane = key for the
// scores, lane = 4 dims for P.V; one wave per query head of the group.
// Pass 2: workgroup per (row, head) merges the chunks.
constexpr int kAttnChunk = 64;

__device__ __forceinline__ float kv_at(const uint8_t *pool, uint32_t fmt, int64_t idx) {
    return fmt == 1 ? h2f(reinterpret_cast<const uint16_t *>(pool)[idx]) : reinterpret_cast<const float *>(pool)[idx];
}

__global__ __launch_bounds__(256) void attn_partial_kernel(const float *__restrict__ q, const uint8_t *__restrict__ kpool,
                                                           const uint8_t *__restrict__ vpool,
                                                           const int32_t *__restrict__ table, AttnArgs a,
                                                           float *__restrict__ part, ModelDyn dyn) {
    extern __shared__ float sm[];
    const int kvh = blockIdx.y, chunk = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int p0 = cur_pos(dyn) + a.displacement;  // position of row 0
    const int last = p0 + a.rows - 1;             // last key any row may see
    const int key0 = chunk * kAttnChunk;
    if (key0 > last) return;  // no row sees this chunk; the merge skips it
    const int D = a.head_dim;
    const int group = a.heads / a.kv_heads;
    float *qs = sm;                                // [group][rows][D]
    float *ps = sm + group * a.rows * D;           // [group][rows][64]
    float *vs = ps + group * a.rows * kAttnChunk;  // [64][D]
    const int qstride = a.gated ? 2 * D : D;
    for (int idx = threadIdx.x; idx < group * a.rows * D; idx += 256) {
        const int g = idx / (a.rows * D), rem = idx % (a.rows * D), r = rem / D, d = rem % D;
        qs[idx] = q[((uint64_t)r * a.heads + kvh * group + g) * qstride + d];
    }
    const int p = key0 + lane;
    const bool key_ok = p <= last;
    int64_t slot = 0;
    if (key_ok) slot = (int64_t)table[p / a.block_size] * a.block_size + p % a.block_size;
    // V chunk to LDS (rows beyond `last` are never weighted)
    for (int idx = threadIdx.x; idx < kAttnChunk * D; idx += 256) {
        const int kk = idx / D, d = idx % D, pp = key0 + kk;
        float val = 0.0f;
        if (pp <= last) {
            const int64_t sl = (int64_t)table[pp / a.block_size] * a.block_size + pp % a.block_size;
            val = kv_at(vpool, a.fmt, sl * a.kv_dim + (int64_t)kvh * D + d);
        }
        vs[idx] = val;
    }
    __syncthreads();
    for (int g = wave; g < group; g += 4) {
        // scores of key `lane` against every row of query head g
        float s[16];
#pragma unroll
        for (int r = 0; r < 16; r++) s[r] = 0.0f;
        if (key_ok) {
            for (int d = 0; d < D; d++) {
                const float kd = kv_at(kpool, a.fmt, slot * a.kv_dim + (int64_t)kvh * D + d);
#pragma unroll
                for (int r = 0; r < 16; r++)
                    if (r < a.rows) s[r] += qs[(g * a.rows + r) * D + d] * kd;
            }
        }
#pragma unroll
        for (int r = 0; r < 16; r++) {
            if (r >= a.rows) break;
            const bool ok = key_ok && p <= p0 + r;
            float sc = ok ? s[r] * a.scale : -INFINITY;
            float m = sc;
            for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
            const float e = ok ? (float)exp((double)(sc - m)) : 0.0f;
            float l = e;
            for (int off = 32; off > 0; off >>= 1) l += __shfl_xor(l, off);
            ps[(g * a.rows + r) * kAttnChunk + lane] = e;
            if (lane == 0) {
                float *rec = part + (((uint64_t)chunk * a.rows + r) * a.heads + kvh * group + g) * (D + 2);
                rec[D] = m;
                rec[D + 1] = l;
            }
        }
    }
    __syncthreads();
    for (int g = wave; g < group; g += 4) {
        for (int r = 0; r < a.rows; r++) {
            float *rec = part + (((uint64_t)chunk * a.rows + r) * a.heads + kvh * group + g) * (D + 2);
            for (int d = lane; d < D; d += 64) {
                float acc = 0.0f;
                for (int kk = 0; kk < kAttnChunk; kk++) acc += ps[(g * a.rows + r) * kAttnChunk + kk] * vs[kk * D + d];
                rec[d] = acc;
            }
        }
    }
}

__global__ __launch_bounds__(256) void attn_merge_kernel(const float *__restrict__ q, const float *__restrict__ part,
                                                         AttnArgs a, int chunks, float *__restrict__ out, ModelDyn dyn) {
    const int r = blockIdx.y, h = blockIdx.x;
    const int D = a.head_dim;
    const int p0 = cur_pos(dyn) + a.displacement;
    const int used = (p0 + r) / kAttnChunk + 1;  // chunks holding keys 0..p0+r
    const int nchunk = min(used, chunks);
    float mx = -INFINITY;
    for (int c = 0; c < nchunk; c++) mx = fmaxf(mx, part[(((uint64_t)c * a.rows + r) * a.heads + h) * (D + 2) + D]);
    float lsum = 0.0f;
    for (int c = 0; c < nchunk; c++) {
        const float *rec = part + (((uint64_t)c * a.rows + r) * a.heads + h) * (D + 2);
        if (rec[D] != -INFINITY) lsum += rec[D + 1] * (float)exp((double)(rec[D] - mx));
    }
    const float inv = 1.0f / lsum;
    const int qstride = a.gated ? 2 * D : D;
    for (int d = threadIdx.x; d < D; d += 256) {
        float acc = 0.0f;
        for (int c = 0; c < nchunk; c++) {
            const float *rec = part + (((uint64_t)c * a.rows + r) * a.heads + h) * (D + 2);
            if (rec[D] != -INFINITY) acc += rec[d] * (float)exp((double)(rec[D] - mx));
        }
        float o = acc * inv;
        if (a.gated) o *= sigmoid_ref(q[((uint64_t)r * a.heads + h) * qstride + D + d]);
        out[((uint64_t)r * a.heads + h) * D + d] = o;
    }
}

// --------------------------------------------------------- Gated DeltaNet
// forward.go:248-268: causal depthwise conv over [conv_state, qkv rows],
// SiLU, then L2 norm of each q (times 1/sqrt(state)) and k group.
// Workgroup per (row, 128-channel group); thread per channel.
__global__ __launch_bounds__(128) void gdn_conv_kernel(const float *__restrict__ conv_state,
                                                       const float *__restrict__ qkv, const float *__restrict__ w,
                                                       float *__restrict__ out, GdnArgs g) {
    __shared__ double red[2];
    const int r = blockIdx.y;
    const int c = blockIdx.x * 128 + threadIdx.x;
    const int K = g.kernel;
    float sum = 0.0f;
    for (int t = 0; t < K - 1; t++) {
        const int idx = r + t - (K - 1);  // time index relative to row 0
        const float xv = idx < 0 ? conv_state[(uint64_t)c * (K - 1) + (K - 1 + idx)] : qkv[(uint64_t)idx * g.conv_dim + c];
        sum = __fadd_rn(sum, __fmul_rn(w[(uint64_t)c * K + t], xv));
    }
    sum = __fadd_rn(sum, __fmul_rn(w[(uint64_t)c * K + K - 1], qkv[(uint64_t)r * g.conv_dim + c]));
    float y = silu_ref(sum);
    const int key_dim = g.groups * g.state;
    if (c < 2 * key_dim) {  // q or k group: L2 norm (forward.go:484-493)
        double s = (double)y * (double)y;
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
        __syncthreads();
        s = red[0] + red[1];
        const float extra = c < key_dim ? g.q_scale : 1.0f;
        const float scale = __fmul_rn((float)(1.0 / sqrt(s + (double)g.eps)), extra);
        y = __fmul_rn(y, scale);
    }
    out[(uint64_t)r * g.conv_dim + c] = y;
}

// recurrent.go:56-105, column-parallel: column j of every head's state
// evolves on its own, so a workgroup owns (head, 64 columns) and its four
// waves split the 128 state rows; the two column sums per token (S^T k and
// S^T q) are reduced across the waves through LDS.
// mode 0 (verify): rows = g.rows, writes the raw per-head outputs, leaves
// the state untouched. mode 1 (commit): rows = accepted + 1 read from the
// acceptance result, writes the state back, no outputs. mode 2 (in place,
// the reference RECURRENT_CHUNK semantics): outputs and state.
__global__ __launch_bounds__(256) void gdn_scan_kernel(float *__restrict__ state, const float *__restrict__ conv,
                                                       const float *__restrict__ alpha_raw,
                                                       const float *__restrict__ beta_raw,
                                                       const float *__restrict__ dt, const float *__restrict__ a_log,
                                                       float *__restrict__ out, GdnArgs g, int mode,
                                                       const int32_t *__restrict__ accept_result) {
    __shared__ float part[2][4][64];
    __shared__ float kq[2][128];
    __shared__ float coef[2];
    const int h = blockIdx.y, jb = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int j = jb * 64 + lane;
    const int S = g.state;  // 128
    const int key_dim = g.groups * S;
    const int kh = h % g.groups;
    int rows = g.rows;
    if (mode == 1) rows = min(accept_result[0] + 1, g.rows);
    float *mat = state + (uint64_t)h * S * S;
    float s_reg[32];
#pragma unroll
    for (int ii = 0; ii < 32; ii++) s_reg[ii] = mat[(uint64_t)(wave * 32 + ii) * S + j];
    for (int r = 0; r < rows; r++) {
        const float *row = conv + (uint64_t)r * g.conv_dim;
        __syncthreads();
        if (threadIdx.x < 128) kq[0][threadIdx.x] = row[key_dim + kh * S + threadIdx.x];
        else kq[1][threadIdx.x - 128] = row[kh * S + threadIdx.x - 128];
        if (threadIdx.x == 0) {
            if (g.coef) {  // decay and sigmoid(beta) precomputed by the projection
                coef[0] = alpha_raw[(uint64_t)r * g.rank + h];
                coef[1] = beta_raw[(uint64_t)r * g.rank + h];
            } else {
                const float act = __fmul_rn(softplus_ref(__fadd_rn(alpha_raw[(uint64_t)r * g.rank + h], dt[h])), a_log[h]);
                coef[0] = (float)exp((double)act);
                coef[1] = sigmoid_ref(beta_raw[(uint64_t)r * g.rank + h]);
            }
        }
        __syncthreads();
        const float decay = coef[0], beta = coef[1];
        float sk = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 32; ii++) {
            s_reg[ii] = __fmul_rn(s_reg[ii], decay);
            sk = __fadd_rn(sk, __fmul_rn(s_reg[ii], kq[0][wave * 32 + ii]));
        }
        part[0][wave][lane] = sk;
        __syncthreads();
        sk = __fadd_rn(__fadd_rn(__fadd_rn(part[0][0][lane], part[0][1][lane]), part[0][2][lane]), part[0][3][lane]);
        const float v = row[2 * key_dim + h * S + j];
        const float d = __fmul_rn(__fsub_rn(v, sk), beta);
        float o = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 32; ii++) {
            s_reg[ii] = __fadd_rn(s_reg[ii], __fmul_rn(kq[0][wave * 32 + ii], d));
            o = __fadd_rn(o, __fmul_rn(s_reg[ii], kq[1][wave * 32 + ii]));
        }
        if (mode != 1) {
            part[1][wave][lane] = o;
            __syncthreads();
            if (wave == 0)
                out[((uint64_t)r * g.rank + h) * S + j] =
                    __fadd_rn(__fadd_rn(__fadd_rn(part[1][0][lane], part[1][1][lane]), part[1][2][lane]), part[1][3][lane]);
        }
    }
    if (mode != 0) {
#pragma unroll
        for (int ii = 0; ii < 32; ii++) mat[(uint64_t)(wave * 32 + ii) * S + j] = s_reg[ii];
    }
}

// recurrent.go:39-50: per (row, head) RMSNorm of the raw outputs, times
// silu(z). Workgroup per (row, head), thread per state column.
__global__ __launch_bounds__(128) void gdn_norm_gate_kernel(const float *__restrict__ raw, const float *__restrict__ z,
                                                            const float *__restrict__ norm, float *__restrict__ out,
                                                            GdnArgs g) {
    __shared__ double red[2];
    const int r = blockIdx.y, h = blockIdx.x, j = threadIdx.x;
    const uint64_t base = ((uint64_t)r * g.rank + h) * g.state;
    const float x = raw[base + j];
    double s = (double)x * (double)x;
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    s = red[0] + red[1];
    const float mean = (float)(s / (double)g.state);
    const float scale = (float)(1.0 / sqrt((double)(mean + g.eps)));
    const float y = __fmul_rn(x, __fmul_rn(scale, norm[j]));
    out[base + j] = __fmul_rn(y, silu_ref(z[base + j]));
}

// Conv-state commit: the state keeps the last (kernel-1) inputs of the
// accepted prefix [old state, qkv rows 0..accepted] (forward.go:259-264).
__global__ __launch_bounds__(256) void gdn_conv_commit_kernel(float *__restrict__ conv_state,
                                                              const float *__restrict__ qkv, GdnArgs g,
                                                              const int32_t *__restrict__ accept_result) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= g.conv_dim) return;
    const int K = g.kernel;
    const int n = accept_result ? min(accept_result[0] + 1, g.rows) : g.rows;  // rows appended
    float win[8];
    for (int t = 0; t < K - 1; t++) {
        const int idx = n + t - (K - 1);  // new state slot t = sequence index n+t relative to row 0
        win[t] = idx < 0 ? conv_state[(uint64_t)c * (K - 1) + (K - 1 + idx)] : qkv[(uint64_t)idx * g.conv_dim + c];
    }
    for (int t = 0; t < K - 1; t++) conv_state[(uint64_t)c * (K - 1) + t] = win[t];
}

__global__ void advance_kernel(ModelDyn dyn, const int32_t *__restrict__ accept_result, int rows,
                               uint64_t *__restrict__ step, int nreq) {
    for (int j = threadIdx.x; j < nreq; j += blockDim.x)
        if (dyn.pos_dev) dyn.pos_dev[2 * j] += min(accept_result[4 * j] + 1, rows);
    if (threadIdx.x == 0 && step) *step += 1;
}

}  // namespace

hipError_t launch_embedding(const void *table, uint32_t dtype, uint64_t row_bytes, const int32_t *tokens, int vocab,
                            int cols, int rows, float *out, hipStream_t s, int host_token) {
    embedding_kernel<<<dim3((unsigned)((cols + 255) / 256), (unsigned)rows), 256, 0, s>>>(
        static_cast<const uint8_t *>(table), dtype, row_bytes, tokens, host_token, vocab, cols, out);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_rows(const float *src, const float *w, float *dst, int cols, int rows, uint64_t src_stride,
                               uint64_t dst_stride, float eps, hipStream_t s) {
    rmsnorm_rows_kernel<<<(unsigned)rows, 256, 0, s>>>(src, w, dst, cols, src_stride, dst_stride, eps);
    return hipGetLastError();
}

hipError_t launch_reduce_rmsnorm_rows(const float *part, uint64_t sstride, int splits, const float *res, float *out,
                                      const float *w, float *dst, int cols, int rows, uint64_t dst_stride, float eps,
                                      hipStream_t s) {
    auto k = cols == 1024   ? reduce_rmsnorm_rows_kernel<4>
             : cols == 2048 ? reduce_rmsnorm_rows_kernel<8>
             : cols == 4096 ? reduce_rmsnorm_rows_kernel<16>
                            : nullptr;
    if (!k) return hipErrorInvalidValue;  // the caller keeps the two kernels for other widths
    k<<<(unsigned)rows, 256, 0, s>>>(part, sstride, splits, res, out, w, dst, cols, dst_stride, eps);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_heads(const float *src, const float *w, float *dst, int size, int heads, int stride, int rows,
                                float eps, hipStream_t s) {
    rmsnorm_heads_kernel<<<dim3((unsigned)heads, (unsigned)rows), 256, 0, s>>>(src, w, dst, size, heads, stride, eps);
    return hipGetLastError();
}

hipError_t launch_rope(float *data, int heads, int stride, int rot_dim, int rows, uint64_t row_stride, double base,
                       const ModelDyn &dyn, int displacement, hipStream_t s) {
    rope_kernel<<<dim3((unsigned)((rot_dim / 2 + 127) / 128), (unsigned)rows), 128, 0, s>>>(
        data, heads, stride, rot_dim, row_stride, base, dyn, displacement);
    return hipGetLastError();
}

hipError_t launch_kv_write(const float *k, const float *v, void *kpool, void *vpool, const int32_t *table, int kv_dim,
                           int rows, int block_size, uint32_t fmt, const ModelDyn &dyn, int displacement,
                           hipStream_t s) {
    kv_write_kernel<<<dim3((unsigned)((kv_dim + 255) / 256), (unsigned)rows), 256, 0, s>>>(
        k, v, static_cast<uint8_t *>(kpool), static_cast<uint8_t *>(vpool), table, kv_dim, block_size, fmt, dyn,
        displacement);
    return hipGetLastError();
}

uint64_t attention_scratch_bytes(const AttnArgs &a) {
    const uint64_t chunks = (uint64_t)(a.capacity + kAttnChunk - 1) / kAttnChunk;
    return chunks * a.rows * a.heads * (a.head_dim + 2) * 4;
}

hipError_t launch_attention(const float *q, const void *kpool, const void *vpool, const int32_t *table, float *out,
                            const AttnArgs &a, void *scratch, const ModelDyn &dyn, int max_pos_hint, hipStream_t s) {
    // chunks needed for the largest position the plan can see
    const int chunks = (a.capacity + kAttnChunk - 1) / kAttnChunk;
    const int launch_chunks = max_pos_hint >= 0 ? std::min(chunks, max_pos_hint / kAttnChunk + 1) : chunks;
    const int group = a.heads / a.kv_heads;
    const size_t lds = (size_t)(group * a.rows * a.head_dim + group * a.rows * kAttnChunk + kAttnChunk * a.head_dim) * 4;
    auto *part = static_cast<float *>(scratch);
    attn_partial_kernel<<<dim3((unsigned)launch_chunks, (unsigned)a.kv_heads), 256, lds, s>>>(
        q, static_cast<const uint8_t *>(kpool), static_cast<const uint8_t *>(vpool), table, a, part, dyn);
    attn_merge_kernel<<<dim3((unsigned)a.heads, (unsigned)a.rows), 256, 0, s>>>(q, part, a, launch_chunks, out, dyn);
    return hipGetLastError();
}

hipError_t launch_gdn_conv(const float *conv_state, const float *qkv, const float *w, float *out, const GdnArgs &g,
                           hipStream_t s) {
    gdn_conv_kernel<<<dim3((unsigned)(g.conv_dim / 128), (unsigned)g.rows), 128, 0, s>>>(conv_state, qkv, w, out, g);
    return hipGetLastError();
}

hipError_t launch_gdn_scan(float *state, const float *conv, const float *alpha, const float *beta, const float *dt,
                           const float *a, float *out, const GdnArgs &g, int mode, const int32_t *accept_result,
                           hipStream_t s) {
    gdn_scan_kernel<<<dim3((unsigned)(g.state / 64), (unsigned)g.rank), 256, 0, s>>>(state, conv, alpha, beta, dt, a,
                                                                                     out, g, mode, accept_result);
    return hipGetLastError();
}

hipError_t launch_gdn_norm_gate(const float *raw, const float *z, const float *norm, float *out, const GdnArgs &g,
                                hipStream_t s) {
    gdn_norm_gate_kernel<<<dim3((unsigned)g.rank, (unsigned)g.rows), 128, 0, s>>>(raw, z, norm, out, g);
    return hipGetLastError();
}

hipError_t launch_gdn_conv_commit(float *conv_state, const float *qkv, const GdnArgs &g, const int32_t *accept_result,
                                  hipStream_t s) {
    gdn_conv_commit_kernel<<<(unsigned)((g.conv_dim + 255) / 256), 256, 0, s>>>(conv_state, qkv, g, accept_result);
    return hipGetLastError();
}

hipError_t launch_advance(const ModelDyn &dyn, const int32_t *accept_result, int rows, uint64_t *step, int nreq,
                          hipStream_t s) {
    advance_kernel<<<1, 256, 0, s>>>(dyn, accept_result, rows, step, nreq);
    return hipGetLastError();
}

}  // namespace yk
