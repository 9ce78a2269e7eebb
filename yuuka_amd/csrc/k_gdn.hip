// k_gdn.hip — Gated DeltaNet block of the verify step, one workgroup per
// value head.
//
// Verify (model/qwen35/recurrent.go:56-105 and forward.go:248-268, 484-493,
// recurrent.go:39-50 in one kernel): for head h the workgroup
//  * runs the causal depthwise conv over [conv state, verify rows] for the
//    head's q, k (group h % groups) and v channels, SiLU, and the L2 norm of
//    q (times 1/sqrt(state)) and k;
//  * keeps the 128 x 128 state in registers (thread = state column j and a
//    quarter of the state rows) and runs the delta rule over the rows;
//  * applies the gated RMSNorm (x * scale * w * silu(z)) to each row's
//    outputs.
// The state and the conv state are left untouched (verify mode); the conv
// outputs are saved for the commit.
//
// Commit: replays the accepted rows (acceptance result[0] + 1) through the
// state and writes it back, and moves the conv state window forward — the
// scan and the conv-state update of one head in one workgroup.
//
// Arithmetic follows the reference's order per element in float32 (the
// compiler may fuse a product into the following sum as one FMA, which
// rounds once where the reference rounds twice), float64 where the
// reference converts (norm sums, exp, log1p). Cross-thread sums add partials
// of 32 state rows in a fixed order.
#include <hip/hip_runtime.h>

#include "model_kernels.h"
#include "refmath.h"

namespace yk {
namespace {

constexpr int kGdnThreads = 512;
constexpr int kS = 128;  // state size (validated by the op)

__device__ __forceinline__ double wave_sum_dd(double v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Sum over the 4 lanes of a quad (quad_perm [1,0,3,2] then [2,3,0,1]), in
// every lane: (p0 + p1) + (p2 + p3).
__device__ __forceinline__ float quad_sum_f(float v) {
    v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, true)));
    return __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, true)));
}

// Causal conv + SiLU of one channel over the rows: every input is requested
// before the first use (one memory round trip).
__device__ __forceinline__ void conv_channel(const float *conv_state, const float *qkv, const float *conv_w,
                                             const GdnArgs &g, int c, float *dst, int dst_stride) {
    const int R = g.rows, K = g.kernel;
    float w[8], st[8], x[16];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        w[i] = i < K ? conv_w[(uint64_t)c * K + i] : 0.0f;
        st[i] = i < K - 1 ? conv_state[(uint64_t)c * (K - 1) + i] : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < 16; r++) x[r] = r < R ? qkv[(uint64_t)r * g.conv_dim + c] : 0.0f;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        if (r >= R) break;
        float sum = 0.0f;
#pragma unroll
        for (int tt = 0; tt < 7; tt++) {
            if (tt >= K - 1) break;
            const int idx = r + tt - (K - 1);
            // idx < 0 reads the conv state slot K - 1 + idx
            float xv = 0.0f;
#pragma unroll
            for (int q = 0; q < 16; q++)
                if (q == idx) xv = x[q];
#pragma unroll
            for (int q = 0; q < 7; q++)
                if (q == K - 1 + idx && idx < 0) xv = st[q];
            sum = __fadd_rn(sum, __fmul_rn(w[tt], xv));
        }
        float wl = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++)
            if (q == K - 1) wl = w[q];
        sum = __fadd_rn(sum, __fmul_rn(wl, x[r]));
        dst[r * dst_stride] = silu_ref(sum);
    }
}

// Sum over each aligned group of 8 lanes, in every lane of the group:
// quad_perm [1,0,3,2], [2,3,0,1], then row_half_mirror (lane i <-> 7 - i).
__device__ __forceinline__ float group8_sum_f(float v) {
    v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xb1, 0xf, 0xf, true)));
    v = __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4e, 0xf, 0xf, true)));
    return __fadd_rn(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, true)));
}

__device__ __forceinline__ float gdn_decay(const GdnArgs &g, const float *alpha_raw, const float *dt,
                                           const float *a_log, int r, int h) {
    if (g.coef) return alpha_raw[(uint64_t)r * g.rank + h];
    const float act = __fmul_rn(softplus_ref(__fadd_rn(alpha_raw[(uint64_t)r * g.rank + h], dt[h])), a_log[h]);
    return (float)exp((double)act);
}

// A row's decay and beta in two steps: the loads (issued early, nothing
// waits for them), then gdn_decay's and the beta map's arithmetic.
struct GdnCoefIn {
    float a, b, dt, al;
};
__device__ __forceinline__ GdnCoefIn gdn_coef_load(const GdnArgs &g, const float *alpha_raw, const float *beta_raw,
                                                   const float *dt, const float *a_log, int r, int h) {
    GdnCoefIn c;
    c.a = alpha_raw[(uint64_t)r * g.rank + h];
    c.b = beta_raw[(uint64_t)r * g.rank + h];
    c.dt = g.coef ? 0.0f : dt[h];  // (read only without precomputed coefficients)
    c.al = g.coef ? 0.0f : a_log[h];
    return c;
}
__device__ __forceinline__ float gdn_coef_decay(const GdnArgs &g, const GdnCoefIn &c) {
    if (g.coef) return c.a;
    return (float)exp((double)__fmul_rn(softplus_ref(__fadd_rn(c.a, c.dt)), c.al));
}
__device__ __forceinline__ float gdn_coef_beta(const GdnArgs &g, const GdnCoefIn &c) {
    return g.coef ? c.b : sigmoid_ref(c.b);
}

// LDS: cv [rows][3][128] conv outputs (q, k, v of this head), raw [rows][128]
// scan outputs.
__global__ __launch_bounds__(kGdnThreads) void gdn_verify_kernel(
    const float *__restrict__ conv_state, const float *__restrict__ state, const float *__restrict__ qkv,
    const float *__restrict__ z, const float *__restrict__ alpha_raw, const float *__restrict__ beta_raw,
    const float *__restrict__ conv_w, const float *__restrict__ dt, const float *__restrict__ a_log,
    const float *__restrict__ norm_w, float *__restrict__ out, float *__restrict__ conv_out, GdnArgs g) {
    extern __shared__ float sm[];
    const int h = blockIdx.x;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int R = g.rows, K = g.kernel;
    const int key_dim = g.groups * kS;
    const int kh = h % g.groups;
    const bool owns_qk = h < g.groups;  // writes the shared q/k conv outputs once
    float *cv = sm;                    // [R][3][128]
    float *raw = cv + R * 3 * kS;      // [R][128]

    // ---- state registers (issued first; used after the conv). Lane l of
    // wave w holds column j = 16 w + l / 4, state rows 32 (l % 4) .. +31: a
    // column's four row quarters sit in one quad.
    const int rq = lane & 3, j = wave * 16 + (lane >> 2);
    const float *mat = state + (uint64_t)h * kS * kS;
    float s_reg[32];
#pragma unroll
    for (int ii = 0; ii < 32; ii++) s_reg[ii] = mat[(uint64_t)(rq * 32 + ii) * kS + j];

    // ---- causal conv + SiLU of the head's 384 channels (forward.go:248-268)
    if (t < 3 * kS) {
        const int part_i = t >> 7, cc = t & (kS - 1);
        const int c = part_i == 0 ? kh * kS + cc : part_i == 1 ? key_dim + kh * kS + cc : 2 * key_dim + h * kS + cc;
        conv_channel(conv_state, qkv, conv_w, g, c, cv + part_i * kS + cc, 3 * kS);
    }
    __syncthreads();
    // ---- L2 norm of q and k per row (forward.go:484-493); save conv outputs
    for (int vec = wave; vec < 2 * R; vec += kGdnThreads / 64) {
        const int r = vec >> 1, which = vec & 1;
        float *x = cv + (r * 3 + which) * kS;
        const float a0 = x[lane], a1 = x[lane + 64];
        double sq = (double)a0 * (double)a0 + (double)a1 * (double)a1;
        sq = wave_sum_dd(sq);
        const float extra = which == 0 ? g.q_scale : 1.0f;
        const float scale = __fmul_rn((float)(1.0 / sqrt(sq + (double)g.eps)), extra);
        const float y0 = __fmul_rn(a0, scale), y1 = __fmul_rn(a1, scale);
        x[lane] = y0;
        x[lane + 64] = y1;
        if (owns_qk) {
            float *dst = conv_out + (uint64_t)r * g.conv_dim + (which == 0 ? 0 : key_dim) + kh * kS;
            dst[lane] = y0;
            dst[lane + 64] = y1;
        }
    }
    for (int idx = t; idx < R * kS; idx += kGdnThreads) {
        const int r = idx / kS, cc = idx % kS;
        conv_out[(uint64_t)r * g.conv_dim + 2 * key_dim + h * kS + cc] = cv[(r * 3 + 2) * kS + cc];
    }
    __syncthreads();

    // ---- delta rule over the rows (recurrent.go:56-105), state untouched;
    // column sums over the quad, no barrier per row
    for (int r = 0; r < R; r++) {
        const float *q = cv + (r * 3 + 0) * kS, *k = cv + (r * 3 + 1) * kS, *v = cv + (r * 3 + 2) * kS;
        const float decay = gdn_decay(g, alpha_raw, dt, a_log, r, h);
        const float beta = g.coef ? beta_raw[(uint64_t)r * g.rank + h] : sigmoid_ref(beta_raw[(uint64_t)r * g.rank + h]);
        float sk = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 32; ii++) {
            s_reg[ii] = __fmul_rn(s_reg[ii], decay);
            sk = __fadd_rn(sk, __fmul_rn(s_reg[ii], k[rq * 32 + ii]));
        }
        sk = quad_sum_f(sk);
        const float d = __fmul_rn(__fsub_rn(v[j], sk), beta);
        float o = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 32; ii++) {
            s_reg[ii] = __fadd_rn(s_reg[ii], __fmul_rn(k[rq * 32 + ii], d));
            o = __fadd_rn(o, __fmul_rn(s_reg[ii], q[rq * 32 + ii]));
        }
        o = quad_sum_f(o);
        if (rq == 0) raw[r * kS + j] = o;
    }
    __syncthreads();
    // ---- gated RMSNorm per row (recurrent.go:39-50)
    for (int r = wave; r < R; r += kGdnThreads / 64) {
        const float x0 = raw[r * kS + lane], x1 = raw[r * kS + lane + 64];
        double s = (double)x0 * (double)x0 + (double)x1 * (double)x1;
        s = wave_sum_dd(s);
        const float mean = (float)(s / (double)kS);
        const float scale = (float)(1.0 / sqrt((double)(mean + g.eps)));
        const uint64_t base = ((uint64_t)r * g.rank + h) * kS;
        const float y0 = __fmul_rn(x0, __fmul_rn(scale, norm_w[lane]));
        const float y1 = __fmul_rn(x1, __fmul_rn(scale, norm_w[lane + 64]));
        out[base + lane] = __fmul_rn(y0, silu_ref(z[base + lane]));
        out[base + lane + 64] = __fmul_rn(y1, silu_ref(z[base + lane + 64]));
    }
}

// Commit of one layer: state replay of the accepted rows and the conv-state
// window (forward.go:259-264); head h owns its v channels and, for
// h < groups, its q/k group's channels.
__global__ __launch_bounds__(kGdnThreads) void gdn_commit_kernel(
    float *__restrict__ conv_state, float *__restrict__ state, const float *__restrict__ qkv,
    const float *__restrict__ conv, const float *__restrict__ alpha_raw, const float *__restrict__ beta_raw,
    const float *__restrict__ dt, const float *__restrict__ a_log, GdnArgs g,
    const int32_t *__restrict__ accept_result) {
    const int h = blockIdx.x;
    const int t = threadIdx.x;
    const int K = g.kernel;
    const int key_dim = g.groups * kS;
    const int kh = h % g.groups;
    const int n = accept_result ? min(accept_result[0] + 1, g.rows) : g.rows;
    // conv-state window: the last K-1 inputs of [old state, raw rows 0..n-1]
    if (t < 3 * kS) {
        const int part_i = t >> 7, cc = t & (kS - 1);
        const bool owner = part_i == 2 || h < g.groups;
        if (owner) {
            const int c = part_i == 0 ? kh * kS + cc : part_i == 1 ? key_dim + kh * kS + cc : 2 * key_dim + h * kS + cc;
            // new slot tt holds sequence index n + tt (relative to row 0);
            // all reads complete before any write (same thread, same channel)
            float win[8];
#pragma unroll
            for (int tt = 0; tt < 7; tt++) {
                const int idx = n + tt - (K - 1);
                win[tt] = tt >= K - 1 ? 0.0f
                          : idx < 0   ? conv_state[(uint64_t)c * (K - 1) + (K - 1 + idx)]
                                      : qkv[(uint64_t)idx * g.conv_dim + c];
            }
#pragma unroll
            for (int tt = 0; tt < 7; tt++)
                if (tt < K - 1) conv_state[(uint64_t)c * (K - 1) + tt] = win[tt];
        }
    }
    const int wave = t >> 6, lane = t & 63;
    const int rq = lane & 3, j = wave * 16 + (lane >> 2);
    float *mat = state + (uint64_t)h * kS * kS;
    float s_reg[32];
#pragma unroll
    for (int ii = 0; ii < 32; ii++) s_reg[ii] = mat[(uint64_t)(rq * 32 + ii) * kS + j];
    for (int r = 0; r < n; r++) {
        const float *row = conv + (uint64_t)r * g.conv_dim;
        const float *k = row + key_dim + kh * kS;
        const float decay = gdn_decay(g, alpha_raw, dt, a_log, r, h);
        const float beta = g.coef ? beta_raw[(uint64_t)r * g.rank + h] : sigmoid_ref(beta_raw[(uint64_t)r * g.rank + h]);
        float kr[32];
#pragma unroll
        for (int ii = 0; ii < 32; ii++) kr[ii] = k[rq * 32 + ii];
        const float vj = row[2 * key_dim + h * kS + j];
        float sk = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 32; ii++) {
            s_reg[ii] = __fmul_rn(s_reg[ii], decay);
            sk = __fadd_rn(sk, __fmul_rn(s_reg[ii], kr[ii]));
        }
        sk = quad_sum_f(sk);
        const float d = __fmul_rn(__fsub_rn(vj, sk), beta);
#pragma unroll
        for (int ii = 0; ii < 32; ii++) s_reg[ii] = __fadd_rn(s_reg[ii], __fmul_rn(kr[ii], d));
    }
#pragma unroll
    for (int ii = 0; ii < 32; ii++) mat[(uint64_t)(rq * 32 + ii) * kS + j] = s_reg[ii];
}


// float64 sum over the wave on the DPP path (16-lane row trees, then the four
// row results through readlane), in every lane.
template <int CTRL>
__device__ __forceinline__ double dpp_dd(double v) {
    const uint64_t b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, 0xf, 0xf, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, 0xf, 0xf, true);
    return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}
__device__ __forceinline__ double rl_dd(double v, int l) {
    const uint64_t b = __double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double wave_sum_dpp(double v) {
    v += dpp_dd<0xb1>(v);
    v += dpp_dd<0x4e>(v);
    v += dpp_dd<0x124>(v);
    v += dpp_dd<0x128>(v);
    return (rl_dd(v, 15) + rl_dd(v, 31)) + (rl_dd(v, 47) + rl_dd(v, 63));
}

// Causal conv + SiLU of two channels (c1 < 0: one) of a width other than 4
// (the models' width takes conv_channels4): a row loop reading the window
// from memory, no register arrays indexed at run time (those would live in
// scratch).
__device__ __forceinline__ void conv_channel2(const float *conv_state, const float *qkv, const float *conv_w,
                                              const GdnArgs &g, int c0, float *dst0, int stride0, int c1, float *dst1,
                                              int stride1) {
    const int R = g.rows, K = g.kernel;
#pragma unroll 1
    for (int u = 0; u < 2; u++) {
        if (u == 1 && c1 < 0) break;
        const uint64_t c = (uint64_t)(u == 0 ? c0 : c1);
        float *dst = u == 0 ? dst0 : dst1;
        const int stride = u == 0 ? stride0 : stride1;
#pragma unroll 1
        for (int r = 0; r < R; r++) {
            float sum = 0.0f;
#pragma unroll 1
            for (int tt = 0; tt < K - 1; tt++) {
                const int idx = r + tt - (K - 1);
                const float xv = idx < 0 ? conv_state[c * (K - 1) + (K - 1 + idx)] : qkv[(uint64_t)idx * g.conv_dim + c];
                sum = __fadd_rn(sum, __fmul_rn(conv_w[c * K + tt], xv));
            }
            sum = __fadd_rn(sum, __fmul_rn(conv_w[c * K + K - 1], qkv[(uint64_t)r * g.conv_dim + c]));
            dst[r * stride] = silu_f32(sum);
        }
    }
}

// Width-4 causal conv + SiLU of N channels (cc[u] < 0: none) with every
// input requested before the first use: one memory round trip for all of
// the thread's channels.
template <int RC, int N>
__device__ __forceinline__ void conv_channels4(const float *conv_state, const float *qkv, const float *conv_w,
                                               const GdnArgs &g, const int (&cc)[N], float *const (&dst)[N],
                                               const int (&stride)[N]) {
    const int R = g.rows;
    float w[N][4], st[N][3], x[N][RC];
#pragma unroll
    for (int u = 0; u < N; u++) {
        const int c = cc[u] < 0 ? 0 : cc[u];  // no channel: loads of channel 0, not used
#pragma unroll
        for (int i = 0; i < 4; i++) w[u][i] = conv_w[(uint64_t)c * 4 + i];
#pragma unroll
        for (int i = 0; i < 3; i++) st[u][i] = conv_state[(uint64_t)c * 3 + i];
#pragma unroll
        for (int r = 0; r < RC; r++) {
            const float xv = qkv[(uint64_t)min(r, R - 1) * g.conv_dim + c];
            x[u][r] = r < R ? xv : 0.0f;
        }
    }
#pragma unroll
    for (int u = 0; u < N; u++) {
        if (cc[u] < 0) continue;
#pragma unroll
        for (int r = 0; r < RC; r++) {
            // a skip, not a break: the loop keeps one exit and unrolls fully,
            // so x[u][...] stays in registers (an early exit left it rolled
            // with x in scratch at 32 rows)
            if (r >= R) continue;
            float sum = 0.0f;
#pragma unroll
            for (int tt = 0; tt < 3; tt++) {
                const int idx = r + tt - 3;
                const float xv = idx >= 0 ? x[u][idx >= 0 ? idx : 0] : st[u][idx >= 0 ? 0 : 3 + idx];
                sum = __fadd_rn(sum, __fmul_rn(w[u][tt], xv));
            }
            sum = __fadd_rn(sum, __fmul_rn(w[u][3], x[u][r]));
            dst[u][r * stride[u]] = silu_f32(sum);
        }
    }
}

// ---- column-split variants: workgroup (head h, block of kCols state
// columns). Lane l of wave w holds column j = kCols * blockIdx.y + 8 w + l / 8
// and state rows 16 (l % 8) .. +15; a column's eight row parts form an
// aligned 8-lane group, so column sums need no barrier.
constexpr int kCols = 32;
constexpr int kMaxRows = 32;  // verify rows of one step (k <= 31 drafts)
constexpr int kColThreads = 256;

// Verify: conv + SiLU + L2 norm of the head's q / k channels and this
// block's v channels, then the delta rule over the rows for this block's
// columns. Writes the raw outputs (the gated norm runs in the consumer) and
// the conv outputs for the commit; the states are left untouched. COLS state
// columns per workgroup (8 per wave); every block of a head repeats the
// head's q / k conv and norm.
template <int RC, int COLS>
__global__ __launch_bounds__(8 * COLS) void gdn_verify_cols_kernel(
    const float *__restrict__ conv_state, const float *__restrict__ state, const float *__restrict__ qkv,
    const float *__restrict__ alpha_raw, const float *__restrict__ beta_raw, const float *__restrict__ conv_w,
    const float *__restrict__ dt, const float *__restrict__ a_log, float *__restrict__ raw_out,
    float *__restrict__ conv_out, GdnArgs g) {
    constexpr int kThr = 8 * COLS;
    extern __shared__ float sm[];
    const int h = blockIdx.x, cb = blockIdx.y;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int R = g.rows;
    {  // request blockIdx.z: states and rows are request-major
        const uint64_t rq = blockIdx.z;
        conv_state += rq * (uint64_t)(g.kernel - 1) * g.conv_dim;
        state += rq * (uint64_t)g.rank * kS * kS;
        qkv += rq * (uint64_t)R * g.conv_dim;
        alpha_raw += rq * (uint64_t)R * g.rank;
        beta_raw += rq * (uint64_t)R * g.rank;
        raw_out += rq * (uint64_t)R * g.rank * kS;
        conv_out += rq * (uint64_t)R * g.conv_dim;
    }
    const int key_dim = g.groups * kS;
    const int kh = h % g.groups;
    float *qk = sm;                 // [R][2][128] q, k
    float *vv = qk + R * 2 * kS;    // [R][COLS]
    float *cf = vv + R * COLS;      // [2][R] decay, beta of every row
    // row t's coefficients: loaded now, computed after the conv (so that no
    // wave waits for them before issuing its state and conv loads)
    const GdnCoefIn cin = gdn_coef_load(g, alpha_raw, beta_raw, dt, a_log, min(t, R - 1), h);
    const int p = lane & 7, j = cb * COLS + wave * 8 + (lane >> 3);
    const float *mat = state + (uint64_t)h * kS * kS;
    float s_reg[16];
#pragma unroll
    for (int ii = 0; ii < 16; ii++) s_reg[ii] = mat[(uint64_t)(p * 16 + ii) * kS + j];
    // conv of the 256 q/k channels (thread t: channels t, t + kThr, ...) and
    // of this block's COLS v channels (threads 0 .. COLS - 1, loaded with
    // their first q/k channel)
    if (g.kernel == 4) {
        constexpr int NQ = (2 * kS + kThr - 1) / kThr, N = NQ + 1;
        int cc[N], stride[N];
        float *dst[N];
#pragma unroll
        for (int u = 0; u < NQ; u++) {
            const int ch = u * kThr + t, which = ch >> 7, c = ch & (kS - 1);
            cc[u] = ch < 2 * kS ? (which == 0 ? 0 : key_dim) + kh * kS + c : -1;
            dst[u] = qk + (which & 1) * kS + c;
            stride[u] = 2 * kS;
        }
        cc[NQ] = t < COLS ? 2 * key_dim + h * kS + cb * COLS + t : -1;
        dst[NQ] = vv + t;
        stride[NQ] = COLS;
        conv_channels4<RC, N>(conv_state, qkv, conv_w, g, cc, dst, stride);
    } else {
#pragma unroll
        for (int base = 0; base < 2 * kS; base += kThr) {
            const int ch = base + t, which = ch >> 7, cc = ch & (kS - 1);
            if (ch >= 2 * kS) break;  // wider blocks: threads past the q / k channels (none of them owns a v channel)
            const int c0 = (which == 0 ? 0 : key_dim) + kh * kS + cc;
            const int c1 = base == 0 && t < COLS ? 2 * key_dim + h * kS + cb * COLS + t : -1;
            conv_channel2(conv_state, qkv, conv_w, g, c0, qk + which * kS + cc, 2 * kS, c1, vv + t, COLS);
        }
    }
    if (t < R) {
        cf[t] = gdn_coef_decay(g, cin);
        cf[R + t] = gdn_coef_beta(g, cin);
    }
    __syncthreads();
    // L2 norm of the 2R q / k vectors. One 16-lane DPP row per vector (lane
    // s of the row holds elements [8 s, 8 s + 8)), two vectors per row at a
    // time: the float64 sums of every vector reduce side by side instead of
    // one wave-wide reduction after another.
    const bool owns_qk = cb == 0 && h < g.groups;
    {
        constexpr int kGroups = kThr / 16;  // DPP rows of the workgroup
        const int s16 = lane & 15, grp = t >> 4;
        for (int v0 = 0; v0 < 2 * R; v0 += 2 * kGroups) {
            float e[2][8];
            double sq[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int vc = min(v0 + u * kGroups + grp, 2 * R - 1);
                const float4 *x = reinterpret_cast<const float4 *>(qk + vc * kS + 8 * s16);
                const float4 x0 = x[0], x1 = x[1];
                e[u][0] = x0.x; e[u][1] = x0.y; e[u][2] = x0.z; e[u][3] = x0.w;
                e[u][4] = x1.x; e[u][5] = x1.y; e[u][6] = x1.z; e[u][7] = x1.w;
                double acc = 0.0;
#pragma unroll
                for (int i = 0; i < 8; i++) acc += (double)e[u][i] * (double)e[u][i];
                sq[u] = acc;
            }
#pragma unroll
            for (int u = 0; u < 2; u++) sq[u] += dpp_dd<0xb1>(sq[u]);
#pragma unroll
            for (int u = 0; u < 2; u++) sq[u] += dpp_dd<0x4e>(sq[u]);
#pragma unroll
            for (int u = 0; u < 2; u++) sq[u] += dpp_dd<0x124>(sq[u]);
#pragma unroll
            for (int u = 0; u < 2; u++) sq[u] += dpp_dd<0x128>(sq[u]);
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int vec = v0 + u * kGroups + grp;
                if (vec >= 2 * R) continue;
                const int r = vec >> 1, which = vec & 1;
                const float extra = which == 0 ? g.q_scale : 1.0f;
                const float scale = __fmul_rn((float)(1.0 / sqrt(sq[u] + (double)g.eps)), extra);
                float y[8];
#pragma unroll
                for (int i = 0; i < 8; i++) y[i] = __fmul_rn(e[u][i], scale);
                float4 *x = reinterpret_cast<float4 *>(qk + vec * kS + 8 * s16);
                x[0] = make_float4(y[0], y[1], y[2], y[3]);
                x[1] = make_float4(y[4], y[5], y[6], y[7]);
                if (owns_qk) {
                    float *dst = conv_out + (uint64_t)r * g.conv_dim + (which == 0 ? 0 : key_dim) + kh * kS + 8 * s16;
#pragma unroll
                    for (int i = 0; i < 8; i++) dst[i] = y[i];
                }
            }
        }
    }
    for (int idx = t; idx < R * COLS; idx += kThr) {
        const int r = idx / COLS, cc = idx % COLS;
        conv_out[(uint64_t)r * g.conv_dim + 2 * key_dim + h * kS + cb * COLS + cc] = vv[r * COLS + cc];
    }
    __syncthreads();
    const int jl = j - cb * COLS;
    // Row r's k, q slices, v and coefficients are read from LDS while row
    // r - 1 is computed (two register sets, alternating).
    struct RowIn {
        float k[16], q[16], v, decay, beta;
    };
    auto fetch = [&](RowIn &in, int r) __attribute__((always_inline)) {
        const float4 *kp = reinterpret_cast<const float4 *>(qk + (r * 2 + 1) * kS + p * 16);
        const float4 *qp = reinterpret_cast<const float4 *>(qk + (r * 2 + 0) * kS + p * 16);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float4 kv = kp[c], qv = qp[c];
            in.k[4 * c] = kv.x; in.k[4 * c + 1] = kv.y; in.k[4 * c + 2] = kv.z; in.k[4 * c + 3] = kv.w;
            in.q[4 * c] = qv.x; in.q[4 * c + 1] = qv.y; in.q[4 * c + 2] = qv.z; in.q[4 * c + 3] = qv.w;
        }
        in.v = vv[r * COLS + jl];
        in.decay = cf[r];
        in.beta = cf[R + r];
    };
    // Column sums over the lane's 16 rows as two interleaved chains (even
    // and odd rows), then the 8-lane group.
    auto step = [&](const RowIn &in, int r) __attribute__((always_inline)) {
        float sk0 = 0.0f, sk1 = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 16; ii += 2) {
            s_reg[ii] = __fmul_rn(s_reg[ii], in.decay);
            s_reg[ii + 1] = __fmul_rn(s_reg[ii + 1], in.decay);
            sk0 = __fadd_rn(sk0, __fmul_rn(s_reg[ii], in.k[ii]));
            sk1 = __fadd_rn(sk1, __fmul_rn(s_reg[ii + 1], in.k[ii + 1]));
        }
        const float sk = group8_sum_f(__fadd_rn(sk0, sk1));
        const float d = __fmul_rn(__fsub_rn(in.v, sk), in.beta);
        float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 16; ii += 2) {
            s_reg[ii] = __fadd_rn(s_reg[ii], __fmul_rn(in.k[ii], d));
            s_reg[ii + 1] = __fadd_rn(s_reg[ii + 1], __fmul_rn(in.k[ii + 1], d));
            o0 = __fadd_rn(o0, __fmul_rn(s_reg[ii], in.q[ii]));
            o1 = __fadd_rn(o1, __fmul_rn(s_reg[ii + 1], in.q[ii + 1]));
        }
        const float o = group8_sum_f(__fadd_rn(o0, o1));
        if (p == 0) raw_out[((uint64_t)r * g.rank + h) * kS + j] = o;
    };
    RowIn ra, rb;
    fetch(ra, 0);
    for (int r = 0; r < R; r += 2) {
        if (r + 1 < R) fetch(rb, r + 1);
        step(ra, r);
        if (r + 1 >= R) break;
        if (r + 2 < R) fetch(ra, r + 2);
        step(rb, r + 1);
    }
}

// Commit of one layer: replay of the accepted rows for this block's
// columns, state written back; this block's v channels and (cb == 0,
// h < groups) the q/k group's channels move their conv window forward.
__device__ __forceinline__ void gdn_commit_cols_body(float *__restrict__ conv_state, float *__restrict__ state,
                                                     const float *__restrict__ qkv, const float *__restrict__ conv,
                                                     const float *__restrict__ alpha_raw,
                                                     const float *__restrict__ beta_raw, const float *__restrict__ dt,
                                                     const float *__restrict__ a_log, const GdnArgs &g, int n) {
    const int h = blockIdx.x, cb = blockIdx.y;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int K = g.kernel;
    const int key_dim = g.groups * kS;
    const int kh = h % g.groups;
    const int p = lane & 7, j = cb * kCols + wave * 8 + (lane >> 3);
    float *mat = state + (uint64_t)h * kS * kS;
    // Every load is issued before the first wait: the block's 128 x 32 state
    // tile (16-byte loads of whole 128-byte row pieces, eight rows per wave
    // instruction), the accepted rows' k, v (this block's columns), decay
    // and beta, and the conv windows. Then the tile goes through LDS, each
    // thread taking its column's 16 rows, and the rows are staged in LDS so
    // that the serial row loop reads LDS only.
    __shared__ float tile[kS][kCols + 1];
    constexpr int kTileIt = kS * kCols / 4 / kColThreads;
    float4 v4[kTileIt];
#pragma unroll
    for (int it = 0; it < kTileIt; it++) {
        const int idx = t + kColThreads * it, row = idx >> 3, c4 = idx & 7;
        v4[it] = *reinterpret_cast<const float4 *>(mat + (uint64_t)row * kS + cb * kCols + 4 * c4);
    }
    // (dynamic LDS sized for the launch's rows: gdn_commit_lds_bytes)
    extern __shared__ float commit_rows[];
    const int R = g.rows;
    float *sk_rows = commit_rows, *sv_rows = sk_rows + R * kS, *scf = sv_rows + R * kCols;  // [R][kS], [R][kCols], [2][R]
    constexpr int kW = kS + kCols;  // staged floats per row
    constexpr int kSG = 4;          // staged values in flight per thread
    const int total = n * kW;
    const GdnCoefIn cin = gdn_coef_load(g, alpha_raw, beta_raw, dt, a_log, min(t, n - 1), h);
    float sv[kSG];
    auto stage_load = [&](int i0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < kSG; u++) {
            const int idx = min(i0 + t + u * kColThreads, total - 1);
            const int r = idx / kW, c = idx - r * kW;
            const float *row = conv + (uint64_t)r * g.conv_dim;
            sv[u] = row[c < kS ? key_dim + kh * kS + c : 2 * key_dim + h * kS + cb * kCols + (c - kS)];
        }
    };
    auto stage_store = [&](int i0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < kSG; u++) {
            const int idx = i0 + t + u * kColThreads;
            if (idx >= total) break;
            const int r = idx / kW, c = idx - r * kW;
            if (c < kS) sk_rows[r * kS + c] = sv[u];
            else sv_rows[r * kCols + c - kS] = sv[u];
        }
    };
    if (total > 0) stage_load(0);
    {  // conv windows: this block's v channels and (cb == 0, h < groups) the q/k group's channels
        const bool qk_owner = cb == 0 && h < g.groups;
        const int nch = kCols + (qk_owner ? 2 * kS : 0);
        for (int ch = t; ch < nch; ch += kColThreads) {
            const int c = ch < kCols ? 2 * key_dim + h * kS + cb * kCols + ch
                                     : ((ch - kCols) < kS ? kh * kS + (ch - kCols) : key_dim + kh * kS + (ch - kCols - kS));
            float win[8];
#pragma unroll
            for (int tt = 0; tt < 7; tt++) {
                const int idx = n + tt - (K - 1);
                win[tt] = tt >= K - 1 ? 0.0f
                          : idx < 0   ? conv_state[(uint64_t)c * (K - 1) + (K - 1 + idx)]
                                      : qkv[(uint64_t)idx * g.conv_dim + c];
            }
#pragma unroll
            for (int tt = 0; tt < 7; tt++)
                if (tt < K - 1) conv_state[(uint64_t)c * (K - 1) + tt] = win[tt];
        }
    }
#pragma unroll
    for (int it = 0; it < kTileIt; it++) {
        const int idx = t + kColThreads * it, row = idx >> 3, c4 = idx & 7;
        tile[row][4 * c4] = v4[it].x;
        tile[row][4 * c4 + 1] = v4[it].y;
        tile[row][4 * c4 + 2] = v4[it].z;
        tile[row][4 * c4 + 3] = v4[it].w;
    }
    for (int i0 = 0; i0 < total; i0 += kSG * kColThreads) {
        if (i0) stage_load(i0);
        stage_store(i0);
    }
    if (t < n) {
        scf[t] = gdn_coef_decay(g, cin);
        scf[R + t] = gdn_coef_beta(g, cin);
    }
    __syncthreads();
    float s_reg[16];
#pragma unroll
    for (int ii = 0; ii < 16; ii++) s_reg[ii] = tile[p * 16 + ii][j - cb * kCols];
    for (int r = 0; r < n; r++) {
        const float *k = sk_rows + r * kS;
        const float decay = scf[r], beta = scf[R + r];
        float kr[16];
#pragma unroll
        for (int ii = 0; ii < 16; ii++) kr[ii] = k[p * 16 + ii];
        const float vj = sv_rows[r * kCols + j - cb * kCols];
        float sk = 0.0f;
#pragma unroll
        for (int ii = 0; ii < 16; ii++) {
            s_reg[ii] = __fmul_rn(s_reg[ii], decay);
            sk = __fadd_rn(sk, __fmul_rn(s_reg[ii], kr[ii]));
        }
        sk = group8_sum_f(sk);
        const float d = __fmul_rn(__fsub_rn(vj, sk), beta);
#pragma unroll
        for (int ii = 0; ii < 16; ii++) s_reg[ii] = __fadd_rn(s_reg[ii], __fmul_rn(kr[ii], d));
    }
    __syncthreads();  // every thread has read its column from the tile
#pragma unroll
    for (int ii = 0; ii < 16; ii++) tile[p * 16 + ii][j - cb * kCols] = s_reg[ii];
    __syncthreads();
#pragma unroll
    for (int it = 0; it < kS * kCols / 4 / kColThreads; it++) {
        const int idx = t + kColThreads * it, row = idx >> 3, c4 = idx & 7;
        *reinterpret_cast<float4 *>(mat + (uint64_t)row * kS + cb * kCols + 4 * c4) =
            make_float4(tile[row][4 * c4], tile[row][4 * c4 + 1], tile[row][4 * c4 + 2], tile[row][4 * c4 + 3]);
    }
}

// Request rq of a request-major launch: its state, rows and result.
__device__ __forceinline__ void gdn_commit_request(float *conv_state, float *state, const float *qkv,
                                                   const float *conv, const float *alpha_raw, const float *beta_raw,
                                                   const float *dt, const float *a_log, const GdnArgs &g,
                                                   const int32_t *accept_result, uint64_t rq) {
    const uint64_t R = (uint64_t)g.rows;
    const int32_t *res = accept_result ? accept_result + 4 * rq : nullptr;
    const int n = res ? min(res[0] + 1, g.rows) : g.rows;
    gdn_commit_cols_body(conv_state + rq * (uint64_t)(g.kernel - 1) * g.conv_dim,
                         state + rq * (uint64_t)g.rank * kS * kS, qkv + rq * R * g.conv_dim,
                         conv + rq * R * g.conv_dim, alpha_raw + rq * R * g.rank, beta_raw + rq * R * g.rank, dt,
                         a_log, g, n);
}

__global__ __launch_bounds__(kColThreads) void gdn_commit_cols_kernel(
    float *__restrict__ conv_state, float *__restrict__ state, const float *__restrict__ qkv,
    const float *__restrict__ conv, const float *__restrict__ alpha_raw, const float *__restrict__ beta_raw,
    const float *__restrict__ dt, const float *__restrict__ a_log, GdnArgs g,
    const int32_t *__restrict__ accept_result) {
    gdn_commit_request(conv_state, state, qkv, conv, alpha_raw, beta_raw, dt, a_log, g, accept_result, blockIdx.z);
}

// Every recurrent layer's commit in one launch (blockIdx.z = layer * nreq +
// request): the layers are independent once the acceptance result is known.
__global__ __launch_bounds__(kColThreads) void gdn_commit_cols_multi_kernel(const GdnCommitSet set, GdnArgs g,
                                                                            const int32_t *__restrict__ accept_result) {
    const int nq = g.nreq > 0 ? g.nreq : 1;
    const GdnCommitLayer &L = set.layer[blockIdx.z / nq];
    gdn_commit_request(L.conv_state, L.state, L.qkv, L.conv, L.alpha, L.beta, L.dt, L.a_log, g, accept_result,
                       blockIdx.z % nq);
}

}  // namespace

// Columns of the state per verify workgroup: the widest of 128 / 64 / 32
// that still gives every CU a workgroup (heads x 128 / COLS x requests >=
// CUs), else 32. Wider blocks share the head's q / k conv and norm over more
// columns; narrower ones spread a small launch over more CUs. Measured per
// launch (16 heads of 128-wide state, 32 / 64 / 128 columns): sixteen
// requests of 9 rows 18.6 / 17.5 / 16.7 us; four requests of 17 rows 19.4 /
// 21.9 / 35.3 us; one request of 5 rows 8.0 / 9.1 / 11.9 us (and 16 columns
// 6.97 against 6.82 us for 32).
static int verify_cols(const GdnArgs &g) {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    const int64_t per = (int64_t)g.rank * (g.nreq > 0 ? g.nreq : 1);  // workgroups per column block
    if (per * 1 >= cus) return 128;
    if (per * 2 >= cus) return 64;
    return 32;
}

static uint32_t verify_cols_lds(const GdnArgs &g, int cols) {
    return (uint32_t)(g.rows * 2 * kS + g.rows * cols + 2 * g.rows) * 4;
}

uint32_t gdn_verify_cols_lds_bytes(const GdnArgs &g) { return verify_cols_lds(g, verify_cols(g)); }

template <int COLS>
static void launch_verify_cols(const float *conv_state, const float *state, const float *qkv, const float *alpha_raw,
                               const float *beta_raw, const float *conv_w, const float *dt, const float *a_log,
                               float *raw_out, float *conv_out, const GdnArgs &g, hipStream_t s) {
    const dim3 grid((unsigned)g.rank, kS / COLS, (unsigned)(g.nreq > 0 ? g.nreq : 1));
    const uint32_t lds = verify_cols_lds(g, COLS);
    // row capacity of the conv registers: the smallest instantiation that holds the rows
    if (g.rows <= 8)
        gdn_verify_cols_kernel<8, COLS><<<grid, 8 * COLS, lds, s>>>(conv_state, state, qkv, alpha_raw, beta_raw,
                                                                    conv_w, dt, a_log, raw_out, conv_out, g);
    else if (g.rows <= 16)
        gdn_verify_cols_kernel<16, COLS><<<grid, 8 * COLS, lds, s>>>(conv_state, state, qkv, alpha_raw, beta_raw,
                                                                     conv_w, dt, a_log, raw_out, conv_out, g);
    else
        gdn_verify_cols_kernel<kMaxRows, COLS><<<grid, 8 * COLS, lds, s>>>(conv_state, state, qkv, alpha_raw,
                                                                           beta_raw, conv_w, dt, a_log, raw_out,
                                                                           conv_out, g);
}

hipError_t launch_gdn_verify_cols(const float *conv_state, const float *state, const float *qkv,
                                  const float *alpha_raw, const float *beta_raw, const float *conv_w, const float *dt,
                                  const float *a_log, float *raw_out, float *conv_out, const GdnArgs &g,
                                  hipStream_t s) {
    switch (verify_cols(g)) {
    case 128:
        launch_verify_cols<128>(conv_state, state, qkv, alpha_raw, beta_raw, conv_w, dt, a_log, raw_out, conv_out, g, s);
        break;
    case 64:
        launch_verify_cols<64>(conv_state, state, qkv, alpha_raw, beta_raw, conv_w, dt, a_log, raw_out, conv_out, g, s);
        break;
    default:
        launch_verify_cols<32>(conv_state, state, qkv, alpha_raw, beta_raw, conv_w, dt, a_log, raw_out, conv_out, g, s);
    }
    return hipGetLastError();
}

// The commit's staged rows: k [rows][128], this block's v [rows][32], decay
// and beta [2][rows] (the state tile is static LDS). Sized by the launch's
// rows, so that more workgroups share a CU at few rows.
static uint32_t gdn_commit_lds_bytes(const GdnArgs &g) { return (uint32_t)(g.rows * (kS + kCols) + 2 * g.rows) * 4; }

hipError_t launch_gdn_commit_cols(float *conv_state, float *state, const float *qkv, const float *conv,
                                  const float *alpha_raw, const float *beta_raw, const float *dt, const float *a_log,
                                  const GdnArgs &g, const int32_t *accept_result, hipStream_t s) {
    if (g.rows < 1 || g.rows > kMaxRows) return hipErrorInvalidValue;
    gdn_commit_cols_kernel<<<dim3((unsigned)g.rank, kS / kCols, (unsigned)(g.nreq > 0 ? g.nreq : 1)), kColThreads,
                             gdn_commit_lds_bytes(g), s>>>(
        conv_state, state, qkv, conv, alpha_raw, beta_raw, dt, a_log, g, accept_result);
    return hipGetLastError();
}

hipError_t launch_gdn_commit_cols_multi(const GdnCommitSet &set, int layers, const GdnArgs &g,
                                        const int32_t *accept_result, hipStream_t s) {
    if (layers < 1 || layers > kGdnCommitMaxLayers || g.rows < 1 || g.rows > kMaxRows) return hipErrorInvalidValue;
    gdn_commit_cols_multi_kernel<<<dim3((unsigned)g.rank, kS / kCols, (unsigned)(layers * (g.nreq > 0 ? g.nreq : 1))),
                                   kColThreads, gdn_commit_lds_bytes(g), s>>>(
        set, g, accept_result);
    return hipGetLastError();
}

uint32_t gdn_verify_lds_bytes(const GdnArgs &g) { return (uint32_t)(g.rows * 3 * kS + g.rows * kS) * 4; }

hipError_t launch_gdn_verify(const float *conv_state, const float *state, const float *qkv, const float *z,
                             const float *alpha_raw, const float *beta_raw, const float *conv_w, const float *dt,
                             const float *a_log, const float *norm_w, float *out, float *conv_out, const GdnArgs &g,
                             hipStream_t s) {
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute(reinterpret_cast<const void *>(gdn_verify_kernel),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
        attr = true;
    }
    gdn_verify_kernel<<<(unsigned)g.rank, kGdnThreads, gdn_verify_lds_bytes(g), s>>>(
        conv_state, state, qkv, z, alpha_raw, beta_raw, conv_w, dt, a_log, norm_w, out, conv_out, g);
    return hipGetLastError();
}

hipError_t launch_gdn_commit(float *conv_state, float *state, const float *qkv, const float *conv,
                             const float *alpha_raw, const float *beta_raw, const float *dt, const float *a_log,
                             const GdnArgs &g, const int32_t *accept_result, hipStream_t s) {
    gdn_commit_kernel<<<(unsigned)g.rank, kGdnThreads, 0, s>>>(conv_state, state, qkv, conv, alpha_raw, beta_raw, dt,
                                                               a_log, g, accept_result);
    return hipGetLastError();
}

}  // namespace yk
