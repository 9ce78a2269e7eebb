// ops.cpp — plan-op validation and dispatch for the non-LM_HEAD ops. Buffer
// layouts follow the reference header comments (yuuka_hip.h:336-476) and the
// Go builders in backend/hip/hip.go (cited per op); extension ops are
// documented in include/yuuka_hip.h.
#include "ops.h"

#include "fgemm.h"
#include "model_kernels.h"

namespace yk {

static bool buf_ok(const yuuka_buffer *b, uint64_t off, uint64_t bytes) {
    return b != nullptr && off <= b->bytes && bytes <= b->bytes - off;
}

template <typename T>
static T *at(const yuuka_op &op, int i) {
    return op.buf[i] ? reinterpret_cast<T *>(static_cast<uint8_t *>(op.buf[i]->ptr) + op.off[i]) : nullptr;
}

static ModelDyn dyn_of(const ExecCtx &ctx) {
    return ModelDyn{ctx.dyn ? const_cast<int32_t *>(ctx.dyn) + 1 : nullptr, (int32_t)ctx.position};
}

// YUUKA_EXT_FLAG_OWN_POS: the op reads its position from its own {token,
// position} buffer in buf15 (one request of a batched plan).
static ModelDyn dyn_of(const ExecCtx &ctx, const yuuka_op &op) {
    if ((op.flags & YUUKA_EXT_FLAG_OWN_POS) && op.buf[15]) return ModelDyn{at<int32_t>(op, 15) + 1, 0};
    return dyn_of(ctx);
}

static uint32_t kv_fmt(uint32_t dtype, bool *ok) {
    *ok = dtype == YUUKA_DTYPE_F32 || dtype == YUUKA_DTYPE_F16;
    return dtype == YUUKA_DTYPE_F16 ? 1u : 0u;
}

static AttnArgs attn_args(const yuuka_op &op) {
    AttnArgs a;
    a.kv_heads = (int)op.n[0];
    a.heads = (int)op.n[1];
    a.head_dim = (int)op.n[2];
    a.kv_dim = (int)op.n[3];
    a.rows = (int)op.n[4];
    a.displacement = (int)op.n[5];
    a.block_size = (int)op.u[0];
    a.capacity = (int)op.u[1];
    bool ok;
    a.fmt = kv_fmt(op.u[2], &ok);
    a.gated = op.u[3] == 0;
    a.scale = op.f[0];
    return a;
}

static AttnVArgs attnv_args(const yuuka_op &op) {
    AttnVArgs a{};
    a.kv_heads = (int)op.n[0];
    a.heads = (int)op.n[1];
    a.head_dim = (int)op.n[2];
    a.kv_dim = (int)op.n[3];
    a.rows = (int)op.n[4];
    a.displacement = (int)op.n[5];
    a.block_size = (int)op.u[0];
    a.capacity = (int)op.u[1];
    bool ok;
    a.fmt = kv_fmt(op.u[2], &ok);
    a.gated = 1;
    a.rope_dim = (int)(op.u[3] & 0xffu);
    a.nreq = (int)((op.u[3] >> 8) & 0xfffu);
    if (a.nreq < 1) a.nreq = 1;
    a.rq_rows = (int)(op.u[3] >> 20);
    if (a.rq_rows < a.rows) a.rq_rows = a.rows;
    a.scale = op.f[0];
    a.eps = op.f[1];
    return a;
}

static GdnArgs gdn_args(const yuuka_op &op) {
    GdnArgs g;
    g.rows = (int)op.n[0];
    g.groups = (int)op.n[1];
    g.rank = (int)op.n[2];
    g.state = (int)op.n[3];
    g.conv_dim = (int)op.n[4];
    g.inner = (int)op.n[5];
    g.kernel = (int)op.u[0];
    g.eps = op.f[0];
    g.q_scale = op.f[1];
    g.coef = (op.flags & YUUKA_EXT_FLAG_GDN_COEF) ? 1 : 0;
    g.nreq = op.u[1] ? (int)op.u[1] : 1;
    return g;
}

// GEMM_FUSED: leading non-null weight buffers (2..5) are the segments.
static int fused_segments(const yuuka_op &op) {
    int n = 0;
    while (n < kFusedMaxSeg && op.buf[2 + n]) n++;
    return n;
}

// 16-row tiles per group: one (the persistent group loop supplies the
// parallelism and keeps registers within one workgroup of eight waves per
// CU); SwiGLU needs a gate and an up tile.
static int fused_tiles(const yuuka_op &op, int) {
    return op.u[1] == kEpiSwiglu ? 2 : 1;
}

// More than 8 rows go to the many-row kernel (k_bgemm.hip).
static bool fused_many_rows(const yuuka_op &op) {
    return op.n[1] > 8;
}

static FusedGemmArgs fused_args(const yuuka_op &op) {
    FusedGemmArgs a{};
    a.x = at<const float>(op, 0);
    a.norm = at<const float>(op, 1);
    a.gate = at<const float>(op, 14);
    a.head_norm = at<const float>(op, 15);
    a.eps = op.f[0];
    a.K = (int)op.n[0];
    a.rows = (int)op.n[1];
    a.chunk_sb = 0;  // set with the tile count
    a.epilogue = (int)op.u[1];
    a.nseg = fused_segments(op);
    for (int i = 0; i < a.nseg; i++) {
        FusedSeg &g = a.seg[i];
        g.dtype = (int)((op.u[0] >> (8 * i)) & 0xff);
        g.n = (int)op.n[2 + i];
        g.row_bytes = (uint32_t)row_bytes((uint32_t)g.dtype, op.n[0]);
        g.w = at<const uint8_t>(op, 2 + i);
        g.w_bytes = (uint32_t)(g.row_bytes * (uint64_t)g.n);
        g.out = at<float>(op, 6 + i);
        g.res = at<const float>(op, 10 + i);
        g.act = (int)((op.u[2] >> (4 * i)) & 0xfu);
        g.p0 = g.p1 = nullptr;
        if (g.act == 3) {  // the (unused) residual slot carries {dt[n], a[n]}
            g.p0 = g.res;
            g.p1 = g.res + g.n;
            g.res = nullptr;
        }
    }
    return a;
}

static yuuka_status check_gdn(const GdnArgs &g, const char *what) {
    if (g.rows <= 0 || g.rows > 64 || g.groups <= 0 || g.rank <= 0 || g.kernel < 2 || g.kernel > 8)
        return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s: invalid rows/groups/heads/kernel", what);
    if (g.state != 128)
        return fail(YUUKA_ERR_UNSUPPORTED, "%s: state size %d (only 128 is served)", what, g.state);
    if (g.conv_dim != 2 * g.groups * g.state + g.inner || g.inner != g.rank * g.state || g.conv_dim % 128)
        return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s: inconsistent conv/inner widths", what);
    return YUUKA_OK;
}


// ------------------------------------------------------------------------
// Single-token decode ops (engine/gpu/plan.go:238-307 buildDecodePlan, layouts
// backend/hip/hip.go): each runs as the one-row form of a verify kernel.

// RECURRENT_TOKEN / GDN read q, k and v from one row laid out [q groups | k
// groups | v heads] (plan.go:484-497: offsets 0, keyDim and 2 keyDim of the
// conv buffer), as the recurrent kernels here do.
static bool qkv_contiguous(const yuuka_op &op, uint64_t key_dim) {
    return op.buf[1] && op.buf[1] == op.buf[2] && op.buf[1] == op.buf[3] && op.off[2] == op.off[1] + key_dim * 4 &&
           op.off[3] == op.off[1] + 2 * key_dim * 4;
}

// GdnArgs of one decode row: groups q/k groups, heads value heads of
// `state` columns, conv_dim channels.
static GdnArgs gdn_row(int groups, int heads, int state, int conv_dim, int kernel, float eps, float q_scale) {
    GdnArgs g{};
    g.rows = 1;
    g.groups = groups;
    g.rank = heads;
    g.state = state;
    g.conv_dim = conv_dim;
    g.inner = heads * state;
    g.kernel = kernel;
    g.eps = eps;
    g.q_scale = q_scale;
    g.coef = 0;
    g.nreq = 1;
    return g;
}

static AttnArgs attn_paged_args(const yuuka_op &op) {  // hip.go:1548-1585
    AttnArgs a{};
    a.kv_heads = (int)op.n[0];
    a.heads = (int)op.n[1];
    a.head_dim = (int)op.n[2];
    a.kv_dim = (int)op.n[3];
    a.rows = 1;
    a.displacement = 0;
    a.block_size = (int)op.u[0];
    a.capacity = (int)op.u[1];
    bool ok;
    a.fmt = kv_fmt(op.u[2], &ok);
    a.gated = op.u[3] == 0;
    a.scale = op.f[0];
    return a;
}

static yuuka_status validate_decode_op(const yuuka_op &op, uint64_t *ws, bool *handled) {
    *handled = true;
    switch (op.code) {
    case YUUKA_OP_EMBEDDING: {  // hip.go:895-921: buf0 W, buf1 out; n={cols, row_bytes}; u0 dtype; the plan's token
        const uint64_t cols = op.n[0], rb = op.n[1];
        const uint32_t dt = op.u[0];
        if (dt != YUUKA_DTYPE_F32 && dt != YUUKA_DTYPE_F16 && dt != YUUKA_DTYPE_Q8_0 && dt != YUUKA_DTYPE_Q4_K &&
            dt != YUUKA_DTYPE_Q6_K)
            return fail(YUUKA_ERR_UNSUPPORTED, "embedding dtype %u", dt);
        if (!cols || row_bytes(dt, cols) != rb) return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid embedding shape");
        if (!buf_ok(op.buf[0], op.off[0], rb) || !buf_ok(op.buf[1], op.off[1], cols * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "embedding buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_RMSNORM: {  // hip.go:541-554: buf0 src, buf1 weight, buf2 dst; n0; f0 eps
        const uint64_t n = op.n[0];
        if (!n || !buf_ok(op.buf[0], op.off[0], n * 4) || !buf_ok(op.buf[1], op.off[1], n * 4) ||
            !buf_ok(op.buf[2], op.off[2], n * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid RMSNorm buffers or width");
        return YUUKA_OK;
    }
    case YUUKA_OP_RMSNORM_HEADS: {  // hip.go:593-608: n={size, heads, stride}
        const uint64_t size = op.n[0], heads = op.n[1], stride = op.n[2];
        if (!size || !heads || stride < size) return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid head RMSNorm dimensions");
        const uint64_t span = (heads - 1) * stride + size;
        if (!buf_ok(op.buf[0], op.off[0], span * 4) || !buf_ok(op.buf[1], op.off[1], size * 4) ||
            !buf_ok(op.buf[2], op.off[2], span * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "head RMSNorm buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_ROPE: {  // hip.go:610-622: buf0 data; n={heads, stride, head_dim, rot_dim}; f0 base
        const uint64_t heads = op.n[0], stride = op.n[1], hd = op.n[2], rot = op.n[3];
        if (!heads || !rot || rot % 2 || rot > hd || stride < hd)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid RoPE dimensions");
        if (!buf_ok(op.buf[0], op.off[0], ((heads - 1) * stride + hd) * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "RoPE buffer too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_KV_WRITE_PAGED: {  // hip.go:1495-1528 with one row
        const uint64_t kv_dim = op.n[0];
        const uint32_t bs = op.u[0], cap = op.u[1];
        bool ok;
        kv_fmt(op.u[2], &ok);
        if (!ok) return fail(YUUKA_ERR_UNSUPPORTED, "KV pool dtype %u (F32 and F16 are served)", op.u[2]);
        if (!kv_dim || !bs || !cap || bs > cap) return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid paged KV write dimensions");
        const uint64_t blocks = (cap + bs - 1) / bs;
        if (!buf_ok(op.buf[0], op.off[0], kv_dim * 4) || !buf_ok(op.buf[1], op.off[1], kv_dim * 4) || !op.buf[2] ||
            !op.buf[3] || !buf_ok(op.buf[4], op.off[4], blocks * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "paged KV write buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_ATTENTION_PAGED: {  // hip.go:1548-1585: buf0 q, buf1/2 pools, buf3 out, buf4 scores, buf5 table
        const AttnArgs a = attn_paged_args(op);
        bool ok;
        kv_fmt(op.u[2], &ok);
        if (!ok) return fail(YUUKA_ERR_UNSUPPORTED, "KV pool dtype %u (F32 and F16 are served)", op.u[2]);
        if (a.heads <= 0 || a.kv_heads <= 0 || a.heads % a.kv_heads || a.kv_dim != a.kv_heads * a.head_dim ||
            a.block_size <= 0 || a.capacity <= 0 || a.block_size > a.capacity || op.n[4] < (uint64_t)a.capacity)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid paged attention dimensions");
        if (a.head_dim % 64 || a.head_dim > 256)
            return fail(YUUKA_ERR_UNSUPPORTED, "attention head dimension %d", a.head_dim);
        const int qs = a.gated ? 2 * a.head_dim : a.head_dim;
        const uint64_t blocks = ((uint64_t)a.capacity + a.block_size - 1) / a.block_size;
        if (!buf_ok(op.buf[0], op.off[0], (uint64_t)a.heads * qs * 4) || !op.buf[1] || !op.buf[2] ||
            !buf_ok(op.buf[3], op.off[3], (uint64_t)a.heads * a.head_dim * 4) ||
            !buf_ok(op.buf[5], op.off[5], blocks * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "paged attention buffers too small");
        *ws = attention_scratch_bytes(a);
        return YUUKA_OK;
    }
    case YUUKA_OP_CONV_L2NORM: {  // hip.go:691-712: n={channels, kernel, qk, q, state}; f={eps, q_scale}
        const uint64_t ch = op.n[0], K = op.n[1], qk = op.n[2], q = op.n[3], st = op.n[4];
        if (K < 2 || K > 8 || !ch || ch % 128 || st != 128 || qk != 2 * q || q % st || qk > ch)
            return fail(YUUKA_ERR_UNSUPPORTED, "conv_l2norm shape (channels %llu, q %llu, k %llu, state %llu)",
                        (unsigned long long)ch, (unsigned long long)q, (unsigned long long)(qk - q),
                        (unsigned long long)st);
        if (!buf_ok(op.buf[0], op.off[0], ch * (K - 1) * 4) || !buf_ok(op.buf[1], op.off[1], ch * K * 4) ||
            !buf_ok(op.buf[2], op.off[2], ch * 4) || !buf_ok(op.buf[3], op.off[3], ch * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "conv_l2norm buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_CONV1D: {  // hip.go:643-655: n={channels, kernel}
        const uint64_t ch = op.n[0], K = op.n[1];
        if (K < 2 || K > 8 || !ch || ch % 128)
            return fail(YUUKA_ERR_UNSUPPORTED, "conv1d shape (channels %llu, kernel %llu)", (unsigned long long)ch,
                        (unsigned long long)K);
        if (!buf_ok(op.buf[0], op.off[0], ch * (K - 1) * 4) || !buf_ok(op.buf[1], op.off[1], ch * K * 4) ||
            !buf_ok(op.buf[2], op.off[2], ch * 4) || !buf_ok(op.buf[3], op.off[3], ch * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "conv1d buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_RECURRENT_TOKEN:  // hip.go:810-834: n={groups, heads, state}; f0 eps
    case YUUKA_OP_GDN: {            // hip.go:657-689: n={groups, heads, state}
        const uint64_t groups = op.n[0], heads = op.n[1], st = op.n[2];
        const bool token = op.code == YUUKA_OP_RECURRENT_TOKEN;
        if (st != 128 || !groups || !heads || heads % groups)
            return fail(YUUKA_ERR_UNSUPPORTED, "recurrent token shape (groups %llu, heads %llu, state %llu)",
                        (unsigned long long)groups, (unsigned long long)heads, (unsigned long long)st);
        const uint64_t key_dim = groups * st, inner = heads * st;
        if (!qkv_contiguous(op, key_dim))
            return fail(YUUKA_ERR_UNSUPPORTED, "recurrent token: q, k and v must be one [q | k | v] row");
        for (int i = 0; i < (token ? 11 : 9); i++)
            if (!op.buf[i]) return fail(YUUKA_ERR_INVALID_ARGUMENT, "recurrent token buffer %d is null", i);
        if (!buf_ok(op.buf[0], op.off[0], heads * st * st * 4) ||
            !buf_ok(op.buf[1], op.off[1], (2 * key_dim + inner) * 4) || !buf_ok(op.buf[4], op.off[4], heads * 4) ||
            !buf_ok(op.buf[5], op.off[5], heads * 4) || !buf_ok(op.buf[6], op.off[6], heads * 4) ||
            !buf_ok(op.buf[7], op.off[7], heads * 4) || !buf_ok(op.buf[8], op.off[8], inner * 4) ||
            (token && (!buf_ok(op.buf[9], op.off[9], st * 4) || !buf_ok(op.buf[10], op.off[10], inner * 4))))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "recurrent token buffers too small");
        *ws = token ? inner * 4 : 0;
        return YUUKA_OK;
    }
    case YUUKA_OP_L2NORM: {  // hip.go:556-575: buf0 src, buf2 dst; n={heads, size, stride}; f={eps, scale}
        const uint64_t heads = op.n[0], size = op.n[1], stride = op.n[2];
        if (!heads || !size || stride < size) return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid L2 norm dimensions");
        const uint64_t span = (heads - 1) * stride + size;
        if (!buf_ok(op.buf[0], op.off[0], span * 4) || !buf_ok(op.buf[2], op.off[2], span * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "L2 norm buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_GATED_RMSNORM: {  // hip.go:577-591: buf0 src, buf1 w, buf2 gate, buf3 dst; n={size, heads, size}
        const uint64_t size = op.n[0], heads = op.n[1];
        if (size != 128 || !heads || op.n[2] != size)
            return fail(YUUKA_ERR_UNSUPPORTED, "gated RMSNorm over heads of %llu (128 is served)",
                        (unsigned long long)size);
        if (!buf_ok(op.buf[0], op.off[0], heads * size * 4) || !buf_ok(op.buf[1], op.off[1], size * 4) ||
            !buf_ok(op.buf[2], op.off[2], heads * size * 4) || !buf_ok(op.buf[3], op.off[3], heads * size * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "gated RMSNorm buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_SCALE: {  // hip.go:884-893: buf0 x; n0; f0 scale
        if (!op.n[0] || !buf_ok(op.buf[0], op.off[0], op.n[0] * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid SCALE buffer or count");
        return YUUKA_OK;
    }
    case YUUKA_OP_QUANT_Q8_1:             // hip.go:1041-1073: buf0 x, buf1 qs, buf2 ds; n={n_in, batch}
    case YUUKA_OP_SILU_MUL_QUANT_Q8_1: {  // hip.go:1075-1093: buf0 gate, buf1 up, buf2 qs, buf3 ds
        const bool swiglu = op.code == YUUKA_OP_SILU_MUL_QUANT_Q8_1;
        const uint64_t n = op.n[0] * (op.n[1] ? op.n[1] : 1);
        const int q = swiglu ? 2 : 1;
        if (!op.n[0] || op.n[0] % 128 || !buf_ok(op.buf[0], op.off[0], n * 4) ||
            (swiglu && !buf_ok(op.buf[1], op.off[1], n * 4)) || !buf_ok(op.buf[q], op.off[q], n) ||
            !buf_ok(op.buf[q + 1], op.off[q + 1], n / 4) || op.off[q + 1] % 8)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid Q8_1 quantization shape or buffers");
        return YUUKA_OK;
    }
    case YUUKA_OP_GEMV_Q8_1: {  // hip.go:1256-1321: buf0 W, buf1 qs (or x), buf2 ds, buf3 out; n={n_in, n_out}; u0 dtype; u1 fused
        const uint64_t K = op.n[0], N = op.n[1];
        const bool fused = op.u[1] != 0;
        yuuka_status st = check_verify_gemm(K, N, 1, op.u[0], 1);
        if (st != YUUKA_OK) return st;
        if (op.off[0] % 16 || !buf_ok(op.buf[0], op.off[0], row_bytes(op.u[0], K) * N) ||
            !buf_ok(op.buf[1], op.off[1], fused ? K * 4 : K) || (!fused && !buf_ok(op.buf[2], op.off[2], K / 4)) ||
            (!fused && op.off[2] % 8) || !buf_ok(op.buf[3], op.off[3], N * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "int8 GEMV buffers too small");
        // the dequantized row (and, fused, its Q8_1 digits and scales)
        *ws = K * 4 + (fused ? ((K + 255) & ~255ull) + K / 4 : 0);
        return YUUKA_OK;
    }
    default:
        *handled = false;
        return YUUKA_OK;
    }
}

static yuuka_status execute_decode_op(const yuuka_op &op, const ExecCtx &ctx, bool *handled) {
    *handled = true;
    hipError_t err = hipSuccess;
    const hipStream_t s = ctx.stream;
    switch (op.code) {
    case YUUKA_OP_EMBEDDING: {
        // the token is the plan's dynamic token (device word 0 of the
        // {token, position} buffer under graph replay, else the host value)
        const uint64_t rb = op.n[1];
        const uint64_t vocab = (op.buf[0]->bytes - op.off[0]) / rb;
        err = launch_embedding(at<const uint8_t>(op, 0), op.u[0], rb, ctx.dyn, (int)std::min<uint64_t>(vocab, INT32_MAX),
                               (int)op.n[0], 1, at<float>(op, 1), s, ctx.token);
        break;
    }
    case YUUKA_OP_RMSNORM:
        err = launch_rmsnorm_rows(at<const float>(op, 0), at<const float>(op, 1), at<float>(op, 2), (int)op.n[0], 1,
                                  op.n[0], op.n[0], op.f[0], s);
        break;
    case YUUKA_OP_RMSNORM_HEADS:
        err = launch_rmsnorm_heads(at<const float>(op, 0), at<const float>(op, 1), at<float>(op, 2), (int)op.n[0],
                                   (int)op.n[1], (int)op.n[2], 1, op.f[0], s);
        break;
    case YUUKA_OP_ROPE:
        err = launch_rope(at<float>(op, 0), (int)op.n[0], (int)op.n[1], (int)op.n[3], 1, op.n[0] * op.n[1],
                          (double)op.f[0], dyn_of(ctx), 0, s);
        break;
    case YUUKA_OP_KV_WRITE_PAGED: {
        if (!ctx.dyn && (uint64_t)ctx.position + 1 > op.u[1])
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "paged KV write at %u exceeds capacity %u", ctx.position, op.u[1]);
        bool ok;
        err = launch_kv_write(at<const float>(op, 0), at<const float>(op, 1), at<uint8_t>(op, 2), at<uint8_t>(op, 3),
                              at<const int32_t>(op, 4), (int)op.n[0], 1, (int)op.u[0], kv_fmt(op.u[2], &ok),
                              dyn_of(ctx), 0, s);
        break;
    }
    case YUUKA_OP_ATTENTION_PAGED: {
        const AttnArgs a = attn_paged_args(op);
        if (!ctx.dyn && ctx.position >= (uint32_t)a.capacity)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "paged attention position %u exceeds capacity %d", ctx.position,
                        a.capacity);
        const int hint = ctx.dyn ? -1 : (int)ctx.position;
        err = launch_attention(at<const float>(op, 0), at<const uint8_t>(op, 1), at<const uint8_t>(op, 2),
                               at<const int32_t>(op, 5), at<float>(op, 3), a, ctx.ws, dyn_of(ctx), hint, s);
        break;
    }
    case YUUKA_OP_CONV_L2NORM:
    case YUUKA_OP_CONV1D: {
        // the convolution of the row against the stored window, SiLU, the q/k
        // L2 norms (CONV_L2NORM only), then the window advances by the row
        const bool norm = op.code == YUUKA_OP_CONV_L2NORM;
        const int st = norm ? (int)op.n[4] : 128;
        const GdnArgs g = gdn_row(norm ? (int)(op.n[3] / op.n[4]) : 0, 0, st, (int)op.n[0], (int)op.n[1],
                                  norm ? op.f[0] : 0.0f, norm ? op.f[1] : 1.0f);
        err = launch_gdn_conv(at<const float>(op, 0), at<const float>(op, 2), at<const float>(op, 1), at<float>(op, 3),
                              g, s);
        if (err == hipSuccess) err = launch_gdn_conv_commit(at<float>(op, 0), at<const float>(op, 2), g, nullptr, s);
        break;
    }
    case YUUKA_OP_RECURRENT_TOKEN:
    case YUUKA_OP_GDN: {
        // one row of the delta rule on the stored state (decay, S^T k, the
        // rank-1 update, S^T q); RECURRENT_TOKEN then applies the gated RMSNorm
        const bool token = op.code == YUUKA_OP_RECURRENT_TOKEN;
        const int groups = (int)op.n[0], heads = (int)op.n[1], st = (int)op.n[2];
        const GdnArgs g = gdn_row(groups, heads, st, 2 * groups * st + heads * st, 2, token ? op.f[0] : 0.0f, 1.0f);
        float *raw = token ? static_cast<float *>(ctx.ws) : at<float>(op, 8);
        err = launch_gdn_scan(at<float>(op, 0), at<const float>(op, 1), at<const float>(op, 4), at<const float>(op, 5),
                              at<const float>(op, 6), at<const float>(op, 7), raw, g, 2, nullptr, s);
        if (err == hipSuccess && token)
            err = launch_gdn_norm_gate(raw, at<const float>(op, 10), at<const float>(op, 9), at<float>(op, 8), g, s);
        break;
    }
    case YUUKA_OP_L2NORM:
        err = launch_l2norm_heads(at<const float>(op, 0), at<float>(op, 2), (int)op.n[0], (int)op.n[1], op.n[2],
                                  op.f[0], op.f[1], s);
        break;
    case YUUKA_OP_GATED_RMSNORM: {
        const GdnArgs g = gdn_row(1, (int)op.n[1], (int)op.n[0], 0, 2, op.f[0], 1.0f);
        err = launch_gdn_norm_gate(at<const float>(op, 0), at<const float>(op, 2), at<const float>(op, 1),
                                   at<float>(op, 3), g, s);
        break;
    }
    case YUUKA_OP_SCALE:
        err = launch_scale_f32(at<float>(op, 0), op.n[0], op.f[0], s);
        break;
    case YUUKA_OP_QUANT_Q8_1:
        err = launch_quant_q8_1(at<const float>(op, 0), nullptr, at<void>(op, 1), at<void>(op, 2),
                                op.n[0] * (op.n[1] ? op.n[1] : 1), s);
        break;
    case YUUKA_OP_SILU_MUL_QUANT_Q8_1:
        err = launch_quant_q8_1(at<const float>(op, 0), at<const float>(op, 1), at<void>(op, 2), at<void>(op, 3),
                                op.n[0] * (op.n[1] ? op.n[1] : 1), s);
        break;
    case YUUKA_OP_GEMV_Q8_1: {
        // the matvec over the Q8_1 row's exact values q * d (the digits are
        // made here from the FP32 row when fused)
        const uint64_t K = op.n[0];
        float *x = static_cast<float *>(ctx.ws);
        const void *qs = at<const void>(op, 1), *ds = at<const void>(op, 2);
        if (op.u[1]) {
            uint8_t *q8 = static_cast<uint8_t *>(ctx.ws) + K * 4;
            uint8_t *d8 = q8 + ((K + 255) & ~255ull);
            err = launch_quant_q8_1(at<const float>(op, 1), nullptr, q8, d8, K, s);
            qs = q8;
            ds = d8;
        }
        if (err == hipSuccess) err = launch_dequant_q8_1(qs, ds, x, K, s);
        if (err != hipSuccess) break;
        FusedGemmArgs a{};
        a.x = x;
        a.K = (int)K;
        a.rows = 1;
        a.epilogue = kEpiStore;
        a.nseg = 1;
        FusedSeg &g = a.seg[0];
        g.dtype = (int)op.u[0];
        g.n = (int)op.n[1];
        g.row_bytes = (uint32_t)row_bytes(op.u[0], K);
        g.w = at<const uint8_t>(op, 0);
        g.w_bytes = (uint32_t)(g.row_bytes * (uint64_t)g.n);
        g.out = at<float>(op, 3);
        a.chunk_sb = fused_gemm_chunk_sb(1, (int)K, 1, false, false);
        err = launch_fused_gemm(a, 1, s);
        break;
    }
    default:
        *handled = false;
        return YUUKA_OK;
    }
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "decode op %u launch: %s", op.code, hip_error(err));
    return YUUKA_OK;
}

bool op_uses_position(const yuuka_op &op) {
    switch (op.code) {
    case YUUKA_OP_ROPE_BATCH:
    case YUUKA_OP_KV_WRITE_BATCH_PAGED:
    case YUUKA_OP_ATTENTION_PREFILL_PAGED:
    case YUUKA_EXT_OP_ROPE_TABLE:
    case YUUKA_EXT_OP_ATTN_VERIFY:
        return !(op.flags & YUUKA_EXT_FLAG_OWN_POS);
    case YUUKA_OP_EMBEDDING:  // the dynamic token
    case YUUKA_OP_ROPE:
    case YUUKA_OP_KV_WRITE_PAGED:
    case YUUKA_OP_ATTENTION_PAGED:
        return true;
    default:
        return false;
    }
}

yuuka_status validate_model_op(const yuuka_op &op, uint64_t *ws) {
    *ws = 0;
    bool decode = false;
    const yuuka_status dst = validate_decode_op(op, ws, &decode);
    if (decode) return dst;
    switch (op.code) {
    case YUUKA_OP_ADD: {  // hip.go:852-861: buf0 x (in/out), buf1 delta; n0
        const uint64_t n = op.n[0];
        if (!n || !buf_ok(op.buf[0], op.off[0], n * 4) || !buf_ok(op.buf[1], op.off[1], n * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid ADD buffers or count");
        return YUUKA_OK;
    }
    case YUUKA_OP_COPY: {  // hip.go:865-884: buf0 dst, buf1 src; n0
        const uint64_t n = op.n[0];
        if (!n || op.off[0] % 4 || op.off[1] % 4 || !buf_ok(op.buf[0], op.off[0], n * 4) ||
            !buf_ok(op.buf[1], op.off[1], n * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid COPY buffers or count");
        return YUUKA_OK;
    }
    case YUUKA_OP_SILU_MUL: {  // hip.go:836-846: buf0 gate, buf1 up, buf2 out; n0
        const uint64_t n = op.n[0];
        if (!n || !buf_ok(op.buf[0], op.off[0], n * 4) || !buf_ok(op.buf[1], op.off[1], n * 4) ||
            !buf_ok(op.buf[2], op.off[2], n * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid SILU_MUL buffers or count");
        return YUUKA_OK;
    }
    case YUUKA_OP_EMBEDDING_BATCH: {  // hip.go:1936-1960
        const uint64_t cols = op.n[0], rows = op.n[1], rb = op.n[2], vocab = op.n[3];
        const uint32_t dt = op.u[0];
        if (dt != YUUKA_DTYPE_F32 && dt != YUUKA_DTYPE_F16 && dt != YUUKA_DTYPE_Q8_0 && dt != YUUKA_DTYPE_Q4_K &&
            dt != YUUKA_DTYPE_Q6_K)
            return fail(YUUKA_ERR_UNSUPPORTED, "embedding dtype %u", dt);
        if (!cols || !rows || !vocab || row_bytes(dt, cols) != rb)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid embedding shape");
        if (!buf_ok(op.buf[0], op.off[0], rb * vocab) || !buf_ok(op.buf[1], op.off[1], cols * rows * 4) ||
            !buf_ok(op.buf[2], op.off[2], rows * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "embedding buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_RMSNORM_BATCH: {  // hip.go:1320-1340
        const uint64_t cols = op.n[0], rows = op.n[1], ss = op.n[2], ds = op.n[3];
        if (!cols || !rows || ss < cols || ds < cols)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid batch RMSNorm dimensions");
        if (!buf_ok(op.buf[0], op.off[0], ((rows - 1) * ss + cols) * 4) || !buf_ok(op.buf[1], op.off[1], cols * 4) ||
            !buf_ok(op.buf[2], op.off[2], ((rows - 1) * ds + cols) * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "batch RMSNorm buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_RMSNORM_HEADS_BATCH: {  // hip.go:1343-1366
        const uint64_t size = op.n[0], heads = op.n[1], stride = op.n[2], rows = op.n[3];
        if (!size || !heads || !rows || stride < size)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid batch head RMSNorm dimensions");
        const uint64_t span = (rows * heads - 1) * stride + size;
        if (!buf_ok(op.buf[0], op.off[0], span * 4) || !buf_ok(op.buf[1], op.off[1], size * 4) ||
            !buf_ok(op.buf[2], op.off[2], span * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "batch head RMSNorm buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_ROPE_BATCH: {  // hip.go:1376-1399
        const uint64_t heads = op.n[0], stride = op.n[1], hd = op.n[2], rot = op.n[3], rows = op.n[4],
                       rs = op.n[5];
        if (!rows || !heads || !rot || rot % 2 || rot > hd || stride < hd || rs < heads * stride)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid batch RoPE dimensions");
        if (!buf_ok(op.buf[0], op.off[0], ((rows - 1) * rs + (heads - 1) * stride + hd) * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "batch RoPE buffer too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_KV_WRITE_BATCH_PAGED: {  // hip.go:1488-1520
        const uint64_t kv_dim = op.n[0], rows = op.n[1];
        const uint32_t bs = op.u[0], cap = op.u[1];
        bool ok;
        kv_fmt(op.u[2], &ok);
        if (!ok) return fail(YUUKA_ERR_UNSUPPORTED, "KV pool dtype %u (F32 and F16 are served)", op.u[2]);
        if (!kv_dim || !rows || !bs || cap < rows || bs > cap)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid paged KV write dimensions");
        const uint64_t blocks = (cap + bs - 1) / bs;
        if (!buf_ok(op.buf[0], op.off[0], rows * kv_dim * 4) || !buf_ok(op.buf[1], op.off[1], rows * kv_dim * 4) ||
            !op.buf[2] || !op.buf[3] || !buf_ok(op.buf[4], op.off[4], blocks * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "paged KV write buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_ATTENTION_PREFILL_PAGED: {  // hip.go:1787-1835
        const AttnArgs a = attn_args(op);
        bool ok;
        kv_fmt(op.u[2], &ok);
        if (!ok) return fail(YUUKA_ERR_UNSUPPORTED, "KV pool dtype %u (F32 and F16 are served)", op.u[2]);
        if (a.rows <= 0 || a.rows > 16 || a.heads <= 0 || a.kv_heads <= 0 || a.heads % a.kv_heads ||
            a.kv_dim != a.kv_heads * a.head_dim || a.block_size <= 0 || a.capacity < a.rows)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid paged attention dimensions");
        if (a.head_dim % 64 || a.head_dim > 256)
            return fail(YUUKA_ERR_UNSUPPORTED, "attention head dimension %d", a.head_dim);
        const int qs = a.gated ? 2 * a.head_dim : a.head_dim;
        const uint64_t blocks = ((uint64_t)a.capacity + a.block_size - 1) / a.block_size;
        if (!buf_ok(op.buf[0], op.off[0], (uint64_t)a.rows * a.heads * qs * 4) || !op.buf[1] || !op.buf[2] ||
            !buf_ok(op.buf[3], op.off[3], (uint64_t)a.rows * a.heads * a.head_dim * 4) ||
            !buf_ok(op.buf[4], op.off[4], blocks * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "paged attention buffers too small");
        *ws = attention_scratch_bytes(a);
        return YUUKA_OK;
    }
    case YUUKA_EXT_OP_ROUTER_NORMAL: {
        const uint64_t rows = op.n[0], E = op.n[1];
        if (!rows || !E || E > 65536 || rows > 65536 || !buf_ok(op.buf[0], op.off[0], rows * E * 4) ||
            (op.buf[1] && (!buf_ok(op.buf[1], op.off[1], 8) || op.off[1] % 8)))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid ROUTER_NORMAL shape or buffers");
        return YUUKA_OK;
    }
    case YUUKA_EXT_OP_ROPE_TABLE: {
        if ((op.flags & YUUKA_EXT_FLAG_OWN_POS) && (!buf_ok(op.buf[15], op.off[15], 8) || op.off[15] % 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "ROPE_TABLE: own position buffer");
        const uint64_t rows = op.n[0], rot = op.n[1], nq = op.n[3] ? op.n[3] : 1;
        const uint64_t rqr = op.n[4] > rows ? op.n[4] : rows;
        if (!rows || rows > 4096 || !rot || rot % 2 || rot > 128 || op.off[0] % 8 || nq > 4096 ||
            !buf_ok(op.buf[0], op.off[0], ((nq - 1) * rqr + rows) * (rot / 2) * 8))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid ROPE_TABLE shape or buffer");
        if (nq > 1 && (!(op.flags & YUUKA_EXT_FLAG_OWN_POS) || !buf_ok(op.buf[15], op.off[15], 8 * nq)))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "ROPE_TABLE: several requests need their own positions");
        return YUUKA_OK;
    }
    case YUUKA_EXT_OP_ATTN_VERIFY: {
        const AttnVArgs a = attnv_args(op);
        if ((op.flags & YUUKA_EXT_FLAG_OWN_POS) &&
            (!buf_ok(op.buf[15], op.off[15], 8ull * a.nreq) || op.off[15] % 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "ATTN_VERIFY: own position buffer");
        if (a.nreq > 1 && !(op.flags & YUUKA_EXT_FLAG_OWN_POS))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "ATTN_VERIFY: several requests need their own positions");
        bool ok;
        kv_fmt(op.u[2], &ok);
        if (!ok) return fail(YUUKA_ERR_UNSUPPORTED, "KV pool dtype %u (F32 and F16 are served)", op.u[2]);
        if (a.rows <= 0 || a.heads <= 0 || a.kv_heads <= 0 || a.heads % a.kv_heads ||
            a.kv_dim != a.kv_heads * a.head_dim || a.block_size <= 0 || a.capacity < a.rows)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid verify attention dimensions");
        if (a.rows > attn_verify_max_rows(a))
            return fail(YUUKA_ERR_UNSUPPORTED, "verify attention: %d rows in one op (at most %d)", a.rows,
                        attn_verify_max_rows(a));
        if (a.head_dim % 64 || a.head_dim > 256 || a.rope_dim <= 0 || a.rope_dim % 2 || a.rope_dim > a.head_dim ||
            a.rope_dim > 128)
            return fail(YUUKA_ERR_UNSUPPORTED, "attention head dimension %d / rotation %d", a.head_dim, a.rope_dim);
        if (!attn_verify_mfma((int)a.fmt, a.heads, a.kv_heads, a.head_dim, a.rope_dim, a.kv_dim) &&
            attn_verify_lds_bytes(a) > 160 * 1024)
            return fail(YUUKA_ERR_UNSUPPORTED, "verify attention: %d query rows per kv head do not fit LDS",
                        a.rows * a.heads / a.kv_heads);
        const uint64_t blocks = ((uint64_t)a.capacity + a.block_size - 1) / a.block_size;
        // rows spanned by the requests, and block table entries
        const uint64_t R = (uint64_t)(a.nreq - 1) * a.rq_rows + a.rows;
        const uint64_t tbl = (uint64_t)a.nreq * blocks;
        if (!buf_ok(op.buf[0], op.off[0], R * a.heads * 2 * a.head_dim * 4) ||
            !buf_ok(op.buf[1], op.off[1], R * a.kv_dim * 4) || !buf_ok(op.buf[2], op.off[2], R * a.kv_dim * 4) ||
            !op.buf[3] || !op.buf[4] || !buf_ok(op.buf[5], op.off[5], R * a.heads * a.head_dim * 4) ||
            !buf_ok(op.buf[6], op.off[6], tbl * 4) || !buf_ok(op.buf[7], op.off[7], (uint64_t)a.head_dim * 4) ||
            !buf_ok(op.buf[8], op.off[8], (uint64_t)a.head_dim * 4) ||
            !buf_ok(op.buf[9], op.off[9], R * (a.rope_dim / 2) * 8))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "verify attention buffers too small");
        const uint64_t esz = a.fmt == 1 ? 2 : 4;
        const uint64_t pool = (uint64_t)blocks * a.block_size * a.kv_dim * esz;
        if (op.buf[3]->bytes < pool || op.buf[4]->bytes < pool)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "verify attention: KV pool smaller than capacity");
        *ws = attn_verify_scratch_bytes(a) * (uint64_t)a.nreq;
        return YUUKA_OK;
    }
    case YUUKA_OP_RECURRENT_CHUNK: {  // hip.go:1874-1934
        const GdnArgs g = gdn_args(op);
        yuuka_status st = check_gdn(g, "recurrent chunk");
        if (st != YUUKA_OK) return st;
        for (int i = 0; i < 12; i++)
            if (!op.buf[i]) return fail(YUUKA_ERR_INVALID_ARGUMENT, "recurrent chunk buffer %d is null", i);
        const uint64_t R = (uint64_t)g.rows * g.nreq, nq = (uint64_t)g.nreq;
        if (g.nreq > 1 && (!(op.flags & YUUKA_EXT_FLAG_DEFER) || !(op.flags & YUUKA_EXT_FLAG_RAW_OUT) || g.rows > 32))
            return fail(YUUKA_ERR_UNSUPPORTED, "recurrent chunk: several requests need deferred raw outputs, <= 32 rows");
        if (!buf_ok(op.buf[0], op.off[0], nq * (g.kernel - 1) * g.conv_dim * 4) ||
            !buf_ok(op.buf[1], op.off[1], nq * g.rank * g.state * g.state * 4) ||
            !buf_ok(op.buf[2], op.off[2], R * g.conv_dim * 4) || !buf_ok(op.buf[3], op.off[3], R * g.inner * 4) ||
            !buf_ok(op.buf[4], op.off[4], R * g.rank * 4) || !buf_ok(op.buf[5], op.off[5], R * g.rank * 4) ||
            !buf_ok(op.buf[10], op.off[10], R * g.inner * 4) || !buf_ok(op.buf[11], op.off[11], R * g.conv_dim * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "recurrent chunk buffers too small");
        if ((op.flags & YUUKA_EXT_FLAG_RAW_OUT) && (!(op.flags & YUUKA_EXT_FLAG_DEFER) || g.rows > 32))
            return fail(YUUKA_ERR_UNSUPPORTED, "recurrent chunk: raw outputs need the deferred mode and <= 32 rows");
        *ws = R * g.inner * 4;  // raw per-head outputs before the gated norm
        return YUUKA_OK;
    }
    case YUUKA_EXT_OP_QUANTIZE_X: {
        const uint64_t K = op.n[0], rows = op.n[1];
        const uint64_t need = rows >= 1 && rows <= 16 && K && K % 256 == 0 ? gemm_plan(K, 1, rows, YUUKA_DTYPE_Q4_K).xq_bytes : 0;
        if (!need || op.off[0] % 16 || op.off[1] % 16 || !buf_ok(op.buf[0], op.off[0], K * rows * 4) ||
            !buf_ok(op.buf[1], op.off[1], need))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid QUANTIZE_X shape or buffers");
        return YUUKA_OK;
    }
    case YUUKA_EXT_OP_GEMM_Q: {
        const uint64_t K = op.n[0], N = op.n[1], rows = op.n[2];
        yuuka_status st = check_verify_gemm(K, N, rows, op.u[0], 16);
        if (st != YUUKA_OK) return st;
        const GemmPlan p = gemm_plan(K, N, rows, op.u[0]);
        if (op.off[0] % 16 || op.off[1] % 16 || !buf_ok(op.buf[0], op.off[0], row_bytes(op.u[0], K) * N) ||
            !buf_ok(op.buf[1], op.off[1], p.xq_bytes) || !buf_ok(op.buf[2], op.off[2], N * rows * 4) ||
            (op.buf[3] && !buf_ok(op.buf[3], op.off[3], N * rows * 4)))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid GEMM_Q buffers");
        *ws = p.part_bytes + 256;
        return YUUKA_OK;
    }
    case YUUKA_EXT_OP_GEMM_FUSED: {
        const uint64_t K = op.n[0], rows = op.n[1];
        const int nseg = fused_segments(op);
        const uint32_t epi = op.u[1];
        if (!K || K % 256 || K > 65536 || rows < 1 || rows > 512 || nseg == 0 || epi > kEpiSwiglu ||
            (epi == kEpiSwiglu && nseg != 2) || op.off[0] % 16 || op.off[1] % 16 ||
            !buf_ok(op.buf[0], op.off[0], K * rows * 4) || (op.buf[1] && !buf_ok(op.buf[1], op.off[1], K * 4)))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid GEMM_FUSED shape or activation buffers");
        for (int i = 0; i < nseg; i++) {
            const uint32_t dt = (op.u[0] >> (8 * i)) & 0xff;
            const uint64_t N = op.n[2 + i];
            if (dt != YUUKA_DTYPE_Q4_K && dt != YUUKA_DTYPE_Q6_K)
                return fail(YUUKA_ERR_UNSUPPORTED, "GEMM_FUSED segment %d: dtype %u (Q4_K and Q6_K only)", i, dt);
            const uint64_t wb = row_bytes(dt, K) * N;
            if (!N || N > (1u << 24) || wb >= (1ull << 32) || !buf_ok(op.buf[2 + i], op.off[2 + i], wb) ||
                (dt == YUUKA_DTYPE_Q4_K && op.off[2 + i] % 16) || op.off[2 + i] % 4)
                return fail(YUUKA_ERR_INVALID_ARGUMENT, "GEMM_FUSED segment %d: weight buffer", i);
            const bool writes = epi != kEpiSwiglu || i == 0;
            if (writes && !buf_ok(op.buf[6 + i], op.off[6 + i], N * rows * 4))
                return fail(YUUKA_ERR_INVALID_ARGUMENT, "GEMM_FUSED segment %d: output buffer", i);
            if (epi == kEpiResidual && !buf_ok(op.buf[10 + i], op.off[10 + i], N * rows * 4))
                return fail(YUUKA_ERR_INVALID_ARGUMENT, "GEMM_FUSED segment %d: residual buffer", i);
        }
        if (epi == kEpiSwiglu && (op.n[2] != op.n[3] || (op.u[0] & 0xff) != ((op.u[0] >> 8) & 0xff)))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "GEMM_FUSED SwiGLU: gate and up must match");
        if (op.buf[14] && (op.buf[1] || !buf_ok(op.buf[14], op.off[14], K * rows * 4) ||
                           !buf_ok(op.buf[15], op.off[15], 128 * 4) || K % 128 || op.off[14] % 16 || op.off[15] % 16))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "GEMM_FUSED gated head norm: buffers (and no RMSNorm weight)");
        if (op.u[2] && epi != kEpiStore)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "GEMM_FUSED: output maps need the store epilogue");
        for (int i = 0; i < nseg; i++) {
            const uint32_t act = (op.u[2] >> (4 * i)) & 0xfu;
            if (act > 3) return fail(YUUKA_ERR_INVALID_ARGUMENT, "GEMM_FUSED segment %d: output map %u", i, act);
            if (act == 3 && !buf_ok(op.buf[10 + i], op.off[10 + i], 2 * op.n[2 + i] * 4))
                return fail(YUUKA_ERR_INVALID_ARGUMENT, "GEMM_FUSED segment %d: decay parameters {dt, a}", i);
        }
        if (fused_many_rows(op)) {  // k_bgemm.hip: quantized rows in the workspace
            if (K > 16384) return fail(YUUKA_ERR_UNSUPPORTED, "GEMM_FUSED: K %llu over 16384 rows > 8",
                                       (unsigned long long)K);
            int nn[kFusedMaxSeg] = {0, 0, 0, 0};
            for (int i = 0; i < nseg; i++) nn[i] = (int)op.n[2 + i];
            *ws = fused_gemm_rows_ws((int)rows, (int)K, nn, nseg, epi == kEpiSwiglu);
            return YUUKA_OK;
        }
        if (fused_gemm_chunk_sb((int)rows, (int)K, fused_tiles(op, nseg), op.buf[1] != nullptr, op.buf[14] != nullptr) < 1)
            return fail(YUUKA_ERR_UNSUPPORTED, "GEMM_FUSED: activations do not fit LDS");
        return YUUKA_OK;
    }
    case YUUKA_EXT_OP_ACCEPT: {
        yuuka_accept_params p{};
        p.mode = op.u[0];
        p.batch = (uint32_t)op.n[0];
        p.drafts = (uint32_t)op.n[1];
        p.vocab = (uint32_t)op.n[2];
        p.row_stride = op.n[3];
        if ((p.mode != YUUKA_ACCEPT_GREEDY && p.mode != YUUKA_ACCEPT_STOCHASTIC) || !p.batch || !p.vocab ||
            p.drafts > 255 || (op.u[3] && op.u[3] < p.drafts))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid ACCEPT parameters");
        const uint64_t dstride = op.u[3] ? op.u[3] : p.drafts;
        if (op.buf[5] && !buf_ok(op.buf[5], op.off[5], (uint64_t)p.batch * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "ACCEPT forced lengths buffer too small");
        if (p.mode == YUUKA_ACCEPT_STOCHASTIC && !(op.f[1] >= 0.0f && op.f[1] <= 1.0f))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "ACCEPT: top-p must be in [0,1]");
        const uint64_t stride = p.row_stride ? p.row_stride : p.vocab;
        const uint64_t rows = (uint64_t)p.batch * (p.drafts + 1);
        if (!buf_ok(op.buf[0], op.off[0], ((rows - 1) * stride + p.vocab) * 4) ||
            (p.drafts && !buf_ok(op.buf[1], op.off[1], ((uint64_t)p.batch - 1) * dstride * 4 + p.drafts * 4)) ||
            !buf_ok(op.buf[2], op.off[2], (uint64_t)p.batch * 16))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "ACCEPT buffers too small");
        *ws = accept_scratch_bytes(p);
        return YUUKA_OK;
    }
    case YUUKA_EXT_OP_GDN_COMMIT: {
        const GdnArgs g = gdn_args(op);
        yuuka_status st = check_gdn(g, "GDN commit");
        if (st != YUUKA_OK) return st;
        for (int i = 0; i < 9; i++)
            if (!op.buf[i]) return fail(YUUKA_ERR_INVALID_ARGUMENT, "GDN commit buffer %d is null", i);
        if (g.nreq > 1 && g.rows > 32)
            return fail(YUUKA_ERR_UNSUPPORTED, "GDN commit: several requests need <= 32 rows");
        const uint64_t nq = (uint64_t)g.nreq, R = nq * g.rows;
        if (!buf_ok(op.buf[0], op.off[0], nq * (g.kernel - 1) * g.conv_dim * 4) ||
            !buf_ok(op.buf[1], op.off[1], nq * g.rank * g.state * g.state * 4) ||
            !buf_ok(op.buf[2], op.off[2], R * g.conv_dim * 4) || !buf_ok(op.buf[3], op.off[3], R * g.conv_dim * 4) ||
            !buf_ok(op.buf[4], op.off[4], R * g.rank * 4) || !buf_ok(op.buf[5], op.off[5], R * g.rank * 4) ||
            !buf_ok(op.buf[8], op.off[8], nq * 16))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "GDN commit buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_OP_MOE_ROUTE: {  // hip.go:1585-1608: n={rows, experts, used}
        const uint64_t rows = op.n[0], E = op.n[1], used = op.n[2];
        if (!rows || !E || !used || used > E)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid MoE route dimensions");
        if (E > 1024 || used > 64 || rows * used > 4096)
            return fail(YUUKA_ERR_UNSUPPORTED, "MoE route: %llu experts, %llu used, %llu rows (<= 1024, 64, 4096 "
                        "assignments are served)", (unsigned long long)E, (unsigned long long)used,
                        (unsigned long long)rows);
        const uint64_t a = E * rows * used * 4;
        if (!buf_ok(op.buf[0], op.off[0], rows * E * 4) || !buf_ok(op.buf[1], op.off[1], rows * used * 4) ||
            !buf_ok(op.buf[2], op.off[2], rows * used * 4) || !buf_ok(op.buf[3], op.off[3], E * 4) ||
            !buf_ok(op.buf[4], op.off[4], a) || !buf_ok(op.buf[5], op.off[5], a) || !buf_ok(op.buf[6], op.off[6], a))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "MoE route buffers too small");
        for (int i = 0; i < 7; i++)
            if (op.off[i] % 4) return fail(YUUKA_ERR_INVALID_ARGUMENT, "MoE route buffer %d misaligned", i);
        return YUUKA_OK;
    }
    case YUUKA_OP_MOE_GATE_UP:    // hip.go:1610-1642: n={hidden, ffn, rows, experts, used}
    case YUUKA_OP_MOE_DOWN: {     // hip.go:1644-1670: n={ffn, hidden, rows, experts, used}
        const bool gu = op.code == YUUKA_OP_MOE_GATE_UP;
        const uint64_t K = op.n[0], N = op.n[1], rows = op.n[2], E = op.n[3], used = op.n[4];
        if (!K || !N || !rows || !E || !used || used > E)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid MoE %s dimensions", gu ? "gate/up" : "down");
        if (op.u[0] != YUUKA_DTYPE_Q4_K)
            return fail(YUUKA_ERR_UNSUPPORTED, "MoE expert dtype %u (Q4_K is served)", op.u[0]);
        if (K % 256 || N % 16 || K > 8192)
            return fail(YUUKA_ERR_UNSUPPORTED, "MoE expert shape %llu x %llu", (unsigned long long)N,
                        (unsigned long long)K);
        // shared: expert E is the shared expert (weights of E + 1 experts), and
        // the activation (down) and output rows have used + 1 slots
        const uint64_t sh = (op.flags & YUUKA_EXT_FLAG_MOE_SHARED) ? 1 : 0, os = used + sh;
        if (rows > 512 || E + sh > 1024 || E + 1 + rows * os / 8 > 2048)
            return fail(YUUKA_ERR_UNSUPPORTED, "MoE %s: %llu rows of %llu experts (at most 512 rows, 1024 experts)",
                        gu ? "gate/up" : "down", (unsigned long long)rows, (unsigned long long)E);
        const uint64_t rb = row_bytes(op.u[0], K), wb = (E + sh) * N * rb, a = E * rows * used * 4;
        const uint64_t x_rows = gu ? rows : rows * os;
        const bool swiglu = gu && (op.flags & YUUKA_EXT_FLAG_MOE_SWIGLU);
        const int ib = gu ? 3 : 2;  // counts, assign_rows, assign_slots, out...
        bool ok = buf_ok(op.buf[0], op.off[0], x_rows * K * 4) && buf_ok(op.buf[1], op.off[1], wb) &&
                  (!gu || buf_ok(op.buf[2], op.off[2], wb)) && buf_ok(op.buf[ib], op.off[ib], E * 4) &&
                  buf_ok(op.buf[ib + 1], op.off[ib + 1], a) && buf_ok(op.buf[ib + 2], op.off[ib + 2], a) &&
                  buf_ok(op.buf[ib + 3], op.off[ib + 3], rows * os * N * 4) &&
                  (!gu || swiglu || buf_ok(op.buf[ib + 4], op.off[ib + 4], rows * os * N * 4));
        if (!ok) return fail(YUUKA_ERR_INVALID_ARGUMENT, "MoE %s buffers too small", gu ? "gate/up" : "down");
        if (op.off[0] % 16 || op.off[1] % 16 || (gu && op.off[2] % 16))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "MoE activations and weights must be 16-byte aligned");
        *ws = moe_gemm_ws((int)x_rows, (int)K);
        return YUUKA_OK;
    }
    case YUUKA_OP_MOE_REDUCE_ADD: {  // hip.go:1672-1690: n={hidden, rows, used}
        const uint64_t H = op.n[0], rows = op.n[1], used = op.n[2];
        if (!H || !rows || !used) return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid MoE reduce dimensions");
        if (!buf_ok(op.buf[0], op.off[0], rows * H * 4) || !buf_ok(op.buf[1], op.off[1], rows * used * H * 4) ||
            !buf_ok(op.buf[2], op.off[2], rows * used * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "MoE reduce buffers too small");
        return YUUKA_OK;
    }
    case YUUKA_EXT_OP_MOE_ROUTER: {
        const uint64_t H = op.n[0], E = op.n[1], rows = op.n[2];
        if (!H || !E || !rows || H % 4) return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid MoE router dimensions");
        if (!buf_ok(op.buf[0], op.off[0], rows * H * 4) || !buf_ok(op.buf[1], op.off[1], E * H * 4) ||
            !buf_ok(op.buf[2], op.off[2], rows * E * 4) ||
            (op.buf[3] && (!buf_ok(op.buf[3], op.off[3], H * 4) || !buf_ok(op.buf[4], op.off[4], rows * 4))))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "MoE router buffers too small");
        if (op.off[0] % 16 || op.off[1] % 16 || (op.buf[3] && op.off[3] % 16))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "MoE router inputs must be 16-byte aligned");
        return YUUKA_OK;
    }
    case YUUKA_EXT_OP_MOE_COMBINE: {
        const uint64_t H = op.n[0], rows = op.n[1], used = op.n[2];
        if (!H || !rows || !used) return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid MoE combine dimensions");
        const bool sh = (op.flags & YUUKA_EXT_FLAG_MOE_SHARED) != 0;  // shared output in eo slot `used`
        if (!buf_ok(op.buf[0], op.off[0], rows * H * 4) || !buf_ok(op.buf[1], op.off[1], rows * (used + sh) * H * 4) ||
            !buf_ok(op.buf[2], op.off[2], rows * used * 4) ||
            (op.buf[3] && !buf_ok(op.buf[3], op.off[3], rows * H * 4)) ||
            ((op.buf[3] || sh) && !buf_ok(op.buf[4], op.off[4], rows * 4)))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "MoE combine buffers too small");
        if (sh && op.buf[3]) return fail(YUUKA_ERR_INVALID_ARGUMENT, "MoE combine: shared output in eo and buf3");
        return YUUKA_OK;
    }
    case YUUKA_EXT_OP_ADVANCE: {
        const uint64_t nq = op.u[0] ? op.u[0] : 1;
        if (nq > 1024 || !buf_ok(op.buf[0], op.off[0], 8 * nq) || op.off[0] % 4 ||
            !buf_ok(op.buf[1], op.off[1], 16 * (nq - 1) + 8) || op.n[0] == 0 ||
            (op.buf[2] && !buf_ok(op.buf[2], op.off[2], 8)))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid ADVANCE buffers or request count");
        return YUUKA_OK;
    }
    default:
        return fail(YUUKA_ERR_UNSUPPORTED, "plan op code %u is not served by this library", op.code);
    }
}

bool gemm_chain_member(const yuuka_op &op) { return op.code == YUUKA_EXT_OP_GEMM_FUSED && fused_many_rows(op); }


bool gemm_chain_ws(const yuuka_op &op, uint64_t *quant, uint64_t *part) {
    if (!gemm_chain_member(op)) return false;
    const int nseg = fused_segments(op);
    int nn[kFusedMaxSeg] = {0, 0, 0, 0};
    for (int i = 0; i < nseg; i++) nn[i] = (int)op.n[2 + i];
    fused_gemm_rows_ws_parts((int)op.n[1], (int)op.n[0], nn, nseg, op.u[1] == kEpiSwiglu, quant, part);
    return true;
}

yuuka_status execute_gemm_chain(const yuuka_op *ops, int n, const yuuka_op *after, const ExecCtx &ctx,
                                bool *after_done) {
    *after_done = false;
    std::vector<FusedGemmArgs> g(n);
    for (int i = 0; i < n; i++) g[i] = fused_args(ops[i]);
    // the last member's split reduction inside the next op's RMSNorm of its
    // output (the MoE FFN norm after the out-projection)
    const yuuka_op &l = ops[n - 1];
    const FusedGemmArgs &la = g[n - 1];
    const bool norm_next = after && after->code == YUUKA_OP_RMSNORM_BATCH && la.nseg == 1 &&
                           la.epilogue == kEpiResidual && after->buf[0] == l.buf[6] && after->off[0] == l.off[6] &&
                           after->n[0] == (uint64_t)la.seg[0].n && after->n[1] == (uint64_t)la.rows &&
                           after->n[2] == after->n[0] &&
                           (after->n[0] == 1024 || after->n[0] == 2048 || after->n[0] == 4096);
    BgDeferred last{};
    hipError_t err = launch_fused_gemm_rows_chain(g.data(), n, ctx.ws, ctx.part_off, norm_next, ctx.stream, &last);
    if (err == hipSuccess && last.on) {
        err = launch_reduce_rmsnorm_rows(last.part, last.sstride, last.splits, la.seg[0].res, la.seg[0].out,
                                         at<const float>(*after, 1), at<float>(*after, 2), (int)after->n[0],
                                         (int)after->n[1], after->n[3], after->f[0], ctx.stream);
        *after_done = true;
    }
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "GEMM_FUSED run launch: %s", hip_error(err));
    return YUUKA_OK;
}

int gdn_commit_run(const yuuka_op *ops, int count) {
    if (count < 2 || ops[0].code != YUUKA_EXT_OP_GDN_COMMIT) return 1;
    const GdnArgs g0 = gdn_args(ops[0]);
    if (g0.rows > 32) return 1;
    int n = 1;
    while (n < count && n < kGdnCommitMaxLayers && ops[n].code == YUUKA_EXT_OP_GDN_COMMIT &&
           ops[n].flags == ops[0].flags && ops[n].buf[8] == ops[0].buf[8] && ops[n].off[8] == ops[0].off[8]) {
        const GdnArgs g = gdn_args(ops[n]);
        if (g.rows != g0.rows || g.nreq != g0.nreq || g.groups != g0.groups || g.rank != g0.rank || g.state != g0.state ||
            g.conv_dim != g0.conv_dim || g.inner != g0.inner || g.kernel != g0.kernel || g.coef != g0.coef)
            break;
        n++;
    }
    return n;
}

yuuka_status execute_gdn_commit_run(const yuuka_op *ops, int count, const ExecCtx &ctx) {
    const GdnArgs g = gdn_args(ops[0]);
    GdnCommitSet set{};
    for (int i = 0; i < count; i++) {
        const yuuka_op &op = ops[i];
        set.layer[i] = GdnCommitLayer{at<float>(op, 0),       at<float>(op, 1),       at<const float>(op, 2),
                                      at<const float>(op, 3), at<const float>(op, 4), at<const float>(op, 5),
                                      at<const float>(op, 6), at<const float>(op, 7)};
    }
    const hipError_t err = launch_gdn_commit_cols_multi(set, count, g, at<const int32_t>(ops[0], 8), ctx.stream);
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "GDN commit launch: %s", hip_error(err));
    return YUUKA_OK;
}

yuuka_status execute_model_op(const yuuka_op &op, const ExecCtx &ctx) {
    bool decode = false;
    const yuuka_status dst = execute_decode_op(op, ctx, &decode);
    if (decode) return dst;
    hipError_t err = hipSuccess;
    const hipStream_t s = ctx.stream;
    switch (op.code) {
    case YUUKA_OP_ADD:
        err = launch_add_f32(at<float>(op, 0), at<const float>(op, 0), at<const float>(op, 1), op.n[0], s);
        break;
    case YUUKA_OP_COPY:
        err = launch_copy_f32(at<float>(op, 0), at<const float>(op, 1), op.n[0], s);
        break;
    case YUUKA_OP_SILU_MUL:
        err = launch_silu_mul(at<const float>(op, 0), at<const float>(op, 1), at<float>(op, 2), op.n[0], s);
        break;
    case YUUKA_OP_EMBEDDING_BATCH:
        err = launch_embedding(at<const uint8_t>(op, 0), op.u[0], op.n[2], at<const int32_t>(op, 2), (int)op.n[3],
                               (int)op.n[0], (int)op.n[1], at<float>(op, 1), s);
        break;
    case YUUKA_OP_RMSNORM_BATCH:
        err = launch_rmsnorm_rows(at<const float>(op, 0), at<const float>(op, 1), at<float>(op, 2), (int)op.n[0],
                                  (int)op.n[1], op.n[2], op.n[3], op.f[0], s);
        break;
    case YUUKA_OP_RMSNORM_HEADS_BATCH:
        err = launch_rmsnorm_heads(at<const float>(op, 0), at<const float>(op, 1), at<float>(op, 2), (int)op.n[0],
                                   (int)op.n[1], (int)op.n[2], (int)op.n[3], op.f[0], s);
        break;
    case YUUKA_OP_ROPE_BATCH:
        err = launch_rope(at<float>(op, 0), (int)op.n[0], (int)op.n[1], (int)op.n[3], (int)op.n[4], op.n[5],
                          (double)op.f[0], dyn_of(ctx), (int)op.u[0], s);
        break;
    case YUUKA_OP_KV_WRITE_BATCH_PAGED: {
        bool ok;
        err = launch_kv_write(at<const float>(op, 0), at<const float>(op, 1), at<uint8_t>(op, 2), at<uint8_t>(op, 3),
                              at<const int32_t>(op, 4), (int)op.n[0], (int)op.n[1], (int)op.u[0], kv_fmt(op.u[2], &ok),
                              dyn_of(ctx), 0, s);
        break;
    }
    case YUUKA_OP_ATTENTION_PREFILL_PAGED: {
        const AttnArgs a = attn_args(op);
        const bool own = (op.flags & YUUKA_EXT_FLAG_OWN_POS) != 0;
        const int hint = ctx.dyn || own ? -1 : (int)ctx.position + a.displacement + a.rows - 1;
        err = launch_attention(at<const float>(op, 0), at<const uint8_t>(op, 1), at<const uint8_t>(op, 2),
                               at<const int32_t>(op, 4), at<float>(op, 3), a, ctx.ws, dyn_of(ctx), hint, s);
        break;
    }
    case YUUKA_EXT_OP_ROUTER_NORMAL:
        err = launch_router_normal(at<float>(op, 0), (int)op.n[0], (int)op.n[1], op.n[2], (uint32_t)op.n[3],
                                   at<const uint64_t>(op, 1), s);
        break;
    case YUUKA_EXT_OP_ROPE_TABLE:
        err = launch_rope_table(at<float2>(op, 0), (int)op.n[0], (int)op.n[1], (double)op.f[0], dyn_of(ctx, op),
                                (int)op.n[2], s, op.n[3] ? (int)op.n[3] : 1,
                                (int)(op.n[4] > op.n[0] ? op.n[4] : op.n[0]));
        break;
    case YUUKA_EXT_OP_ATTN_VERIFY: {
        const AttnVArgs a = attnv_args(op);
        const bool own = (op.flags & YUUKA_EXT_FLAG_OWN_POS) != 0;
        const int hint = ctx.dyn || own ? -1 : (int)ctx.position + a.displacement + a.rows - 1;
        err = launch_attn_verify(at<const float>(op, 0), at<const float>(op, 1), at<const float>(op, 2),
                                 at<uint8_t>(op, 3), at<uint8_t>(op, 4), at<const int32_t>(op, 6),
                                 at<const float>(op, 7), at<const float>(op, 8), at<const float2>(op, 9),
                                 at<float>(op, 5), a, ctx.ws, dyn_of(ctx, op), hint, s);
        break;
    }
    case YUUKA_OP_RECURRENT_CHUNK: {
        const GdnArgs g = gdn_args(op);
        const bool defer = (op.flags & YUUKA_EXT_FLAG_DEFER) != 0;
        float *conv = at<float>(op, 11);
        float *raw = static_cast<float *>(ctx.ws);
        if (defer && (op.flags & YUUKA_EXT_FLAG_RAW_OUT) && g.rows <= 32) {  // column-split scan (k_gdn.hip)
            err = launch_gdn_verify_cols(at<const float>(op, 0), at<const float>(op, 1), at<const float>(op, 2),
                                         at<const float>(op, 4), at<const float>(op, 5), at<const float>(op, 6),
                                         at<const float>(op, 7), at<const float>(op, 8), at<float>(op, 10), conv, g, s);
            break;
        }
        if (defer && g.rows <= 16) {  // one fused kernel per layer (k_gdn.hip)
            err = launch_gdn_verify(at<const float>(op, 0), at<const float>(op, 1), at<const float>(op, 2),
                                    at<const float>(op, 3), at<const float>(op, 4), at<const float>(op, 5),
                                    at<const float>(op, 6), at<const float>(op, 7), at<const float>(op, 8),
                                    at<const float>(op, 9), at<float>(op, 10), conv, g, s);
            break;
        }
        err = launch_gdn_conv(at<const float>(op, 0), at<const float>(op, 2), at<const float>(op, 6), conv, g, s);
        if (err == hipSuccess)
            err = launch_gdn_scan(at<float>(op, 1), conv, at<const float>(op, 4), at<const float>(op, 5),
                                  at<const float>(op, 7), at<const float>(op, 8), raw, g, defer ? 0 : 2, nullptr, s);
        if (err == hipSuccess && !defer)
            err = launch_gdn_conv_commit(at<float>(op, 0), at<const float>(op, 2), g, nullptr, s);
        if (err == hipSuccess)
            err = launch_gdn_norm_gate(raw, at<const float>(op, 3), at<const float>(op, 9), at<float>(op, 10), g, s);
        break;
    }
    case YUUKA_EXT_OP_QUANTIZE_X:
        err = launch_quantize_x(at<const float>(op, 0), op.n[0], op.n[1], at<uint8_t>(op, 1), s);
        break;
    case YUUKA_EXT_OP_GEMM_Q: {
        const GemmPlan p = gemm_plan(op.n[0], op.n[1], op.n[2], op.u[0]);
        err = launch_gemm_q(at<const uint8_t>(op, 0), op.u[0], at<const uint8_t>(op, 1), at<float>(op, 2), op.n[0],
                            op.n[1], op.n[2], p, ctx.ws, nullptr, s, at<const float>(op, 3));
        break;
    }
    case YUUKA_EXT_OP_GEMM_FUSED: {
        FusedGemmArgs a = fused_args(op);
        if (fused_many_rows(op)) {
            err = launch_fused_gemm_rows(a, ctx.ws, s);
            break;
        }
        const int tt = fused_tiles(op, a.nseg);
        a.chunk_sb = fused_gemm_chunk_sb(a.rows, a.K, tt, a.norm != nullptr, a.gate != nullptr);
        err = launch_fused_gemm(a, tt, s);
        break;
    }
    case YUUKA_EXT_OP_ACCEPT: {
        yuuka_accept_params p{};
        p.mode = op.u[0];
        p.batch = (uint32_t)op.n[0];
        p.drafts = (uint32_t)op.n[1];
        p.vocab = (uint32_t)op.n[2];
        p.row_stride = op.n[3];
        p.seed = op.n[4];
        p.step = op.n[5];
        p.top_k = op.u[1];
        p.request_base = op.u[2];
        p.temperature = op.f[0];
        p.top_p = op.f[1];
        err = launch_verify_accept(at<const float>(op, 0), at<const int32_t>(op, 1), at<int32_t>(op, 2),
                                   at<double>(op, 3), p, ctx.ws, s, at<const uint64_t>(op, 4), op.u[3],
                                   at<const int32_t>(op, 5));
        break;
    }
    case YUUKA_EXT_OP_GDN_COMMIT: {
        const GdnArgs g = gdn_args(op);
        const int32_t *res = at<const int32_t>(op, 8);
        if (g.rows <= 32) {  // scan replay + conv window, column-split (k_gdn.hip)
            err = launch_gdn_commit_cols(at<float>(op, 0), at<float>(op, 1), at<const float>(op, 2), at<const float>(op, 3),
                                    at<const float>(op, 4), at<const float>(op, 5), at<const float>(op, 6),
                                    at<const float>(op, 7), g, res, s);
            break;
        }
        err = launch_gdn_scan(at<float>(op, 1), at<const float>(op, 3), at<const float>(op, 4), at<const float>(op, 5),
                              at<const float>(op, 6), at<const float>(op, 7), nullptr, g, 1, res, s);
        if (err == hipSuccess) err = launch_gdn_conv_commit(at<float>(op, 0), at<const float>(op, 2), g, res, s);
        break;
    }
    case YUUKA_OP_MOE_ROUTE:
        err = launch_moe_route(at<const float>(op, 0), (int)op.n[0], (int)op.n[1], (int)op.n[2], at<int32_t>(op, 1),
                               at<float>(op, 2), at<int32_t>(op, 3), at<int32_t>(op, 4), at<int32_t>(op, 5),
                               at<float>(op, 6), s);
        break;
    case YUUKA_OP_MOE_GATE_UP:
    case YUUKA_OP_MOE_DOWN: {
        const bool gu = op.code == YUUKA_OP_MOE_GATE_UP;
        const int ib = gu ? 3 : 2;
        MoeGemm g{};
        g.x = at<const float>(op, 0);
        g.w0 = at<const void>(op, 1);
        g.w1 = gu ? at<const void>(op, 2) : nullptr;
        g.row_bytes = row_bytes(op.u[0], op.n[0]);
        g.counts = at<const int32_t>(op, ib);
        g.arows = at<const int32_t>(op, ib + 1);
        g.aslots = at<const int32_t>(op, ib + 2);
        g.K = (int)op.n[0];
        g.N = (int)op.n[1];
        g.rows = (int)op.n[2];
        g.experts = (int)op.n[3];
        g.used = (int)op.n[4];
        g.by_slot = gu ? 0 : 1;
        g.swiglu = gu && (op.flags & YUUKA_EXT_FLAG_MOE_SWIGLU) ? 1 : 0;
        g.packed = (op.flags & YUUKA_EXT_FLAG_MOE_PACKED) ? 1 : 0;
        g.shared = (op.flags & YUUKA_EXT_FLAG_MOE_SHARED) ? 1 : 0;
        g.out0 = at<float>(op, ib + 3);
        g.out1 = gu ? at<float>(op, ib + 4) : nullptr;
        err = launch_moe_gemm(g, ctx.ws, s);
        break;
    }
    case YUUKA_OP_MOE_REDUCE_ADD:
        err = launch_moe_combine(at<float>(op, 0), at<const float>(op, 1), at<const float>(op, 2), (int)op.n[1],
                                 (int)op.n[2], (int)op.n[0], nullptr, nullptr, s);
        break;
    case YUUKA_EXT_OP_MOE_ROUTER:
        err = launch_moe_router(at<const float>(op, 0), (int)op.n[0], (int)op.n[2], at<const float>(op, 1),
                                (int)op.n[1], at<float>(op, 2), at<const float>(op, 3), at<float>(op, 4), s);
        break;
    case YUUKA_EXT_OP_MOE_COMBINE:
        err = launch_moe_combine(at<float>(op, 0), at<const float>(op, 1), at<const float>(op, 2), (int)op.n[1],
                                 (int)op.n[2], (int)op.n[0], at<const float>(op, 3), at<const float>(op, 4), s,
                                 (op.flags & YUUKA_EXT_FLAG_MOE_SHARED) != 0);
        break;
    case YUUKA_EXT_OP_ADVANCE: {
        ModelDyn d{at<int32_t>(op, 0) + 1, 0};
        err = launch_advance(d, at<const int32_t>(op, 1), (int)op.n[0], at<uint64_t>(op, 2), op.u[0] ? (int)op.u[0] : 1, s);
        break;
    }
    default:
        return fail(YUUKA_ERR_UNSUPPORTED, "plan op code %u is not served by this library", op.code);
    }
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "op %u launch: %s", op.code, hip_error(err));
    return YUUKA_OK;
}

}  // namespace yk
