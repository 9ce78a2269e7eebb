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

bool op_uses_position(const yuuka_op &op) {
    switch (op.code) {
    case YUUKA_OP_ROPE_BATCH:
    case YUUKA_OP_KV_WRITE_BATCH_PAGED:
    case YUUKA_OP_ATTENTION_PREFILL_PAGED:
    case YUUKA_EXT_OP_ROPE_TABLE:
    case YUUKA_EXT_OP_ATTN_VERIFY:
        return !(op.flags & YUUKA_EXT_FLAG_OWN_POS);
    default:
        return false;
    }
}

yuuka_status validate_model_op(const yuuka_op &op, uint64_t *ws) {
    *ws = 0;
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
