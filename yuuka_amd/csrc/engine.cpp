// engine.cpp — qwen35 / qwen35moe verify engine: the host side of the
// speculative verify path, in C++ over this library's own plan API.
//
// Counterparts in the reference: engine/gpu/runtime.go + session.go (weights
// and per-request state on the device, PrefillLogits, Snapshot/Restore),
// engine/gpu/plan.go:569-988 (buildPrefillPlan and the per-layer blocks),
// model/qwen35/forward.go:320-439 (the MoE FFN), memory/memory.go and
// memory/prefix.go (paged KV tables over a shared pool, prefix sharing by
// reference count) and engine/speculative.go:68-261 (generateSpeculative).
// Differences by design:
//  * a step covers the k+1 rows {pending token, d1..dk} of every active
//    request; the dense projections run over all rows at once, attention and
//    the recurrent scan per request (own position, block table and state);
//  * the step ends with the fused acceptance of every request and commits
//    only each request's accepted prefix of the recurrent state on the
//    device (GDN_COMMIT), then advances the device positions, so no
//    snapshot / restore / replay crosses PCIe per step;
//  * every plan is captured once per (requests, rows, mode) into a HIP graph.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <tuple>
#include <vector>

#include "fgemm.h"
#include "internal.h"
#include "model_kernels.h"
#include "plan.h"

namespace {

using yk::fail;

constexpr int kRowBlock = 16;   // rows of one streaming GEMM launch at most
constexpr int kAttnRows = 8;    // query rows of one verify-attention launch (non-MFMA path)

struct Tensor {
    yuuka_buffer *b = nullptr;
    uint64_t rows = 0, cols = 0;
    uint32_t dtype = 0;
};

struct Layer {
    bool recurrent = false;
    bool moe = false;
    yuuka_buffer *attn_norm = nullptr, *post_norm = nullptr;
    Tensor qkv, gate, out, beta, alpha, q, k, v, o, ffn_gate, ffn_up, ffn_down;
    Tensor router, shared_gate, shared_up, shared_down, gate_exps, up_exps, down_exps;
    yuuka_buffer *shared_gate_vec = nullptr;
    yuuka_buffer *conv = nullptr, *dt = nullptr, *a = nullptr, *ssm_norm = nullptr, *q_norm = nullptr,
                 *k_norm = nullptr;
    yuuka_buffer *dt_a = nullptr;  // {dt[rank], a[rank]}: decay parameters of the projection epilogue
    // per-request state, request-major: [batch][...]
    yuuka_buffer *conv_state = nullptr, *mat_state = nullptr;
    uint64_t conv_bytes = 0, mat_bytes = 0;  // one request's slice
    // KV pool shared by the requests (attention layers)
    yuuka_buffer *kpool = nullptr, *vpool = nullptr;
    // per-step saved inputs of the recurrent block (read by GDN_COMMIT), [rows][...]
    yuuka_buffer *qkv_rows = nullptr, *conv_rows = nullptr, *alpha_rows = nullptr, *beta_rows = nullptr;
};

struct Graphs {
    yuuka_plan *plan = nullptr;
    yuuka_graph *graph = nullptr;
};

struct Request {
    std::vector<int32_t> blocks;  // table entries in use
    int32_t pos = 0;              // host mirror of the device position
};

}  // namespace

struct yuuka_q35 {
    yuuka_device *dev = nullptr;
    yuuka_stream *stream = nullptr;
    yuuka_q35_config cfg{};
    int conv_dim = 0;
    int B = 1;           // requests
    int MR = 16;         // rows per request
    int M = 16;          // B * MR rows of the activation buffers
    int max_blocks = 0;  // table entries per request
    std::vector<yuuka_buffer *> owned;
    std::vector<Layer> layers;
    Tensor embedding, output;
    yuuka_buffer *output_norm = nullptr;
    // activations [M][...]
    yuuka_buffer *x = nullptr, *xn = nullptr, *q = nullptr, *k = nullptr, *v = nullptr,
                 *attn = nullptr, *z = nullptr, *gdn_out = nullptr, *fg = nullptr, *fu = nullptr, *logits = nullptr,
                 *rope = nullptr;
    // MoE scratch
    yuuka_buffer *moe_logits = nullptr, *moe_sg = nullptr, *moe_ids = nullptr, *moe_w = nullptr,
                 *moe_counts = nullptr, *moe_arows = nullptr, *moe_aslots = nullptr, *moe_aw = nullptr,
                 *moe_act = nullptr, *moe_eo = nullptr, *moe_sfg = nullptr, *moe_so = nullptr;
    // the shared expert runs inside the grouped GEMMs as expert n_experts
    // (its width equals the experts'): output slot n_experts_used of every row
    bool moe_shared = false;
    // step I/O and per-request device state
    yuuka_buffer *tokens = nullptr, *result = nullptr, *dyn = nullptr, *step = nullptr, *table = nullptr,
                 *forced = nullptr;
    int32_t *pinned = nullptr;  // staging {tokens[M], result[4B], forced[B]}
    hipEvent_t ev0 = nullptr, ev1 = nullptr;  // around the last graph replay
    bool eager = false;  // YUUKA_Q35_EAGER=1: launch plans op by op (profilers), no graphs
    float last_ms = 0.0f;
    // plans keyed by (first request, requests, rows, mode, forced)
    std::map<std::tuple<int, int, int, int, int>, Graphs> plans;
    yuuka_q35_accept accept_cfg{};
    bool accept_set = false;
    int last_rows = 0, last_first = 0, last_nreq = 1;
    // KV block pool
    std::vector<int32_t> refs;
    std::vector<int32_t> free_blocks;
    std::vector<Request> req;
};

namespace {

int32_t *pin_tokens(yuuka_q35 *q) { return q->pinned; }
int32_t *pin_result(yuuka_q35 *q) { return q->pinned + q->M; }
int32_t *pin_forced(yuuka_q35 *q) { return q->pinned + q->M + 4 * q->B; }

yuuka_status alloc(yuuka_q35 *q, uint64_t bytes, yuuka_buffer **out) {
    yuuka_status st = yuuka_buffer_alloc(q->dev, bytes ? bytes : 4, out);
    if (st == YUUKA_OK) q->owned.push_back(*out);
    return st;
}

yuuka_status upload(yuuka_q35 *q, const void *data, uint64_t bytes, yuuka_buffer **out) {
    yuuka_status st = alloc(q, bytes, out);
    if (st == YUUKA_OK && data && bytes) st = yuuka_memcpy_h2d(*out, data, bytes);
    return st;
}

yuuka_status upload_tensor(yuuka_q35 *q, const yuuka_q35_tensor &t, uint64_t rows, uint64_t cols, const char *what,
                           Tensor *out) {
    if (!t.data) return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s: missing data", what);
    if (t.rows != rows || t.cols != cols)
        return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s: shape %llux%llu, want %llux%llu", what,
                    (unsigned long long)t.rows, (unsigned long long)t.cols, (unsigned long long)rows,
                    (unsigned long long)cols);
    const uint64_t rb = yk::row_bytes(t.dtype, cols);
    if (!rb) return fail(YUUKA_ERR_UNSUPPORTED, "%s: dtype %u with %llu columns", what, t.dtype, (unsigned long long)cols);
    out->rows = rows;
    out->cols = cols;
    out->dtype = t.dtype;
    return upload(q, t.data, rb * rows, &out->b);
}

// Expert matrices in the grouped GEMM's packed layout (yuuka_moe_pack_q4k,
// the same bytes rearranged): the v10 layout goes to a staging buffer that
// is rewritten on the device and freed.
// With `extra` (the shared expert, extra_rows rows) that matrix is packed
// after the experts, as expert index rows / expert rows.
yuuka_status upload_experts(yuuka_q35 *q, const yuuka_q35_tensor &t, uint64_t rows, uint64_t cols, const char *what,
                            Tensor *out, const yuuka_q35_tensor *extra = nullptr, uint64_t extra_rows = 0,
                            const char *extra_what = nullptr) {
    const uint64_t rb = yk::row_bytes(t.dtype, cols);
    Tensor staged, staged_x;
    yuuka_status st = upload_tensor(q, t, rows, cols, what, &staged);
    if (st == YUUKA_OK && extra) {
        if (extra->dtype != t.dtype) return fail(YUUKA_ERR_UNSUPPORTED, "%s: dtype %u", extra_what, extra->dtype);
        st = upload_tensor(q, *extra, extra_rows, cols, extra_what, &staged_x);
    }
    if (st != YUUKA_OK) return st;
    *out = staged;
    out->rows = rows + extra_rows;
    st = alloc(q, rb * (rows + extra_rows), &out->b);
    if (st == YUUKA_OK) st = yuuka_moe_pack_q4k(q->stream, out->b, staged.b, rows, cols, nullptr);
    if (st == YUUKA_OK && extra) {
        // the packed layout is tile-major: the extra matrix's tiles follow at
        // the same byte offset as its rows would
        yuuka_buffer view = *out->b;
        view.ptr = static_cast<uint8_t *>(out->b->ptr) + rb * rows;
        view.bytes = rb * extra_rows;
        st = yuuka_moe_pack_q4k(q->stream, &view, staged_x.b, extra_rows, cols, nullptr);
    }
    if (st == YUUKA_OK && hipStreamSynchronize(q->stream->stream) != hipSuccess)
        st = fail(YUUKA_ERR_DEVICE, "%s: packing the experts failed", what);
    for (yuuka_buffer *b : {staged.b, staged_x.b}) {
        if (!b) continue;
        q->owned.erase(std::find(q->owned.begin(), q->owned.end(), b));
        yuuka_buffer_free(b);
    }
    return st;
}

yuuka_status upload_vec(yuuka_q35 *q, const float *v, uint64_t n, const char *what, yuuka_buffer **out) {
    if (!v) return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s: missing data", what);
    return upload(q, v, n * 4, out);
}

// ------------------------------------------------------------ plan build

constexpr uint64_t kMoeRows = 512;  // rows of one grouped-GEMM launch

struct Builder {
    yuuka_plan *plan;
    yuuka_status st = YUUKA_OK;
    void add(uint32_t code, std::initializer_list<yuuka_buffer *> bufs, std::initializer_list<uint64_t> n,
             std::initializer_list<uint32_t> u = {}, std::initializer_list<float> f = {}, uint32_t flags = 0,
             std::initializer_list<uint64_t> offs = {}, yuuka_buffer *own_pos = nullptr, uint64_t own_off = 0) {
        if (st != YUUKA_OK) return;
        yuuka_op op{};
        op.code = code;
        op.flags = flags;
        int i = 0;
        for (auto *b : bufs) op.buf[i++] = b;
        i = 0;
        for (auto v : n) op.n[i++] = v;
        i = 0;
        for (auto v : u) op.u[i++] = v;
        i = 0;
        for (auto v : f) op.f[i++] = v;
        i = 0;
        for (auto v : offs) op.off[i++] = v;
        if (own_pos) {
            op.flags |= YUUKA_EXT_FLAG_OWN_POS;
            op.buf[15] = own_pos;
            op.off[15] = own_off;
        }
        st = yuuka_plan_add(plan, &op);
    }
    struct Seg {
        const Tensor *w;
        yuuka_buffer *out, *res;
    };
    // GEMM_FUSED ops over `rows` activation rows of x (optionally
    // RMS-normalised with `norm`), in launches of at most kRowBlock rows:
    // every segment reads the same rows, outputs are [rows][N_i].
    void fused(yuuka_buffer *x, yuuka_buffer *norm, float eps, uint64_t rows, std::initializer_list<Seg> segs,
               uint32_t epilogue, uint32_t out_map = 0, yuuka_buffer *gate = nullptr,
               yuuka_buffer *head_norm = nullptr) {
        // rows per launch: what the streaming kernel serves for this K and
        // prologue (it reads the weights at verify shapes fastest), else 16
        const uint64_t K0 = segs.begin()->w->cols;
        int per = yk::fused_gemm_stream_rows((int)K0, norm != nullptr, gate != nullptr);
        if (per < 1) per = kRowBlock;
        // more than 8 rows: one launch of the many-row kernel (every weight
        // read once per 64 rows)
        if (rows > 8) per = (int)rows;
        const uint64_t blocks = (rows + per - 1) / per;
        for (uint64_t bi = 0; bi < blocks && st == YUUKA_OK; bi++) {
            // equal blocks (rows 40 -> 8 x 5), so no launch is nearly empty
            const uint64_t r0 = rows * bi / blocks, r1 = rows * (bi + 1) / blocks;
            yuuka_op op{};
            op.code = YUUKA_EXT_OP_GEMM_FUSED;
            op.buf[1] = norm;
            op.buf[15] = head_norm;
            op.u[2] = out_map;
            op.n[1] = r1 - r0;
            op.u[1] = epilogue;
            op.f[0] = eps;
            int i = 0;
            uint64_t K = 0;
            for (const Seg &g : segs) {
                K = g.w->cols;
                op.buf[2 + i] = g.w->b;
                op.buf[6 + i] = g.out;
                op.off[6 + i] = g.out ? r0 * g.w->rows * 4 : 0;
                op.buf[10 + i] = g.res;
                // residual rows (epilogue 1) follow the output rows; the decay
                // parameters of output map 3 are per column, not per row
                op.off[10 + i] = g.res && epilogue == 1 ? r0 * g.w->rows * 4 : 0;
                op.n[2 + i] = g.w->rows;
                op.u[0] |= g.w->dtype << (8 * i);
                i++;
            }
            op.n[0] = K;
            op.buf[0] = x;
            op.off[0] = r0 * K * 4;
            op.buf[14] = gate;
            op.off[14] = gate ? r0 * K * 4 : 0;
            st = yuuka_plan_add(plan, &op);
        }
    }
};

struct PlanKey {
    int first, nreq, rows, mode, forced;
};

// mode 0: verify (acceptance on device), mode 1: commit every row (prefill).
yuuka_status build_plan(yuuka_q35 *q, const PlanKey &key, yuuka_plan **out) {
    const yuuka_q35_config &c = q->cfg;
    yuuka_plan *plan = nullptr;
    yuuka_status st = yuuka_plan_create(q->dev, &plan);
    if (st != YUUKA_OK) return st;
    Builder b{plan};
    const int first = key.first, nreq = key.nreq, mode = key.mode;
    const uint64_t R1 = (uint64_t)key.rows, R = (uint64_t)nreq * R1;
    const uint64_t H = (uint64_t)c.hidden, hd = (uint64_t)c.head_dim;
    const uint64_t qdim = (uint64_t)c.heads * hd * 2, kvdim = (uint64_t)c.kv_heads * hd, odim = (uint64_t)c.heads * hd;
    const uint64_t cd = (uint64_t)q->conv_dim, half = (uint64_t)(c.rope_dim / 2);
    // plan.go:585-588 EMBEDDING_BATCH
    b.add(YUUKA_OP_EMBEDDING_BATCH, {q->embedding.b, q->x, q->tokens},
          {H, R, yk::row_bytes(q->embedding.dtype, H), (uint64_t)c.vocab}, {q->embedding.dtype});
    const float qscale = (float)(1.0 / std::sqrt((double)c.state_size));
    auto dyn_off = [&](int j) { return (uint64_t)(first + j) * 8; };
    // attention: ATTN_VERIFY ops with their own position per request
    bool any_attn = false;
    for (const Layer &L : q->layers) any_attn |= !L.recurrent;
    if (any_attn)  // every request's rotation table in one op (request rows R1 apart)
        b.add(YUUKA_EXT_OP_ROPE_TABLE, {q->rope}, {R1, (uint64_t)c.rope_dim, 0, (uint64_t)nreq, R1}, {},
              {(float)c.rope_base}, 0, {0}, q->dyn, dyn_off(0));
    // the recurrent scan of every request in one op (requests in grid z;
    // states and rows request-major); the split path goes request by request
    auto recurrent = [&](Layer &L, uint32_t extra_flags) {
        const bool together = (extra_flags & YUUKA_EXT_FLAG_RAW_OUT) && R1 <= 32;
        for (int j = 0; j < nreq; j += together ? nreq : 1) {
            const uint64_t r0 = (uint64_t)j * R1, rq = (uint64_t)(first + j);
            b.add(YUUKA_OP_RECURRENT_CHUNK,
                  {L.conv_state, L.mat_state, L.qkv_rows, q->z, L.alpha_rows, L.beta_rows, L.conv, L.dt, L.a,
                   L.ssm_norm, q->gdn_out, L.conv_rows},
                  {R1, (uint64_t)c.groups, (uint64_t)c.rank, (uint64_t)c.state_size, cd, (uint64_t)c.inner},
                  {(uint32_t)c.conv_kernel, together ? (uint32_t)nreq : 1u}, {c.eps, qscale},
                  YUUKA_EXT_FLAG_DEFER | extra_flags,
                  {rq * L.conv_bytes, rq * L.mat_bytes, r0 * cd * 4, r0 * c.inner * 4, r0 * c.rank * 4,
                   r0 * c.rank * 4, 0, 0, 0, 0, r0 * c.inner * 4, r0 * cd * 4});
        }
    };
    auto attention = [&](Layer &L) {
        {
            // one op per block of kAttnRows query rows, every request in it
            // (grid z; request rows R1 apart, tables max_blocks apart)
            const uint32_t packed = (uint32_t)c.rope_dim | ((uint32_t)nreq << 8) | ((uint32_t)R1 << 20);
            // the MFMA kernel walks up to 32 rows in one launch (the key chunk
            // read once); the other kernel takes kAttnRows at a time
            const uint64_t per = yk::attn_verify_mfma(c.kv_dtype == YUUKA_DTYPE_F16 ? 1 : 0, c.heads, c.kv_heads,
                                                      (int)hd, c.rope_dim, (int)kvdim)
                                     ? 32
                                     : kAttnRows;
            for (uint64_t c0 = 0; c0 < R1; c0 += per) {
                const uint64_t n = std::min<uint64_t>(per, R1 - c0), r0 = c0;
                b.add(YUUKA_EXT_OP_ATTN_VERIFY,
                      {q->q, q->k, q->v, L.kpool, L.vpool, q->attn, q->table, L.q_norm, L.k_norm, q->rope},
                      {(uint64_t)c.kv_heads, (uint64_t)c.heads, hd, kvdim, n, c0},
                      {(uint32_t)c.block_size, (uint32_t)c.capacity, c.kv_dtype, packed},
                      {(float)(1.0 / std::sqrt((double)hd)), c.eps}, 0,
                      {r0 * qdim * 4, r0 * kvdim * 4, r0 * kvdim * 4, 0, 0, r0 * odim * 4,
                       (uint64_t)first * q->max_blocks * 4, 0, 0, r0 * half * 8},
                      q->dyn, dyn_off(0));
            }
        }
    };
    // forward.go:320-389 forwardMoEFFN over all rows: router, top-k binning,
    // grouped expert SwiGLU and down projections, shared expert, weighted sum.
    auto moe_ffn = [&](Layer &L, uint64_t li) {
        const uint64_t E = (uint64_t)c.n_experts, used = (uint64_t)c.n_experts_used;
        const uint64_t ef = (uint64_t)c.expert_ffn;
        const bool sh = q->moe_shared;
        const uint32_t mf = YUUKA_EXT_FLAG_MOE_PACKED | (sh ? YUUKA_EXT_FLAG_MOE_SHARED : 0u);
        b.add(YUUKA_OP_RMSNORM_BATCH, {q->x, L.post_norm, q->xn}, {H, R, H, H}, {}, {c.eps});
        b.add(YUUKA_EXT_OP_MOE_ROUTER, {q->xn, L.router.b, q->moe_logits, L.shared_gate_vec, q->moe_sg}, {H, E, R});
        if (c.router_normal_seed)  // the configured routing: logits N(0,1) per row and expert
            b.add(YUUKA_EXT_OP_ROUTER_NORMAL, {q->moe_logits, q->step}, {R, E, (uint64_t)c.router_normal_seed, li});
        if (!sh) {  // the shared expert as its own GEMMs (its width differs from the experts')
            b.fused(q->xn, nullptr, 0.0f, R, {{&L.shared_gate, q->moe_sfg, nullptr}, {&L.shared_up, nullptr, nullptr}},
                    2);
            b.fused(q->moe_sfg, nullptr, 0.0f, R, {{&L.shared_down, q->moe_so, nullptr}}, 0);
        }
        // the grouped GEMMs take at most kMoeRows rows: row blocks (MoE rows are
        // independent), the bins and expert buffers reused by each block in turn
        for (uint64_t r0 = 0; r0 < R; r0 += kMoeRows) {
            const uint64_t n = std::min<uint64_t>(kMoeRows, R - r0);
            // each layer's expert counts stay in their own slice (yuuka_q35_moe_counts)
            const uint64_t co = li * E * 4;
            b.add(YUUKA_OP_MOE_ROUTE,
                  {q->moe_logits, q->moe_ids, q->moe_w, q->moe_counts, q->moe_arows, q->moe_aslots, q->moe_aw},
                  {n, E, used}, {}, {}, 0, {r0 * E * 4, 0, 0, co});
            b.add(YUUKA_OP_MOE_GATE_UP,
                  {q->xn, L.gate_exps.b, L.up_exps.b, q->moe_counts, q->moe_arows, q->moe_aslots, q->moe_act, nullptr},
                  {H, ef, n, E, used}, {L.gate_exps.dtype}, {}, YUUKA_EXT_FLAG_MOE_SWIGLU | mf, {r0 * H * 4, 0, 0, co});
            b.add(YUUKA_OP_MOE_DOWN, {q->moe_act, L.down_exps.b, q->moe_counts, q->moe_arows, q->moe_aslots, q->moe_eo},
                  {ef, H, n, E, used}, {L.down_exps.dtype}, {}, mf, {0, 0, co});
            b.add(YUUKA_EXT_OP_MOE_COMBINE, {q->x, q->moe_eo, q->moe_w, sh ? nullptr : q->moe_so, q->moe_sg},
                  {H, n, used}, {}, {}, sh ? YUUKA_EXT_FLAG_MOE_SHARED : 0u, {r0 * H * 4, 0, 0, sh ? 0 : r0 * H * 4, r0 * 4});
        }
    };
    for (int i = 0; i < c.n_layers; i++) {
        Layer &L = q->layers[i];
        if (L.recurrent) {  // plan.go:806-913
            // z is stored as SiLU(z); the scan writes raw per-head outputs
            // and the out projection applies the gated RMSNorm in its
            // prologue (recurrent.go:39-50)
            // beta is stored as sigmoid(beta), alpha as the decay
            // exp(softplus(alpha + dt) * a) (recurrent.go:66-70)
            b.fused(q->x, L.attn_norm, c.eps, R,
                    {{&L.qkv, L.qkv_rows, nullptr}, {&L.gate, q->z, nullptr}, {&L.beta, L.beta_rows, nullptr},
                     {&L.alpha, L.alpha_rows, L.dt_a}},
                    0, (1u << 4) | (2u << 8) | (3u << 12));
            recurrent(L, YUUKA_EXT_FLAG_RAW_OUT | YUUKA_EXT_FLAG_GDN_COEF);
            b.fused(q->gdn_out, nullptr, c.eps, R, {{&L.out, q->x, q->x}}, 1, 0, q->z, L.ssm_norm);
        } else {  // plan.go:684-804
            b.fused(q->x, L.attn_norm, c.eps, R,
                    {{&L.q, q->q, nullptr}, {&L.k, q->k, nullptr}, {&L.v, q->v, nullptr}}, 0);
            attention(L);
            b.fused(q->attn, nullptr, 0.0f, R, {{&L.o, q->x, q->x}}, 1);
        }
        if (L.moe) {
            moe_ffn(L, (uint64_t)i);
        } else {
            // plan.go:915-988 FFN: norm + gate/up + SwiGLU in one op, down + residual
            b.fused(q->x, L.post_norm, c.eps, R, {{&L.ffn_gate, q->fg, nullptr}, {&L.ffn_up, nullptr, nullptr}},
                    2);
            b.fused(q->fg, nullptr, 0.0f, R, {{&L.ffn_down, q->x, q->x}}, 1);
        }
    }
    // plan.go:635-662 all-logits tail
    b.fused(q->x, q->output_norm, c.eps, R, {{&q->output, q->logits, nullptr}}, 0);
    if (mode == 0) {
        const yuuka_q35_accept &a = q->accept_cfg;
        // drafts are tokens[j][1..k]; request index j of this plan is
        // request first + j (its Philox stream and result slot)
        b.add(YUUKA_EXT_OP_ACCEPT,
              {q->logits, q->tokens, q->result, nullptr, q->step, key.forced ? q->forced : nullptr},
              {(uint64_t)nreq, R1 - 1, (uint64_t)c.vocab, 0, a.seed, 0},
              {a.mode, a.top_k, (uint32_t)first, (uint32_t)R1}, {a.temperature, a.top_p}, 0,
              {0, 4, (uint64_t)first * 16, 0, 0, (uint64_t)first * 4});
    }
    // commit of every request's accepted prefix: one op per layer covering
    // all requests (consecutive layers merge into one launch)
    const bool commit_together = R1 <= 32;
    for (int j = 0; j < nreq; j += commit_together ? nreq : 1) {
        const uint64_t r0 = (uint64_t)j * R1, rq = (uint64_t)(first + j);
        for (int i = 0; i < c.n_layers; i++) {
            Layer &L = q->layers[i];
            if (!L.recurrent) continue;
            b.add(YUUKA_EXT_OP_GDN_COMMIT,
                  {L.conv_state, L.mat_state, L.qkv_rows, L.conv_rows, L.alpha_rows, L.beta_rows, L.dt, L.a,
                   q->result},
                  {R1, (uint64_t)c.groups, (uint64_t)c.rank, (uint64_t)c.state_size, cd, (uint64_t)c.inner},
                  {(uint32_t)c.conv_kernel, commit_together ? (uint32_t)nreq : 1u}, {},
                  YUUKA_EXT_FLAG_GDN_COEF,
                  {rq * L.conv_bytes, rq * L.mat_bytes, r0 * cd * 4, r0 * cd * 4, r0 * c.rank * 4, r0 * c.rank * 4, 0,
                   0, rq * 16});
        }
    }
    // every request's position in one launch; the step counter (Philox)
    // advances once per verify step, prefill chunks leave it alone
    b.add(YUUKA_EXT_OP_ADVANCE, {q->dyn, q->result, mode == 0 ? q->step : nullptr}, {R1}, {(uint32_t)nreq}, {}, 0,
          {dyn_off(0), (uint64_t)first * 16, 0});
    if (b.st != YUUKA_OK) {
        yuuka_plan_destroy(plan);
        return b.st;
    }
    *out = plan;
    return YUUKA_OK;
}

yuuka_status get_graph(yuuka_q35 *q, const PlanKey &k, Graphs **out) {
    auto key = std::make_tuple(k.first, k.nreq, k.rows, k.mode, k.forced);
    auto it = q->plans.find(key);
    if (it == q->plans.end()) {
        Graphs g;
        yuuka_status st = build_plan(q, k, &g.plan);
        if (st != YUUKA_OK) return st;
        if (!q->eager) st = yuuka_graph_create(g.plan, q->stream, q->dyn, 1, &g.graph);
        if (st != YUUKA_OK) {
            yuuka_plan_destroy(g.plan);
            return st;
        }
        it = q->plans.emplace(key, g).first;
    }
    *out = &it->second;
    return YUUKA_OK;
}

void drop_graphs(yuuka_q35 *q, bool verify_only) {
    for (auto it = q->plans.begin(); it != q->plans.end();) {
        if (verify_only && std::get<3>(it->first) != 0) {
            ++it;
            continue;
        }
        yuuka_graph_destroy(it->second.graph);
        yuuka_plan_destroy(it->second.plan);
        it = q->plans.erase(it);
    }
}

// ------------------------------------------------------------ KV blocks

void release_blocks(yuuka_q35 *q, int r) {
    for (int32_t blk : q->req[r].blocks)
        if (--q->refs[blk] == 0) q->free_blocks.push_back(blk);
    q->req[r].blocks.clear();
}

yuuka_status upload_table(yuuka_q35 *q, int r) {
    std::vector<int32_t> t(q->max_blocks, 0);
    std::copy(q->req[r].blocks.begin(), q->req[r].blocks.end(), t.begin());
    hipError_t err = hipMemcpy(static_cast<uint8_t *>(q->table->ptr) + (uint64_t)r * q->max_blocks * 4, t.data(),
                               (size_t)q->max_blocks * 4, hipMemcpyHostToDevice);
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "block table upload: %s", yk::hip_error(err));
    return YUUKA_OK;
}

// Makes request r's table cover positions [0, upto).
yuuka_status ensure_blocks(yuuka_q35 *q, int r, int upto) {
    const int need = (upto + q->cfg.block_size - 1) / q->cfg.block_size;
    if (need > q->max_blocks) return fail(YUUKA_ERR_INVALID_ARGUMENT, "request %d exceeds its context capacity", r);
    bool grew = false;
    while ((int)q->req[r].blocks.size() < need) {
        if (q->free_blocks.empty()) return fail(YUUKA_ERR_ALLOCATION, "KV pool exhausted (%zu blocks)", q->refs.size());
        const int32_t blk = q->free_blocks.back();
        q->free_blocks.pop_back();
        q->refs[blk] = 1;
        q->req[r].blocks.push_back(blk);
        grew = true;
    }
    return grew ? upload_table(q, r) : YUUKA_OK;
}

// ------------------------------------------------------------ stepping

// Runs one step of `key.rows` tokens for requests first..first+nreq-1
// (tokens already in the pinned staging). mode 1 presets result[0] =
// rows - 1 so the commit keeps every row.
yuuka_status run_step(yuuka_q35 *q, const PlanKey &key, int32_t *result_out) {
    for (int j = 0; j < key.nreq; j++) {
        yuuka_status st = ensure_blocks(q, key.first + j, q->req[key.first + j].pos + key.rows);
        if (st != YUUKA_OK) return st;
    }
    Graphs *g = nullptr;
    yuuka_status st = get_graph(q, key, &g);
    if (st != YUUKA_OK) return st;
    hipStream_t s = q->stream->stream;
    const size_t nt = (size_t)key.nreq * key.rows;
    hipError_t err = hipMemcpyAsync(q->tokens->ptr, pin_tokens(q), nt * 4, hipMemcpyHostToDevice, s);
    int32_t *pr = pin_result(q) + 4 * key.first;
    if (err == hipSuccess && key.mode == 1) {
        for (int j = 0; j < key.nreq; j++) {
            pr[4 * j] = key.rows - 1;
            pr[4 * j + 1] = -1;
            pr[4 * j + 2] = -1;
            pr[4 * j + 3] = 0;
        }
        err = hipMemcpyAsync(static_cast<uint8_t *>(q->result->ptr) + (uint64_t)key.first * 16, pr,
                             (size_t)key.nreq * 16, hipMemcpyHostToDevice, s);
    }
    if (err == hipSuccess && key.forced)
        err = hipMemcpyAsync(static_cast<uint8_t *>(q->forced->ptr) + (uint64_t)key.first * 4,
                             pin_forced(q) + key.first, (size_t)key.nreq * 4, hipMemcpyHostToDevice, s);
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "step upload: %s", yk::hip_error(err));
    (void)hipEventRecord(q->ev0, s);
    if (g->graph)
        st = yuuka_graph_replay(g->graph, q->stream, nullptr);
    else
        st = yk::plan_run_dynamic(g->plan, s, static_cast<const int32_t *>(q->dyn->ptr));
    if (st != YUUKA_OK) return st;
    (void)hipEventRecord(q->ev1, s);
    err = hipMemcpyAsync(pr, static_cast<uint8_t *>(q->result->ptr) + (uint64_t)key.first * 16,
                         (size_t)key.nreq * 16, hipMemcpyDeviceToHost, s);
    if (err == hipSuccess) err = hipStreamSynchronize(s);
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "verify step: %s", yk::hip_error(err));
    (void)hipEventElapsedTime(&q->last_ms, q->ev0, q->ev1);
    q->last_rows = key.rows;
    q->last_first = key.first;
    q->last_nreq = key.nreq;
    for (int j = 0; j < key.nreq; j++) q->req[key.first + j].pos += pr[4 * j] + 1;
    if (result_out) std::memcpy(result_out, pr, (size_t)key.nreq * 16);
    return YUUKA_OK;
}

int32_t read_pos(const yuuka_q35 *q, int r) {
    int32_t d[2] = {0, 0};
    if (hipMemcpy(d, static_cast<const uint8_t *>(q->dyn->ptr) + (uint64_t)r * 8, 8, hipMemcpyDeviceToHost) !=
        hipSuccess)
        return -1;  // reported as an invalid position
    return d[1];
}

template <typename F>
yuuka_status guard(const char *what, F &&f) {
    try {
        return f();
    } catch (const std::bad_alloc &) {
        return fail(YUUKA_ERR_ALLOCATION, "%s: host allocation failed", what);
    } catch (const std::exception &e) {
        return fail(YUUKA_ERR_INTERNAL, "%s: %s", what, e.what());
    } catch (...) {
        return fail(YUUKA_ERR_INTERNAL, "%s: unknown exception", what);
    }
}

bool same_accept(const yuuka_q35_accept &a, const yuuka_q35_accept &b) {
    return a.mode == b.mode && a.temperature == b.temperature && a.top_k == b.top_k && a.top_p == b.top_p &&
           a.seed == b.seed;
}

void set_accept(yuuka_q35 *q, const yuuka_q35_accept &a) {
    if (q->accept_set && same_accept(a, q->accept_cfg)) return;
    drop_graphs(q, true);  // acceptance settings are baked into the captured graphs
    q->accept_cfg = a;
    q->accept_set = true;
}

yuuka_status check_tokens(const yuuka_q35 *q, const int32_t *t, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (t[i] < 0 || t[i] >= q->cfg.vocab) return fail(YUUKA_ERR_INVALID_ARGUMENT, "token id %d is out of range", t[i]);
    return YUUKA_OK;
}

yuuka_status reset_request(yuuka_q35 *q, int r) {
    hipStream_t s = q->stream->stream;
    hipError_t eq = hipSuccess;  // first enqueue failure
    auto enq = [&](hipError_t e) { if (eq == hipSuccess) eq = e; };
    for (auto &L : q->layers) {
        if (!L.recurrent) continue;
        enq(hipMemsetAsync(static_cast<uint8_t *>(L.conv_state->ptr) + (uint64_t)r * L.conv_bytes, 0, L.conv_bytes, s));
        enq(hipMemsetAsync(static_cast<uint8_t *>(L.mat_state->ptr) + (uint64_t)r * L.mat_bytes, 0, L.mat_bytes, s));
    }
    enq(hipMemsetAsync(static_cast<uint8_t *>(q->dyn->ptr) + (uint64_t)r * 8, 0, 8, s));
    hipError_t err = hipStreamSynchronize(s);
    if (eq != hipSuccess) return fail(YUUKA_ERR_DEVICE, "reset enqueue: %s", yk::hip_error(eq));
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "reset: %s", yk::hip_error(err));
    release_blocks(q, r);
    q->req[r].pos = 0;
    return upload_table(q, r);
}

yuuka_status prefill_request(yuuka_q35 *q, int r, const int32_t *tokens, int32_t n, float *last_logits) {
    if (!tokens || n <= 0) return fail(YUUKA_ERR_INVALID_ARGUMENT, "empty token sequence");
    if (q->req[r].pos + n > q->cfg.capacity)
        return fail(YUUKA_ERR_INVALID_ARGUMENT, "token sequence of %d exceeds remaining context %d", n,
                    q->cfg.capacity - q->req[r].pos);
    yuuka_status st = check_tokens(q, tokens, (size_t)n);
    if (st != YUUKA_OK) return st;
    int done = 0;
    while (done < n) {
        const int rows = std::min(n - done, q->MR);
        std::memcpy(pin_tokens(q), tokens + done, (size_t)rows * 4);
        st = run_step(q, PlanKey{r, 1, rows, 1, 0}, nullptr);
        if (st != YUUKA_OK) return st;
        done += rows;
    }
    if (last_logits) {
        hipError_t err = hipMemcpy(last_logits,
                                   static_cast<float *>(q->logits->ptr) + (uint64_t)(q->last_rows - 1) * q->cfg.vocab,
                                   (size_t)q->cfg.vocab * 4, hipMemcpyDeviceToHost);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "logits copy: %s", yk::hip_error(err));
    }
    return YUUKA_OK;
}

// engine/speculative.go:39-66 lookupDraft.
int lookup_draft(const std::vector<int32_t> &h, int max_draft, int min_match, int32_t *out) {
    const int n = (int)h.size();
    if (max_draft <= 0 || min_match <= 0 || n <= min_match) return 0;
    const int max_n = std::min(8, n - 1);
    for (int len = max_n; len >= min_match; len--) {
        const int32_t *suffix = h.data() + n - len;
        for (int start = n - len - 1; start >= 0; start--) {
            if (std::memcmp(h.data() + start, suffix, (size_t)len * 4) != 0) continue;
            const int follow = start + len;
            const int take = std::min(max_draft, n - follow);
            if (take <= 0) continue;
            std::memcpy(out, h.data() + follow, (size_t)take * 4);
            return take;
        }
    }
    return 0;
}

}  // namespace

extern "C" {

yuuka_status yuuka_q35_create(yuuka_device *dev, const yuuka_q35_config *cfg, const yuuka_q35_weights *w,
                              yuuka_q35 **out) {
    return guard("q35_create", [&]() -> yuuka_status {
        if (!dev || !cfg || !w || !out || !w->layers) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        *out = nullptr;
        yuuka_q35_config c = *cfg;
        if (c.batch <= 0) c.batch = 1;
        if (c.n_layers <= 0 || c.hidden <= 0 || c.ffn < 0 || c.heads <= 0 || c.kv_heads <= 0 ||
            c.heads % c.kv_heads || c.vocab <= 0 || c.full_interval <= 0 || c.capacity <= 0 || c.block_size <= 0 ||
            c.max_rows < 1 || c.max_rows > 32 || c.conv_kernel < 2 || c.inner != c.rank * c.state_size ||
            c.batch > 256 || c.kv_blocks < 0)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid qwen35 configuration");
        const bool moe = c.n_experts > 0;
        if (moe && (c.n_experts_used <= 0 || c.n_experts_used > c.n_experts || c.expert_ffn <= 0 || c.shared_ffn <= 0))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid MoE configuration");
        if (!moe && c.ffn <= 0) return fail(YUUKA_ERR_INVALID_ARGUMENT, "dense FFN size must be positive");
        if (c.kv_dtype != YUUKA_DTYPE_F16 && c.kv_dtype != YUUKA_DTYPE_F32)
            return fail(YUUKA_ERR_UNSUPPORTED, "KV dtype %u", c.kv_dtype);
        std::unique_ptr<yuuka_q35> q(new yuuka_q35());
        q->dev = dev;
        q->cfg = c;
        q->B = c.batch;
        q->MR = c.max_rows;
        q->M = q->B * q->MR;
        q->moe_shared = moe && c.shared_ffn == c.expert_ffn;
        q->max_blocks = (c.capacity + c.block_size - 1) / c.block_size;
        q->conv_dim = 2 * c.groups * c.state_size + c.inner;
        q->req.resize(q->B);
        const int pool_blocks = c.kv_blocks > 0 ? c.kv_blocks : q->B * q->max_blocks;
        q->refs.assign(pool_blocks, 0);
        for (int i = pool_blocks - 1; i >= 0; i--) q->free_blocks.push_back(i);
        yuuka_status st = yuuka_stream_create(dev, &q->stream);
        if (st != YUUKA_OK) return st;
        hipError_t err = hipHostMalloc(reinterpret_cast<void **>(&q->pinned), (size_t)(q->M + 5 * q->B + 16) * 4,
                                       hipHostMallocDefault);
        if (err != hipSuccess) return fail(YUUKA_ERR_ALLOCATION, "pinned staging: %s", yk::hip_error(err));
        q->eager = getenv("YUUKA_Q35_EAGER") && getenv("YUUKA_Q35_EAGER")[0] == '1';
        if (hipEventCreate(&q->ev0) != hipSuccess || hipEventCreate(&q->ev1) != hipSuccess)
            return fail(YUUKA_ERR_DEVICE, "timing events");
        const uint64_t H = c.hidden, M = (uint64_t)q->M, hd = c.head_dim, Bq = (uint64_t)q->B;
        const uint64_t qdim = (uint64_t)c.heads * hd * 2, kvdim = (uint64_t)c.kv_heads * hd;
        const uint64_t cd = (uint64_t)q->conv_dim;
#define CHK(x)                              \
    do {                                    \
        yuuka_status s_ = (x);              \
        if (s_ != YUUKA_OK) {               \
            yuuka_q35_destroy(q.release()); \
            return s_;                      \
        }                                   \
    } while (0)
        CHK(upload_tensor(q.get(), w->embedding, c.vocab, H, "token_embd", &q->embedding));
        CHK(upload_tensor(q.get(), w->output, c.vocab, H, "output", &q->output));
        CHK(upload_vec(q.get(), w->output_norm, H, "output_norm", &q->output_norm));
        q->layers.resize(c.n_layers);
        const uint64_t kv_bytes = (uint64_t)pool_blocks * c.block_size * kvdim * (c.kv_dtype == YUUKA_DTYPE_F16 ? 2 : 4);
        for (int i = 0; i < c.n_layers; i++) {
            const yuuka_q35_layer_weights &lw = w->layers[i];
            Layer &L = q->layers[i];
            L.recurrent = (i + 1) % c.full_interval != 0;  // config.go:280-282
            L.moe = moe;
            CHK(upload_vec(q.get(), lw.attn_norm, H, "attn_norm", &L.attn_norm));
            CHK(upload_vec(q.get(), lw.post_norm, H, "post_attention_norm", &L.post_norm));
            if (L.recurrent) {
                CHK(upload_tensor(q.get(), lw.qkv, cd, H, "attn_qkv", &L.qkv));
                CHK(upload_tensor(q.get(), lw.gate, c.inner, H, "attn_gate", &L.gate));
                CHK(upload_tensor(q.get(), lw.out, H, c.inner, "ssm_out", &L.out));
                CHK(upload_tensor(q.get(), lw.beta, c.rank, H, "ssm_beta", &L.beta));
                CHK(upload_tensor(q.get(), lw.alpha, c.rank, H, "ssm_alpha", &L.alpha));
                CHK(upload_vec(q.get(), lw.conv, cd * c.conv_kernel, "ssm_conv1d", &L.conv));
                CHK(upload_vec(q.get(), lw.dt, c.rank, "ssm_dt", &L.dt));
                CHK(upload_vec(q.get(), lw.a, c.rank, "ssm_a", &L.a));
                {
                    std::vector<float> da(2 * (size_t)c.rank);
                    std::memcpy(da.data(), lw.dt, (size_t)c.rank * 4);
                    std::memcpy(da.data() + c.rank, lw.a, (size_t)c.rank * 4);
                    CHK(upload(q.get(), da.data(), da.size() * 4, &L.dt_a));
                }
                CHK(upload_vec(q.get(), lw.ssm_norm, c.state_size, "ssm_norm", &L.ssm_norm));
                L.conv_bytes = (uint64_t)(c.conv_kernel - 1) * cd * 4;
                L.mat_bytes = (uint64_t)c.rank * c.state_size * c.state_size * 4;
                CHK(alloc(q.get(), Bq * L.conv_bytes, &L.conv_state));
                CHK(alloc(q.get(), Bq * L.mat_bytes, &L.mat_state));
                CHK(alloc(q.get(), M * cd * 4, &L.qkv_rows));
                CHK(alloc(q.get(), M * cd * 4, &L.conv_rows));
                CHK(alloc(q.get(), M * c.rank * 4, &L.alpha_rows));
                CHK(alloc(q.get(), M * c.rank * 4, &L.beta_rows));
            } else {
                CHK(upload_tensor(q.get(), lw.q, qdim, H, "attn_q", &L.q));
                CHK(upload_tensor(q.get(), lw.k, kvdim, H, "attn_k", &L.k));
                CHK(upload_tensor(q.get(), lw.v, kvdim, H, "attn_v", &L.v));
                CHK(upload_tensor(q.get(), lw.o, H, (uint64_t)c.heads * hd, "attn_output", &L.o));
                CHK(upload_vec(q.get(), lw.q_norm, hd, "attn_q_norm", &L.q_norm));
                CHK(upload_vec(q.get(), lw.k_norm, hd, "attn_k_norm", &L.k_norm));
                CHK(alloc(q.get(), kv_bytes, &L.kpool));
                CHK(alloc(q.get(), kv_bytes, &L.vpool));
            }
            if (moe) {
                const uint64_t E = c.n_experts, ef = c.expert_ffn, sf = c.shared_ffn;
                if (lw.router.dtype != YUUKA_DTYPE_F32 || lw.gate_exps.dtype != YUUKA_DTYPE_Q4_K ||
                    lw.up_exps.dtype != YUUKA_DTYPE_Q4_K || lw.down_exps.dtype != YUUKA_DTYPE_Q4_K)
                    CHK(fail(YUUKA_ERR_UNSUPPORTED, "MoE layer %d: router F32 and Q4_K experts are served", i));
                CHK(upload_tensor(q.get(), lw.router, E, H, "ffn_gate_inp", &L.router));
                CHK(upload_vec(q.get(), lw.shared_gate_vec, H, "ffn_gate_inp_shexp", &L.shared_gate_vec));
                if (q->moe_shared) {
                    CHK(upload_experts(q.get(), lw.gate_exps, E * ef, H, "ffn_gate_exps", &L.gate_exps, &lw.shared_gate,
                                       sf, "ffn_gate_shexp"));
                    CHK(upload_experts(q.get(), lw.up_exps, E * ef, H, "ffn_up_exps", &L.up_exps, &lw.shared_up, sf,
                                       "ffn_up_shexp"));
                    CHK(upload_experts(q.get(), lw.down_exps, E * H, ef, "ffn_down_exps", &L.down_exps, &lw.shared_down,
                                       H, "ffn_down_shexp"));
                } else {
                    CHK(upload_tensor(q.get(), lw.shared_gate, sf, H, "ffn_gate_shexp", &L.shared_gate));
                    CHK(upload_tensor(q.get(), lw.shared_up, sf, H, "ffn_up_shexp", &L.shared_up));
                    CHK(upload_tensor(q.get(), lw.shared_down, H, sf, "ffn_down_shexp", &L.shared_down));
                    CHK(upload_experts(q.get(), lw.gate_exps, E * ef, H, "ffn_gate_exps", &L.gate_exps));
                    CHK(upload_experts(q.get(), lw.up_exps, E * ef, H, "ffn_up_exps", &L.up_exps));
                    CHK(upload_experts(q.get(), lw.down_exps, E * H, ef, "ffn_down_exps", &L.down_exps));
                }
            } else {
                CHK(upload_tensor(q.get(), lw.ffn_gate, c.ffn, H, "ffn_gate", &L.ffn_gate));
                CHK(upload_tensor(q.get(), lw.ffn_up, c.ffn, H, "ffn_up", &L.ffn_up));
                CHK(upload_tensor(q.get(), lw.ffn_down, H, c.ffn, "ffn_down", &L.ffn_down));
            }
        }
        const uint64_t ffn_w = moe ? (uint64_t)c.shared_ffn : (uint64_t)c.ffn;
        CHK(alloc(q.get(), M * H * 4, &q->x));
        CHK(alloc(q.get(), M * H * 4, &q->xn));
        CHK(alloc(q.get(), M * qdim * 4, &q->q));
        CHK(alloc(q.get(), M * kvdim * 4, &q->k));
        CHK(alloc(q.get(), M * kvdim * 4, &q->v));
        CHK(alloc(q.get(), M * c.heads * hd * 4, &q->attn));
        CHK(alloc(q.get(), M * (uint64_t)(c.rope_dim / 2) * 8, &q->rope));
        CHK(alloc(q.get(), M * c.inner * 4, &q->z));
        CHK(alloc(q.get(), M * c.inner * 4, &q->gdn_out));
        CHK(alloc(q.get(), M * ffn_w * 4, &q->fg));
        CHK(alloc(q.get(), M * ffn_w * 4, &q->fu));
        CHK(alloc(q.get(), M * (uint64_t)c.vocab * 4, &q->logits));
        if (moe) {
            const uint64_t E = c.n_experts, used = c.n_experts_used;
            CHK(alloc(q.get(), M * E * 4, &q->moe_logits));
            CHK(alloc(q.get(), M * 4, &q->moe_sg));
            CHK(alloc(q.get(), M * used * 4, &q->moe_ids));
            CHK(alloc(q.get(), M * used * 4, &q->moe_w));
            CHK(alloc(q.get(), E * (uint64_t)c.n_layers * 4, &q->moe_counts));
            CHK(alloc(q.get(), E * M * used * 4, &q->moe_arows));
            CHK(alloc(q.get(), E * M * used * 4, &q->moe_aslots));
            CHK(alloc(q.get(), E * M * used * 4, &q->moe_aw));
            // with the shared expert fused, one more output slot per row
            const uint64_t os = used + (q->moe_shared ? 1 : 0), mb = std::min<uint64_t>(M, kMoeRows);
            CHK(alloc(q.get(), mb * os * c.expert_ffn * 4, &q->moe_act));
            CHK(alloc(q.get(), mb * os * H * 4, &q->moe_eo));
            if (!q->moe_shared) {
                CHK(alloc(q.get(), M * c.shared_ffn * 4, &q->moe_sfg));
                CHK(alloc(q.get(), M * H * 4, &q->moe_so));
            }
        }
        CHK(alloc(q.get(), (M + 64) * 4, &q->tokens));
        CHK(alloc(q.get(), Bq * 16, &q->result));
        CHK(alloc(q.get(), Bq * 8, &q->dyn));
        CHK(alloc(q.get(), 8, &q->step));
        CHK(alloc(q.get(), Bq * 4, &q->forced));
        CHK(alloc(q.get(), Bq * q->max_blocks * 4, &q->table));
        *out = q.release();
        return yuuka_q35_reset(*out);
#undef CHK
    });
}

void yuuka_q35_destroy(yuuka_q35 *q) {
    if (!q) return;
    if (q->stream) (void)hipStreamSynchronize(q->stream->stream);
    drop_graphs(q, false);
    for (auto *b : q->owned) yuuka_buffer_free(b);
    if (q->pinned) (void)hipHostFree(q->pinned);
    if (q->ev0) (void)hipEventDestroy(q->ev0);
    if (q->ev1) (void)hipEventDestroy(q->ev1);
    yuuka_stream_destroy(q->stream);
    delete q;
}

yuuka_status yuuka_q35_reset(yuuka_q35 *q) {
    return guard("q35_reset", [&]() -> yuuka_status {
        if (!q) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null engine");
        for (int r = 0; r < q->B; r++) {
            yuuka_status st = reset_request(q, r);
            if (st != YUUKA_OK) return st;
        }
        hipError_t eq = hipMemsetAsync(q->step->ptr, 0, 8, q->stream->stream);
        hipError_t err = hipStreamSynchronize(q->stream->stream);
        if (eq != hipSuccess) return fail(YUUKA_ERR_DEVICE, "reset enqueue: %s", yk::hip_error(eq));
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "reset: %s", yk::hip_error(err));
        return YUUKA_OK;
    });
}

yuuka_status yuuka_q35_reset_request(yuuka_q35 *q, int32_t request) {
    return guard("q35_reset_request", [&]() -> yuuka_status {
        if (!q || request < 0 || request >= q->B) return fail(YUUKA_ERR_INVALID_ARGUMENT, "bad request index");
        return reset_request(q, request);
    });
}

float yuuka_q35_last_step_ms(const yuuka_q35 *q) { return q ? q->last_ms : 0.0f; }

int32_t yuuka_q35_position(const yuuka_q35 *q) { return q ? read_pos(q, 0) : -1; }

int32_t yuuka_q35_request_position(const yuuka_q35 *q, int32_t request) {
    return q && request >= 0 && request < q->B ? read_pos(q, request) : -1;
}

yuuka_status yuuka_q35_prefill(yuuka_q35 *q, const int32_t *tokens, int32_t n, float *last_logits) {
    return guard("q35_prefill", [&]() -> yuuka_status {
        if (!q || (!tokens && n)) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        return prefill_request(q, 0, tokens, n, last_logits);
    });
}

yuuka_status yuuka_q35_prefill_request(yuuka_q35 *q, int32_t request, const int32_t *tokens, int32_t n,
                                       float *last_logits) {
    return guard("q35_prefill_request", [&]() -> yuuka_status {
        if (!q || (!tokens && n)) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (request < 0 || request >= q->B) return fail(YUUKA_ERR_INVALID_ARGUMENT, "bad request index");
        return prefill_request(q, request, tokens, n, last_logits);
    });
}

yuuka_status yuuka_q35_fork(yuuka_q35 *q, int32_t src, int32_t dst) {
    return guard("q35_fork", [&]() -> yuuka_status {
        if (!q || src < 0 || dst < 0 || src >= q->B || dst >= q->B || src == dst)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "bad request indices");
        yuuka_status st = reset_request(q, dst);
        if (st != YUUKA_OK) return st;
        const int32_t pos = q->req[src].pos, bs = q->cfg.block_size;
        const int full = pos / bs;
        hipStream_t s = q->stream->stream;
        hipError_t eq = hipSuccess;  // first enqueue failure
        auto enq = [&](hipError_t e) { if (eq == hipSuccess) eq = e; };
        Request &d = q->req[dst];
        for (int i = 0; i < full; i++) {  // memory/prefix.go: shared blocks, one more reference each
            const int32_t blk = q->req[src].blocks[i];
            q->refs[blk]++;
            d.blocks.push_back(blk);
        }
        if (pos % bs) {  // the partial last block is copied: both requests write past it
            st = ensure_blocks(q, dst, pos);
            if (st != YUUKA_OK) return st;
            const int32_t from = q->req[src].blocks[full], to = d.blocks[full];
            const uint64_t kvdim = (uint64_t)q->cfg.kv_heads * q->cfg.head_dim;
            const uint64_t blk_bytes = (uint64_t)bs * kvdim * (q->cfg.kv_dtype == YUUKA_DTYPE_F16 ? 2 : 4);
            for (auto &L : q->layers) {
                if (L.recurrent) continue;
                for (yuuka_buffer *pool : {L.kpool, L.vpool}) {
                    uint8_t *base = static_cast<uint8_t *>(pool->ptr);
                    enq(hipMemcpyAsync(base + (uint64_t)to * blk_bytes, base + (uint64_t)from * blk_bytes, blk_bytes,
                                       hipMemcpyDeviceToDevice, s));
                }
            }
        }
        st = upload_table(q, dst);
        if (st != YUUKA_OK) return st;
        for (auto &L : q->layers) {
            if (!L.recurrent) continue;
            uint8_t *cs = static_cast<uint8_t *>(L.conv_state->ptr), *ms = static_cast<uint8_t *>(L.mat_state->ptr);
            enq(hipMemcpyAsync(cs + (uint64_t)dst * L.conv_bytes, cs + (uint64_t)src * L.conv_bytes, L.conv_bytes,
                               hipMemcpyDeviceToDevice, s));
            enq(hipMemcpyAsync(ms + (uint64_t)dst * L.mat_bytes, ms + (uint64_t)src * L.mat_bytes, L.mat_bytes,
                               hipMemcpyDeviceToDevice, s));
        }
        uint8_t *dy = static_cast<uint8_t *>(q->dyn->ptr);
        enq(hipMemcpyAsync(dy + (uint64_t)dst * 8, dy + (uint64_t)src * 8, 8, hipMemcpyDeviceToDevice, s));
        hipError_t err = hipStreamSynchronize(s);
        if (eq != hipSuccess) return fail(YUUKA_ERR_DEVICE, "fork enqueue: %s", yk::hip_error(eq));
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "fork: %s", yk::hip_error(err));
        d.pos = pos;
        return YUUKA_OK;
    });
}

yuuka_status yuuka_q35_verify(yuuka_q35 *q, const int32_t *tokens, int32_t rows, const yuuka_q35_accept *accept,
                              int32_t *result) {
    return guard("q35_verify", [&]() -> yuuka_status {
        if (!q || !tokens || !accept) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (rows < 1 || rows > q->MR)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "verify rows %d outside 1..%d", rows, q->MR);
        yuuka_status st = check_tokens(q, tokens, (size_t)rows);
        if (st != YUUKA_OK) return st;
        if (q->req[0].pos + rows > q->cfg.capacity)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "context capacity exhausted");
        set_accept(q, *accept);
        std::memcpy(pin_tokens(q), tokens, (size_t)rows * 4);
        return run_step(q, PlanKey{0, 1, rows, 0, 0}, result);
    });
}

yuuka_status yuuka_q35_step_batch(yuuka_q35 *q, int32_t n_req, const int32_t *tokens, int32_t rows, int32_t mode,
                                  const yuuka_q35_accept *accept, const int32_t *forced, int32_t *result) {
    return guard("q35_step_batch", [&]() -> yuuka_status {
        if (!q || !tokens) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (n_req < 1 || n_req > q->B) return fail(YUUKA_ERR_INVALID_ARGUMENT, "requests %d outside 1..%d", n_req, q->B);
        if (rows < 1 || rows > q->MR) return fail(YUUKA_ERR_INVALID_ARGUMENT, "rows %d outside 1..%d", rows, q->MR);
        if (mode != 0 && mode != 1) return fail(YUUKA_ERR_INVALID_ARGUMENT, "mode %d", mode);
        if (mode == 0 && !accept) return fail(YUUKA_ERR_INVALID_ARGUMENT, "verify needs acceptance settings");
        yuuka_status st = check_tokens(q, tokens, (size_t)n_req * rows);
        if (st != YUUKA_OK) return st;
        for (int r = 0; r < n_req; r++)
            if (q->req[r].pos + rows > q->cfg.capacity)
                return fail(YUUKA_ERR_INVALID_ARGUMENT, "request %d: context capacity exhausted", r);
        if (mode == 0) set_accept(q, *accept);
        std::memcpy(pin_tokens(q), tokens, (size_t)n_req * rows * 4);
        const bool use_forced = mode == 0 && forced != nullptr;
        if (use_forced) std::memcpy(pin_forced(q), forced, (size_t)n_req * 4);
        return run_step(q, PlanKey{0, n_req, rows, mode, use_forced ? 1 : 0}, result);
    });
}

yuuka_status yuuka_q35_logits(yuuka_q35 *q, float *out, int32_t rows) {
    return guard("q35_logits", [&]() -> yuuka_status {
        if (!q || !out || rows < 1 || rows > q->M) return fail(YUUKA_ERR_INVALID_ARGUMENT, "bad arguments");
        hipError_t err = hipMemcpy(out, q->logits->ptr, (size_t)rows * q->cfg.vocab * 4, hipMemcpyDeviceToHost);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "logits copy: %s", yk::hip_error(err));
        return YUUKA_OK;
    });
}

yuuka_status yuuka_q35_moe_counts(yuuka_q35 *q, int32_t layer, int32_t *counts, int32_t n) {
    return guard("q35_moe_counts", [&]() -> yuuka_status {
        if (!q || !counts || layer < 0 || layer >= q->cfg.n_layers || q->cfg.n_experts <= 0 || n < q->cfg.n_experts)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "bad arguments");
        const uint64_t E = (uint64_t)q->cfg.n_experts;
        hipError_t err = hipStreamSynchronize(q->stream->stream);
        if (err == hipSuccess)
            err = hipMemcpy(counts, static_cast<const uint8_t *>(q->moe_counts->ptr) + (uint64_t)layer * E * 4, E * 4,
                            hipMemcpyDeviceToHost);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "MoE counts copy: %s", yk::hip_error(err));
        return YUUKA_OK;
    });
}

uint64_t yuuka_q35_snapshot_bytes(const yuuka_q35 *q) {
    if (!q) return 0;
    uint64_t n = 0;
    for (auto &L : q->layers)
        if (L.recurrent) n += L.conv_bytes + L.mat_bytes;
    return n;
}

yuuka_status yuuka_q35_snapshot(yuuka_q35 *q, void *out, int32_t *position) {
    return guard("q35_snapshot", [&]() -> yuuka_status {
        if (!q || !out) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        uint8_t *p = static_cast<uint8_t *>(out);
        for (auto &L : q->layers) {
            if (!L.recurrent) continue;
            hipError_t err = hipMemcpy(p, L.conv_state->ptr, L.conv_bytes, hipMemcpyDeviceToHost);
            p += L.conv_bytes;
            if (err == hipSuccess) err = hipMemcpy(p, L.mat_state->ptr, L.mat_bytes, hipMemcpyDeviceToHost);
            p += L.mat_bytes;
            if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "snapshot: %s", yk::hip_error(err));
        }
        if (position) *position = read_pos(q, 0);
        return YUUKA_OK;
    });
}

yuuka_status yuuka_q35_restore(yuuka_q35 *q, const void *data, uint64_t bytes, int32_t position) {
    return guard("q35_restore", [&]() -> yuuka_status {
        if (!q || !data) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (bytes != yuuka_q35_snapshot_bytes(q))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "state snapshot is %llu bytes, want %llu",
                        (unsigned long long)bytes, (unsigned long long)yuuka_q35_snapshot_bytes(q));
        if (position < 0 || position > q->cfg.capacity)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "position %d exceeds capacity %d", position, q->cfg.capacity);
        const uint8_t *p = static_cast<const uint8_t *>(data);
        for (auto &L : q->layers) {
            if (!L.recurrent) continue;
            hipError_t err = hipMemcpy(L.conv_state->ptr, p, L.conv_bytes, hipMemcpyHostToDevice);
            p += L.conv_bytes;
            if (err == hipSuccess) err = hipMemcpy(L.mat_state->ptr, p, L.mat_bytes, hipMemcpyHostToDevice);
            p += L.mat_bytes;
            if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "restore: %s", yk::hip_error(err));
        }
        // the KV rows up to `position` stay where they are (state.go:230-263
        // restores the recurrent state only; the KV cache is position-indexed)
        yuuka_status st = ensure_blocks(q, 0, position);
        if (st != YUUKA_OK) return st;
        q->req[0].pos = position;
        int32_t d[2] = {0, position};
        hipError_t err = hipMemcpy(q->dyn->ptr, d, 8, hipMemcpyHostToDevice);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "restore: %s", yk::hip_error(err));
        return YUUKA_OK;
    });
}

yuuka_status yuuka_q35_generate(yuuka_q35 *q, const int32_t *prompt, int32_t n_prompt,
                                const yuuka_q35_generate_opts *o, int32_t *out_tokens,
                                yuuka_q35_generate_stats *stats) {
    return guard("q35_generate", [&]() -> yuuka_status {
        if (!q || !prompt || !o || !out_tokens) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (n_prompt <= 0) return fail(YUUKA_ERR_INVALID_ARGUMENT, "prompt is empty");
        if (o->max_tokens <= 0) return fail(YUUKA_ERR_INVALID_ARGUMENT, "max tokens must be positive");
        if (n_prompt > q->cfg.capacity)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "prompt length %d exceeds context capacity %d", n_prompt,
                        q->cfg.capacity);
        // speculative.go:21-34 normalize, capped by the engine's row block
        int k = o->max_draft <= 0 ? 4 : std::min(o->max_draft, 16);
        k = std::min(k, q->MR - 1);
        int min_match = o->min_match <= 0 ? 2 : std::min(o->min_match, 8);
        int max_tokens = std::min(o->max_tokens, q->cfg.capacity - n_prompt);
        if (max_tokens <= 0) return fail(YUUKA_ERR_INVALID_ARGUMENT, "no context space remains");
        yuuka_q35_generate_stats st_local{};
        yuuka_status st = reset_request(q, 0);
        if (st != YUUKA_OK) return st;
        // a generation starts its Philox step counter at 0
        hipError_t err0 = hipMemset(q->step->ptr, 0, 8);
        if (err0 != hipSuccess) return fail(YUUKA_ERR_DEVICE, "step counter: %s", yk::hip_error(err0));
        auto t0 = std::chrono::steady_clock::now();
        if (n_prompt > 1) {
            st = prefill_request(q, 0, prompt, n_prompt - 1, nullptr);
            if (st != YUUKA_OK) return st;
        }
        auto t1 = std::chrono::steady_clock::now();
        std::vector<int32_t> history(prompt, prompt + n_prompt);
        int32_t pending = prompt[n_prompt - 1];
        int emitted = 0;
        bool stop = false;
        std::vector<int32_t> rows_tok(33);
        while (emitted < max_tokens && !stop) {
            const int32_t pos = q->req[0].pos;
            int limit = std::min(k, max_tokens - emitted);
            limit = std::min(limit, q->cfg.capacity - pos - 1);
            if (limit < 0) break;
            int32_t draft[32];
            int nd = lookup_draft(history, limit, min_match, draft);
            for (int i = nd; i < limit; i++) draft[i] = pending;  // padding guess
            rows_tok[0] = pending;
            for (int i = 0; i < limit; i++) rows_tok[1 + i] = draft[i];
            int32_t res[4];
            st = yuuka_q35_verify(q, rows_tok.data(), limit + 1, &o->accept, res);
            if (st != YUUKA_OK) return st;
            st_local.steps++;
            st_local.draft_tokens += limit;
            st_local.accepted_draft += res[0];
            for (int i = 0; i <= res[0] && !stop; i++) {
                const int32_t tok = i < res[0] ? draft[i] : res[1];
                if (tok == o->stop_token && o->stop_token >= 0) {
                    stop = true;
                    break;
                }
                out_tokens[emitted++] = tok;
                history.push_back(tok);
                if (emitted >= max_tokens) break;
            }
            pending = res[1];
        }
        auto t2 = std::chrono::steady_clock::now();
        st_local.output_tokens = emitted;
        st_local.prefill_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
        st_local.decode_ms = std::chrono::duration<double, std::milli>(t2 - t1).count();
        if (stats) *stats = st_local;
        return YUUKA_OK;
    });
}

}  // extern "C"
