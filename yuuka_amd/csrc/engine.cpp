// engine.cpp — qwen35 verify engine: the host side of the speculative verify
// path, in C++ over this library's own plan API.
//
// Counterparts in the reference: engine/gpu/runtime.go + session.go (weights
// and per-request state on the device, PrefillLogits, Snapshot/Restore),
// engine/gpu/plan.go:569-988 (buildPrefillPlan and the per-layer blocks) and
// engine/speculative.go:68-261 (generateSpeculative). Differences by design:
//  * the verify plan covers k+1 rows {pending token, d1..dk}, ends with the
//    fused acceptance and commits only the accepted prefix of the recurrent
//    state on the device (GDN_COMMIT), then advances the device position, so
//    no snapshot / restore / replay crosses PCIe per step;
//  * every plan is captured once per row count into a HIP graph.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "internal.h"
#include "plan.h"

namespace {

using yk::fail;

struct DevBuf {
    yuuka_buffer *b = nullptr;
    ~DevBuf() { yuuka_buffer_free(b); }
};

struct Tensor {
    yuuka_buffer *b = nullptr;
    uint64_t rows = 0, cols = 0;
    uint32_t dtype = 0;
};

struct Layer {
    bool recurrent = false;
    yuuka_buffer *attn_norm = nullptr, *post_norm = nullptr;
    Tensor qkv, gate, out, beta, alpha, q, k, v, o, ffn_gate, ffn_up, ffn_down;
    yuuka_buffer *conv = nullptr, *dt = nullptr, *a = nullptr, *ssm_norm = nullptr, *q_norm = nullptr,
                 *k_norm = nullptr;
    yuuka_buffer *dt_a = nullptr;  // {dt[rank], a[rank]}: decay parameters of the projection epilogue
    // per-request state
    yuuka_buffer *conv_state = nullptr, *mat_state = nullptr, *kpool = nullptr, *vpool = nullptr;
    // per-step saved inputs of the recurrent block (read by GDN_COMMIT)
    yuuka_buffer *qkv_rows = nullptr, *conv_rows = nullptr, *alpha_rows = nullptr, *beta_rows = nullptr;
};

struct Graphs {
    yuuka_plan *plan = nullptr;
    yuuka_graph *graph = nullptr;
};

}  // namespace

struct yuuka_q35 {
    yuuka_device *dev = nullptr;
    yuuka_stream *stream = nullptr;
    yuuka_q35_config cfg{};
    int conv_dim = 0;
    std::vector<yuuka_buffer *> owned;
    std::vector<Layer> layers;
    Tensor embedding, output;
    yuuka_buffer *output_norm = nullptr;
    // activations [max_rows][...]
    yuuka_buffer *x = nullptr, *xn = nullptr, *xq = nullptr, *q = nullptr, *k = nullptr, *v = nullptr,
                 *attn = nullptr, *z = nullptr, *gdn_out = nullptr, *fg = nullptr, *fu = nullptr, *logits = nullptr,
                 *tokens = nullptr, *result = nullptr, *dyn = nullptr, *step = nullptr, *table = nullptr,
                 *rope = nullptr;
    int32_t *pinned = nullptr;  // tokens staging {tokens[16], result[4]}
    hipEvent_t ev0 = nullptr, ev1 = nullptr;  // around the last graph replay
    bool eager = false;  // YUUKA_Q35_EAGER=1: launch plans op by op (profilers), no graphs
    float last_ms = 0.0f;
    // plans keyed by (rows, mode): mode 0 verify greedy/stochastic, 1 commit-all
    std::map<std::pair<int, int>, Graphs> plans;
    yuuka_q35_accept accept_cfg{};
    bool accept_set = false;
    int last_rows = 0;
};

namespace {

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

yuuka_status upload_vec(yuuka_q35 *q, const float *v, uint64_t n, const char *what, yuuka_buffer **out) {
    if (!v) return fail(YUUKA_ERR_INVALID_ARGUMENT, "%s: missing data", what);
    return upload(q, v, n * 4, out);
}

// ------------------------------------------------------------ plan build

struct Builder {
    yuuka_plan *plan;
    yuuka_status st = YUUKA_OK;
    void add(uint32_t code, std::initializer_list<yuuka_buffer *> bufs, std::initializer_list<uint64_t> n,
             std::initializer_list<uint32_t> u = {}, std::initializer_list<float> f = {}, uint32_t flags = 0,
             std::initializer_list<uint64_t> offs = {}) {
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
        st = yuuka_plan_add(plan, &op);
    }
    void gemm(const Tensor &w, yuuka_buffer *xq, yuuka_buffer *out, uint64_t rows, yuuka_buffer *residual = nullptr) {
        add(YUUKA_EXT_OP_GEMM_Q, {w.b, xq, out, residual}, {w.cols, w.rows, rows}, {w.dtype});
    }
    void quant(yuuka_buffer *x, uint64_t K, uint64_t rows, yuuka_buffer *xq) {
        add(YUUKA_EXT_OP_QUANTIZE_X, {x, xq}, {K, rows});
    }
    struct Seg {
        const Tensor *w;
        yuuka_buffer *out, *res;
    };
    // One GEMM_FUSED op: every segment reads the same activation rows x
    // (optionally RMS-normalised with `norm`).
    void fused(yuuka_buffer *x, yuuka_buffer *norm, float eps, uint64_t rows, std::initializer_list<Seg> segs,
               uint32_t epilogue, uint32_t silu_mask = 0, yuuka_buffer *gate = nullptr,
               yuuka_buffer *head_norm = nullptr) {
        if (st != YUUKA_OK) return;
        yuuka_op op{};
        op.code = YUUKA_EXT_OP_GEMM_FUSED;
        op.buf[0] = x;
        op.buf[1] = norm;
        op.buf[14] = gate;
        op.buf[15] = head_norm;
        op.u[2] = silu_mask;
        op.n[1] = rows;
        op.u[1] = epilogue;
        op.f[0] = eps;
        int i = 0;
        for (const Seg &g : segs) {
            op.buf[2 + i] = g.w->b;
            op.buf[6 + i] = g.out;
            op.buf[10 + i] = g.res;
            op.n[0] = g.w->cols;
            op.n[2 + i] = g.w->rows;
            op.u[0] |= g.w->dtype << (8 * i);
            i++;
        }
        st = yuuka_plan_add(plan, &op);
    }
};

// Fused projections need Q4_K / Q6_K weights; YUUKA_Q35_FUSED=0 selects the
// separate quantize / GEMM / reduce ops (comparison and fallback).
bool use_fused(const yuuka_q35 *q) {
    if (const char *e = getenv("YUUKA_Q35_FUSED"))
        if (e[0] == '0') return false;
    auto ok = [](const Tensor &t) { return !t.b || t.dtype == YUUKA_DTYPE_Q4_K || t.dtype == YUUKA_DTYPE_Q6_K; };
    if (!ok(q->output)) return false;
    for (const Layer &L : q->layers)
        for (const Tensor *t : {&L.qkv, &L.gate, &L.beta, &L.alpha, &L.out, &L.q, &L.k, &L.v, &L.o, &L.ffn_gate,
                                &L.ffn_up, &L.ffn_down})
            if (!ok(*t)) return false;
    return true;
}

// mode 0: verify (acceptance on device), mode 1: commit every row (prefill).
yuuka_status build_plan(yuuka_q35 *q, int rows, int mode, yuuka_plan **out) {
    const yuuka_q35_config &c = q->cfg;
    yuuka_plan *plan = nullptr;
    yuuka_status st = yuuka_plan_create(q->dev, &plan);
    if (st != YUUKA_OK) return st;
    Builder b{plan};
    const uint64_t R = (uint64_t)rows, H = (uint64_t)c.hidden, hd = (uint64_t)c.head_dim;
    const uint64_t qdim = (uint64_t)c.heads * hd * 2, kvdim = (uint64_t)c.kv_heads * hd, odim = (uint64_t)c.heads * hd;
    // plan.go:585-588 EMBEDDING_BATCH
    b.add(YUUKA_OP_EMBEDDING_BATCH, {q->embedding.b, q->x, q->tokens},
          {H, R, yk::row_bytes(q->embedding.dtype, H), (uint64_t)c.vocab}, {q->embedding.dtype});
    const bool fused = use_fused(q);
    const float qscale = (float)(1.0 / std::sqrt((double)c.state_size));
    auto recurrent_chunk = [&](Layer &L, uint32_t extra_flags) {
        b.add(YUUKA_OP_RECURRENT_CHUNK,
              {L.conv_state, L.mat_state, L.qkv_rows, q->z, L.alpha_rows, L.beta_rows, L.conv, L.dt, L.a, L.ssm_norm,
               q->gdn_out, L.conv_rows},
              {R, (uint64_t)c.groups, (uint64_t)c.rank, (uint64_t)c.state_size, (uint64_t)q->conv_dim,
               (uint64_t)c.inner},
              {(uint32_t)c.conv_kernel}, {c.eps, qscale}, YUUKA_EXT_FLAG_DEFER | extra_flags);
    };
    // YUUKA_Q35_ATTN=0 selects the separate norm / RoPE / KV-write /
    // attention ops (comparison); by default one ATTN_VERIFY op per layer.
    const char *attn_env = getenv("YUUKA_Q35_ATTN");
    const bool attn_fused = !(attn_env && attn_env[0] == '0');
    bool any_attn = false;
    for (const Layer &L : q->layers) any_attn |= !L.recurrent;
    if (attn_fused && any_attn)
        b.add(YUUKA_EXT_OP_ROPE_TABLE, {q->rope}, {R, (uint64_t)c.rope_dim, 0}, {}, {(float)c.rope_base});
    auto attention = [&](Layer &L) {
        if (attn_fused) {
            b.add(YUUKA_EXT_OP_ATTN_VERIFY,
                  {q->q, q->k, q->v, L.kpool, L.vpool, q->attn, q->table, L.q_norm, L.k_norm, q->rope},
                  {(uint64_t)c.kv_heads, (uint64_t)c.heads, hd, kvdim, R, 0},
                  {(uint32_t)c.block_size, (uint32_t)c.capacity, c.kv_dtype, (uint32_t)c.rope_dim},
                  {(float)(1.0 / std::sqrt((double)hd)), c.eps});
            return;
        }
        b.add(YUUKA_OP_RMSNORM_HEADS_BATCH, {q->k, L.k_norm, q->k}, {hd, (uint64_t)c.kv_heads, hd, R}, {}, {c.eps});
        b.add(YUUKA_OP_ROPE_BATCH, {q->k}, {(uint64_t)c.kv_heads, hd, hd, (uint64_t)c.rope_dim, R, kvdim}, {0},
              {(float)c.rope_base});
        b.add(YUUKA_OP_KV_WRITE_BATCH_PAGED, {q->k, q->v, L.kpool, L.vpool, q->table}, {kvdim, R},
              {(uint32_t)c.block_size, (uint32_t)c.capacity, c.kv_dtype});
        b.add(YUUKA_OP_RMSNORM_HEADS_BATCH, {q->q, L.q_norm, q->q}, {hd, (uint64_t)c.heads, 2 * hd, R}, {}, {c.eps});
        b.add(YUUKA_OP_ROPE_BATCH, {q->q}, {(uint64_t)c.heads, 2 * hd, hd, (uint64_t)c.rope_dim, R, qdim}, {0},
              {(float)c.rope_base});
        b.add(YUUKA_OP_ATTENTION_PREFILL_PAGED, {q->q, L.kpool, L.vpool, q->attn, q->table},
              {(uint64_t)c.kv_heads, (uint64_t)c.heads, hd, kvdim, R, 0},
              {(uint32_t)c.block_size, (uint32_t)c.capacity, c.kv_dtype, 0}, {(float)(1.0 / std::sqrt((double)hd))});
    };
    for (int i = 0; i < c.n_layers; i++) {
        Layer &L = q->layers[i];
        if (fused) {
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
                recurrent_chunk(L, YUUKA_EXT_FLAG_RAW_OUT | YUUKA_EXT_FLAG_GDN_COEF);
                b.fused(q->gdn_out, nullptr, c.eps, R, {{&L.out, q->x, q->x}}, 1, 0, q->z, L.ssm_norm);
            } else {  // plan.go:684-804
                b.fused(q->x, L.attn_norm, c.eps, R,
                        {{&L.q, q->q, nullptr}, {&L.k, q->k, nullptr}, {&L.v, q->v, nullptr}}, 0);
                attention(L);
                b.fused(q->attn, nullptr, 0.0f, R, {{&L.o, q->x, q->x}}, 1);
            }
            // plan.go:915-988 FFN: norm + gate/up + SwiGLU in one op, down + residual
            b.fused(q->x, L.post_norm, c.eps, R, {{&L.ffn_gate, q->fg, nullptr}, {&L.ffn_up, nullptr, nullptr}}, 2);
            b.fused(q->fg, nullptr, 0.0f, R, {{&L.ffn_down, q->x, q->x}}, 1);
            continue;
        }
        b.add(YUUKA_OP_RMSNORM_BATCH, {q->x, L.attn_norm, q->xn}, {H, R, H, H}, {}, {c.eps});
        b.quant(q->xn, H, R, q->xq);
        if (L.recurrent) {
            b.gemm(L.qkv, q->xq, L.qkv_rows, R);
            b.gemm(L.gate, q->xq, q->z, R);
            b.gemm(L.beta, q->xq, L.beta_rows, R);
            b.gemm(L.alpha, q->xq, L.alpha_rows, R);
            recurrent_chunk(L, 0);
            b.quant(q->gdn_out, (uint64_t)c.inner, R, q->xq);
            b.gemm(L.out, q->xq, q->x, R, q->x);
        } else {
            b.gemm(L.q, q->xq, q->q, R);
            b.gemm(L.k, q->xq, q->k, R);
            b.gemm(L.v, q->xq, q->v, R);
            attention(L);
            b.quant(q->attn, odim, R, q->xq);
            b.gemm(L.o, q->xq, q->x, R, q->x);
        }
        b.add(YUUKA_OP_RMSNORM_BATCH, {q->x, L.post_norm, q->xn}, {H, R, H, H}, {}, {c.eps});
        b.quant(q->xn, H, R, q->xq);
        b.gemm(L.ffn_gate, q->xq, q->fg, R);
        b.gemm(L.ffn_up, q->xq, q->fu, R);
        b.add(YUUKA_OP_SILU_MUL, {q->fg, q->fu, q->fg}, {R * (uint64_t)c.ffn});
        b.quant(q->fg, (uint64_t)c.ffn, R, q->xq);
        b.gemm(L.ffn_down, q->xq, q->x, R, q->x);
    }
    // plan.go:635-662 all-logits tail
    if (fused) {
        b.fused(q->x, q->output_norm, c.eps, R, {{&q->output, q->logits, nullptr}}, 0);
    } else {
        b.add(YUUKA_OP_RMSNORM_BATCH, {q->x, q->output_norm, q->xn}, {H, R, H, H}, {}, {c.eps});
        b.quant(q->xn, H, R, q->xq);
        b.gemm(q->output, q->xq, q->logits, R);
    }
    if (mode == 0) {
        const yuuka_q35_accept &a = q->accept_cfg;
        // drafts are tokens[1..k]
        b.add(YUUKA_EXT_OP_ACCEPT, {q->logits, q->tokens, q->result, nullptr, q->step},
              {1, R - 1, (uint64_t)c.vocab, 0, a.seed, 0}, {a.mode, a.top_k, 0}, {a.temperature, a.top_p}, 0,
              {0, 4, 0, 0, 0});
    }
    for (int i = 0; i < c.n_layers; i++) {
        Layer &L = q->layers[i];
        if (!L.recurrent) continue;
        b.add(YUUKA_EXT_OP_GDN_COMMIT,
              {L.conv_state, L.mat_state, L.qkv_rows, L.conv_rows, L.alpha_rows, L.beta_rows, L.dt, L.a, q->result},
              {R, (uint64_t)c.groups, (uint64_t)c.rank, (uint64_t)c.state_size, (uint64_t)q->conv_dim,
               (uint64_t)c.inner},
              {(uint32_t)c.conv_kernel}, {}, fused ? YUUKA_EXT_FLAG_GDN_COEF : 0u);
    }
    b.add(YUUKA_EXT_OP_ADVANCE, {q->dyn, q->result, q->step}, {R});
    if (b.st != YUUKA_OK) {
        yuuka_plan_destroy(plan);
        return b.st;
    }
    *out = plan;
    return YUUKA_OK;
}

yuuka_status get_graph(yuuka_q35 *q, int rows, int mode, Graphs **out) {
    auto key = std::make_pair(rows, mode);
    auto it = q->plans.find(key);
    if (it == q->plans.end()) {
        Graphs g;
        yuuka_status st = build_plan(q, rows, mode, &g.plan);
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

void drop_graphs(yuuka_q35 *q) {
    for (auto &kv : q->plans) {
        yuuka_graph_destroy(kv.second.graph);
        yuuka_plan_destroy(kv.second.plan);
    }
    q->plans.clear();
}

// Runs one step over `rows` tokens (already in q->pinned). mode 1 presets
// result[0] = rows - 1 so the commit keeps every row.
yuuka_status run_step(yuuka_q35 *q, int rows, int mode, int32_t *result_out) {
    Graphs *g = nullptr;
    yuuka_status st = get_graph(q, rows, mode, &g);
    if (st != YUUKA_OK) return st;
    hipStream_t s = q->stream->stream;
    hipError_t err = hipMemcpyAsync(q->tokens->ptr, q->pinned, (size_t)rows * 4, hipMemcpyHostToDevice, s);
    if (err == hipSuccess && mode == 1) {
        q->pinned[16] = rows - 1;
        q->pinned[17] = -1;
        err = hipMemcpyAsync(q->result->ptr, q->pinned + 16, 8, hipMemcpyHostToDevice, s);
    }
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "token upload: %s", yk::hip_error(err));
    (void)hipEventRecord(q->ev0, s);
    if (g->graph)
        st = yuuka_graph_replay(g->graph, q->stream, nullptr);
    else
        st = yk::plan_run_dynamic(g->plan, s, static_cast<const int32_t *>(q->dyn->ptr));
    if (st != YUUKA_OK) return st;
    (void)hipEventRecord(q->ev1, s);
    err = hipMemcpyAsync(q->pinned + 16, q->result->ptr, 16, hipMemcpyDeviceToHost, s);
    if (err == hipSuccess) err = hipStreamSynchronize(s);
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "verify step: %s", yk::hip_error(err));
    (void)hipEventElapsedTime(&q->last_ms, q->ev0, q->ev1);
    q->last_rows = rows;
    if (result_out) std::memcpy(result_out, q->pinned + 16, 16);
    return YUUKA_OK;
}

int32_t read_pos(yuuka_q35 *q) {
    int32_t d[2] = {0, 0};
    (void)hipMemcpy(d, q->dyn->ptr, 8, hipMemcpyDeviceToHost);
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
        const yuuka_q35_config &c = *cfg;
        if (c.n_layers <= 0 || c.hidden <= 0 || c.ffn <= 0 || c.heads <= 0 || c.kv_heads <= 0 ||
            c.heads % c.kv_heads || c.vocab <= 0 || c.full_interval <= 0 || c.capacity <= 0 || c.block_size <= 0 ||
            c.max_rows < 1 || c.max_rows > 16 || c.conv_kernel < 2 || c.inner != c.rank * c.state_size)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "invalid qwen35 configuration");
        if (c.kv_dtype != YUUKA_DTYPE_F16 && c.kv_dtype != YUUKA_DTYPE_F32)
            return fail(YUUKA_ERR_UNSUPPORTED, "KV dtype %u", c.kv_dtype);
        std::unique_ptr<yuuka_q35> q(new yuuka_q35());
        q->dev = dev;
        q->cfg = c;
        q->conv_dim = 2 * c.groups * c.state_size + c.inner;
        yuuka_status st = yuuka_stream_create(dev, &q->stream);
        if (st != YUUKA_OK) return st;
        hipError_t err = hipHostMalloc(reinterpret_cast<void **>(&q->pinned), 32 * 4, hipHostMallocDefault);
        if (err != hipSuccess) return fail(YUUKA_ERR_ALLOCATION, "pinned staging: %s", yk::hip_error(err));
        q->eager = getenv("YUUKA_Q35_EAGER") && getenv("YUUKA_Q35_EAGER")[0] == '1';
        if (hipEventCreate(&q->ev0) != hipSuccess || hipEventCreate(&q->ev1) != hipSuccess)
            return fail(YUUKA_ERR_DEVICE, "timing events");
        const uint64_t H = c.hidden, M = c.max_rows, hd = c.head_dim;
        const uint64_t qdim = (uint64_t)c.heads * hd * 2, kvdim = (uint64_t)c.kv_heads * hd;
        const uint64_t cd = (uint64_t)q->conv_dim;
#define CHK(x)                           \
    do {                                 \
        yuuka_status s_ = (x);           \
        if (s_ != YUUKA_OK) {            \
            yuuka_q35_destroy(q.release()); \
            return s_;                   \
        }                                \
    } while (0)
        CHK(upload_tensor(q.get(), w->embedding, c.vocab, H, "token_embd", &q->embedding));
        CHK(upload_tensor(q.get(), w->output, c.vocab, H, "output", &q->output));
        CHK(upload_vec(q.get(), w->output_norm, H, "output_norm", &q->output_norm));
        q->layers.resize(c.n_layers);
        const int blocks = (c.capacity + c.block_size - 1) / c.block_size;
        const uint64_t kv_bytes = (uint64_t)blocks * c.block_size * kvdim * (c.kv_dtype == YUUKA_DTYPE_F16 ? 2 : 4);
        for (int i = 0; i < c.n_layers; i++) {
            const yuuka_q35_layer_weights &lw = w->layers[i];
            Layer &L = q->layers[i];
            L.recurrent = (i + 1) % c.full_interval != 0;  // config.go:280-282
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
                CHK(alloc(q.get(), (uint64_t)(c.conv_kernel - 1) * cd * 4, &L.conv_state));
                CHK(alloc(q.get(), (uint64_t)c.rank * c.state_size * c.state_size * 4, &L.mat_state));
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
            CHK(upload_tensor(q.get(), lw.ffn_gate, c.ffn, H, "ffn_gate", &L.ffn_gate));
            CHK(upload_tensor(q.get(), lw.ffn_up, c.ffn, H, "ffn_up", &L.ffn_up));
            CHK(upload_tensor(q.get(), lw.ffn_down, H, c.ffn, "ffn_down", &L.ffn_down));
        }
        const uint64_t kmax = std::max<uint64_t>({H, (uint64_t)c.ffn, (uint64_t)c.inner, (uint64_t)c.heads * hd});
        CHK(alloc(q.get(), M * H * 4, &q->x));
        CHK(alloc(q.get(), M * H * 4, &q->xn));
        CHK(alloc(q.get(), yk::gemm_plan(kmax, 1, M, YUUKA_DTYPE_Q4_K).xq_bytes + 256, &q->xq));
        CHK(alloc(q.get(), M * qdim * 4, &q->q));
        CHK(alloc(q.get(), M * kvdim * 4, &q->k));
        CHK(alloc(q.get(), M * kvdim * 4, &q->v));
        CHK(alloc(q.get(), M * c.heads * hd * 4, &q->attn));
        CHK(alloc(q.get(), M * (uint64_t)(c.rope_dim / 2) * 8, &q->rope));
        CHK(alloc(q.get(), M * c.inner * 4, &q->z));
        CHK(alloc(q.get(), M * c.inner * 4, &q->gdn_out));
        CHK(alloc(q.get(), M * c.ffn * 4, &q->fg));
        CHK(alloc(q.get(), M * c.ffn * 4, &q->fu));
        CHK(alloc(q.get(), M * (uint64_t)c.vocab * 4, &q->logits));
        CHK(alloc(q.get(), 64 * 4, &q->tokens));
        CHK(alloc(q.get(), 16, &q->result));
        CHK(alloc(q.get(), 16, &q->dyn));
        CHK(alloc(q.get(), 8, &q->step));
        // identity block table (memory/memory.go Table over a private pool)
        std::vector<int32_t> table(blocks);
        for (int i = 0; i < blocks; i++) table[i] = i;
        CHK(upload(q.get(), table.data(), (uint64_t)blocks * 4, &q->table));
        *out = q.release();
        return yuuka_q35_reset(*out);
#undef CHK
    });
}

void yuuka_q35_destroy(yuuka_q35 *q) {
    if (!q) return;
    if (q->stream) (void)hipStreamSynchronize(q->stream->stream);
    drop_graphs(q);
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
        hipStream_t s = q->stream->stream;
        for (auto &L : q->layers) {
            if (!L.recurrent) continue;
            (void)hipMemsetAsync(L.conv_state->ptr, 0, L.conv_state->bytes, s);
            (void)hipMemsetAsync(L.mat_state->ptr, 0, L.mat_state->bytes, s);
        }
        (void)hipMemsetAsync(q->dyn->ptr, 0, q->dyn->bytes, s);
        (void)hipMemsetAsync(q->step->ptr, 0, 8, s);
        hipError_t err = hipStreamSynchronize(s);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "reset: %s", yk::hip_error(err));
        return YUUKA_OK;
    });
}

float yuuka_q35_last_step_ms(const yuuka_q35 *q) { return q ? q->last_ms : 0.0f; }

int32_t yuuka_q35_position(const yuuka_q35 *q) { return q ? read_pos(const_cast<yuuka_q35 *>(q)) : -1; }

yuuka_status yuuka_q35_prefill(yuuka_q35 *q, const int32_t *tokens, int32_t n, float *last_logits) {
    return guard("q35_prefill", [&]() -> yuuka_status {
        if (!q || (!tokens && n)) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (n <= 0) return fail(YUUKA_ERR_INVALID_ARGUMENT, "empty token sequence");
        const int32_t pos = read_pos(q);
        if (pos + n > q->cfg.capacity)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "token sequence of %d exceeds remaining context %d", n,
                        q->cfg.capacity - pos);
        for (int i = 0; i < n; i++)
            if (tokens[i] < 0 || tokens[i] >= q->cfg.vocab)
                return fail(YUUKA_ERR_INVALID_ARGUMENT, "token id %d is out of range", tokens[i]);
        int done = 0;
        while (done < n) {
            const int rows = std::min(n - done, q->cfg.max_rows);
            std::memcpy(q->pinned, tokens + done, (size_t)rows * 4);
            yuuka_status st = run_step(q, rows, 1, nullptr);
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
    });
}

yuuka_status yuuka_q35_verify(yuuka_q35 *q, const int32_t *tokens, int32_t rows, const yuuka_q35_accept *accept,
                              int32_t *result) {
    return guard("q35_verify", [&]() -> yuuka_status {
        if (!q || !tokens || !accept) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        if (rows < 1 || rows > q->cfg.max_rows)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "verify rows %d outside 1..%d", rows, q->cfg.max_rows);
        for (int i = 0; i < rows; i++)
            if (tokens[i] < 0 || tokens[i] >= q->cfg.vocab)
                return fail(YUUKA_ERR_INVALID_ARGUMENT, "token id %d is out of range", tokens[i]);
        if (read_pos(q) + rows > q->cfg.capacity) return fail(YUUKA_ERR_INVALID_ARGUMENT, "context capacity exhausted");
        if (!q->accept_set || !same_accept(*accept, q->accept_cfg)) {
            // acceptance settings are baked into the captured graphs
            for (auto it = q->plans.begin(); it != q->plans.end();) {
                if (it->first.second == 0) {
                    yuuka_graph_destroy(it->second.graph);
                    yuuka_plan_destroy(it->second.plan);
                    it = q->plans.erase(it);
                } else {
                    ++it;
                }
            }
            q->accept_cfg = *accept;
            q->accept_set = true;
        }
        std::memcpy(q->pinned, tokens, (size_t)rows * 4);
        return run_step(q, rows, 0, result);
    });
}

yuuka_status yuuka_q35_logits(yuuka_q35 *q, float *out, int32_t rows) {
    return guard("q35_logits", [&]() -> yuuka_status {
        if (!q || !out || rows < 1 || rows > q->cfg.max_rows) return fail(YUUKA_ERR_INVALID_ARGUMENT, "bad arguments");
        hipError_t err = hipMemcpy(out, q->logits->ptr, (size_t)rows * q->cfg.vocab * 4, hipMemcpyDeviceToHost);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "logits copy: %s", yk::hip_error(err));
        return YUUKA_OK;
    });
}

uint64_t yuuka_q35_snapshot_bytes(const yuuka_q35 *q) {
    if (!q) return 0;
    uint64_t n = 0;
    for (auto &L : q->layers)
        if (L.recurrent) n += L.conv_state->bytes + L.mat_state->bytes;
    return n;
}

yuuka_status yuuka_q35_snapshot(yuuka_q35 *q, void *out, int32_t *position) {
    return guard("q35_snapshot", [&]() -> yuuka_status {
        if (!q || !out) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        uint8_t *p = static_cast<uint8_t *>(out);
        for (auto &L : q->layers) {
            if (!L.recurrent) continue;
            yuuka_status st = yuuka_memcpy_d2h(p, L.conv_state, L.conv_state->bytes);
            if (st != YUUKA_OK) return st;
            p += L.conv_state->bytes;
            st = yuuka_memcpy_d2h(p, L.mat_state, L.mat_state->bytes);
            if (st != YUUKA_OK) return st;
            p += L.mat_state->bytes;
        }
        if (position) *position = read_pos(q);
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
            yuuka_status st = yuuka_memcpy_h2d(L.conv_state, p, L.conv_state->bytes);
            if (st != YUUKA_OK) return st;
            p += L.conv_state->bytes;
            st = yuuka_memcpy_h2d(L.mat_state, p, L.mat_state->bytes);
            if (st != YUUKA_OK) return st;
            p += L.mat_state->bytes;
        }
        int32_t d[2] = {0, position};
        return yuuka_memcpy_h2d(q->dyn, d, 8);
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
        k = std::min(k, q->cfg.max_rows - 1);
        int min_match = o->min_match <= 0 ? 2 : std::min(o->min_match, 8);
        int max_tokens = std::min(o->max_tokens, q->cfg.capacity - n_prompt);
        if (max_tokens <= 0) return fail(YUUKA_ERR_INVALID_ARGUMENT, "no context space remains");
        yuuka_q35_generate_stats st_local{};
        yuuka_status st = yuuka_q35_reset(q);
        if (st != YUUKA_OK) return st;
        auto t0 = std::chrono::steady_clock::now();
        if (n_prompt > 1) {
            st = yuuka_q35_prefill(q, prompt, n_prompt - 1, nullptr);
            if (st != YUUKA_OK) return st;
        }
        auto t1 = std::chrono::steady_clock::now();
        std::vector<int32_t> history(prompt, prompt + n_prompt);
        int32_t pending = prompt[n_prompt - 1];
        int emitted = 0;
        bool stop = false;
        std::vector<int32_t> rows_tok(17);
        while (emitted < max_tokens && !stop) {
            const int32_t pos = read_pos(q);
            int limit = std::min(k, max_tokens - emitted);
            limit = std::min(limit, q->cfg.capacity - pos - 1);
            if (limit < 0) break;
            int32_t draft[16];
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
