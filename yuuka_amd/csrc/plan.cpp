// plan.cpp — yuuka_plan_* and yuuka_graph_* (reference yuuka_hip.h:477-496,
// bridge.cpp:3453-3870). Ops are validated and copied at add time; a rejected
// op is not appended. Execution submits every op on the caller's stream.
#include "plan.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <new>

#include "ops.h"

namespace yk {

static bool buf_ok(const yuuka_buffer *b, uint64_t off, uint64_t bytes) {
    return b != nullptr && off <= b->bytes && bytes <= b->bytes - off;
}

template <typename T>
static T *at(const yuuka_op &op, int i) {
    return reinterpret_cast<T *>(static_cast<uint8_t *>(op.buf[i]->ptr) + op.off[i]);
}

// ------------------------------------------------------------ validation

struct Need {
    uint64_t ws = 0;
    uint32_t tickets = 0;
};

// LM_HEAD / GEMV_BATCH as the fused verify GEMM (GEMM_FUSED with one
// segment and the store epilogue, no norm): the streaming kernel for up to 8
// rows, the many-row kernel beyond. True when that op serves the shape (its
// workspace in *ws); otherwise the split quantize + GEMM kernels run it.
static bool fused_form(const yuuka_op &op, yuuka_op *f, uint64_t *ws) {
    *f = yuuka_op{};
    f->code = YUUKA_EXT_OP_GEMM_FUSED;
    if (op.code == YUUKA_OP_GEMM_SWIGLU) {
        // hip.go:1149-1176: buf0 gate W, buf1 up W, buf2 x, buf3 out;
        // n = {K, N, rows}; out = SiLU(x gate^T) * (x up^T)
        f->buf[0] = op.buf[2];
        f->off[0] = op.off[2];
        f->buf[2] = op.buf[0];
        f->off[2] = op.off[0];
        f->buf[3] = op.buf[1];
        f->off[3] = op.off[1];
        f->buf[6] = op.buf[3];
        f->off[6] = op.off[3];
        f->n[0] = op.n[0];
        f->n[1] = op.n[2];
        f->n[2] = f->n[3] = op.n[1];
        f->u[0] = op.u[0] | (op.u[0] << 8);
        f->u[1] = 2;  // SwiGLU epilogue
        uint64_t need = 0;
        if (validate_model_op(*f, &need) != YUUKA_OK) return false;
        *ws = need;
        return true;
    }
    if (op.code == YUUKA_OP_GEMV_PAIR) {
        // hip.go:748-783: buf0 A, buf1 B, buf2 x, buf3 outA, buf4 outB;
        // n = {K, N_A, N_B}; u = {dtype A, dtype B, epilogue}: both rows
        // written (0) or outA = SiLU(A x) * (B x) (1)
        f->buf[0] = op.buf[2];
        f->off[0] = op.off[2];
        f->buf[2] = op.buf[0];
        f->off[2] = op.off[0];
        f->buf[3] = op.buf[1];
        f->off[3] = op.off[1];
        f->buf[6] = op.buf[3];
        f->off[6] = op.off[3];
        if (op.u[2] == 0) {
            f->buf[7] = op.buf[4];
            f->off[7] = op.off[4];
        } else if (op.u[2] != 1) {
            return false;
        }
        f->n[0] = op.n[0];
        f->n[1] = 1;
        f->n[2] = op.n[1];
        f->n[3] = op.n[2];
        f->u[0] = (op.u[0] & 0xff) | ((op.u[1] & 0xff) << 8);
        f->u[1] = op.u[2] == 1 ? 2 : 0;
        uint64_t need = 0;
        if (validate_model_op(*f, &need) != YUUKA_OK) return false;
        *ws = need;
        return true;
    }
    // LM_HEAD / GEMV_BATCH / GEMV (one row) / GEMV_RESIDUAL (hip.go:714-742:
    // buf3 the residual, out = W x + res)
    f->buf[0] = op.buf[1];
    f->off[0] = op.off[1];
    f->buf[2] = op.buf[0];
    f->off[2] = op.off[0];
    f->buf[6] = op.buf[2];
    f->off[6] = op.off[2];
    f->n[0] = op.n[0];
    f->n[1] = op.code == YUUKA_OP_GEMV ? 1 : op.n[2];
    f->n[2] = op.n[1];
    f->u[0] = op.u[0];
    if (op.code == YUUKA_OP_GEMV_RESIDUAL) {
        f->buf[10] = op.buf[3];
        f->off[10] = op.off[3];
        f->u[1] = 1;  // residual epilogue
    }
    uint64_t need = 0;
    if (validate_model_op(*f, &need) != YUUKA_OK) return false;
    *ws = need;
    return true;
}

static yuuka_status validate(const yuuka_op &op, Need *need) {
    switch (op.code) {
    case YUUKA_OP_GEMV_RESIDUAL:
    case YUUKA_OP_GEMV_PAIR: {
        // the single-token decode plan's fused projections (plan.go:84-149)
        for (int i = 0; i < 4; i++)
            if (!op.buf[i]) return fail(YUUKA_ERR_INVALID_ARGUMENT, "decode matvec buffer %d is null", i);
        if (op.code == YUUKA_OP_GEMV_PAIR && op.u[2] == 0 && !op.buf[4])
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "a matvec pair that writes both rows needs both outputs");
        const uint64_t rows = op.code == YUUKA_OP_GEMV_RESIDUAL ? op.n[2] : 1;
        yuuka_status st = check_verify_gemm(op.n[0], op.n[1], rows, op.u[0], 16);
        if (st == YUUKA_OK && op.code == YUUKA_OP_GEMV_PAIR) st = check_verify_gemm(op.n[0], op.n[2], 1, op.u[1], 1);
        if (st != YUUKA_OK) return st;
        yuuka_op f;
        if (!fused_form(op, &f, &need->ws))
            return fail(YUUKA_ERR_UNSUPPORTED, "decode matvec %u: shape %llux%llu is not served", op.code,
                        (unsigned long long)op.n[1], (unsigned long long)op.n[0]);
        return YUUKA_OK;
    }
    case YUUKA_OP_GEMV:
    case YUUKA_OP_LM_HEAD:
    case YUUKA_OP_GEMV_BATCH: {
        // LM_HEAD: buf0 W, buf1 x, buf2 out; n={K,N,rows}; u0 dtype (reference :385-387).
        // GEMV_BATCH (hip.go:492-520): buf0 W, buf1 x, buf2 out; n={K,N,batch}; u0 dtype.
        // GEMV (hip.go:449-472): the same for one row (n2 unused).
        for (int i = 0; i < 3; i++)
            if (!op.buf[i]) return fail(YUUKA_ERR_INVALID_ARGUMENT, "verify GEMM buffer %d is null", i);
        const uint64_t K = op.n[0], N = op.n[1], rows = op.code == YUUKA_OP_GEMV ? 1 : op.n[2];
        yuuka_status st = check_verify_gemm(K, N, rows, op.u[0], 16);
        if (st != YUUKA_OK) return st;
        if (op.off[0] % 16 || op.off[1] % 16 || op.off[2] % 4)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "verify GEMM offsets must be 16-byte aligned");
        if (!buf_ok(op.buf[0], op.off[0], row_bytes(op.u[0], K) * N))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "verify GEMM weight buffer is too small");
        if (!buf_ok(op.buf[1], op.off[1], K * rows * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "verify GEMM input buffer is too small");
        if (!buf_ok(op.buf[2], op.off[2], N * rows * 4))
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "verify GEMM output buffer is too small");
        yuuka_op f;
        if (fused_form(op, &f, &need->ws)) return YUUKA_OK;
        need->ws = verify_gemm_ws_bytes(K, N, rows, op.u[0]);
        need->tickets = verify_gemm_tickets(K, N, rows, op.u[0]);
        return YUUKA_OK;
    }
    case YUUKA_OP_GEMM_SWIGLU: {
        for (int i = 0; i < 4; i++)
            if (!op.buf[i]) return fail(YUUKA_ERR_INVALID_ARGUMENT, "GEMM_SWIGLU buffer %d is null", i);
        yuuka_status st = check_verify_gemm(op.n[0], op.n[1], op.n[2], op.u[0], 512);
        if (st != YUUKA_OK) return st;
        yuuka_op f;
        if (!fused_form(op, &f, &need->ws))
            return fail(YUUKA_ERR_UNSUPPORTED, "GEMM_SWIGLU shape %llux%llu at %llu rows is not served",
                        (unsigned long long)op.n[1], (unsigned long long)op.n[0], (unsigned long long)op.n[2]);
        return YUUKA_OK;
    }
    case YUUKA_OP_GEMM: {
        // hip.go:966-997 AddGemmPathAt (the WMMA route SelectPrefillPath
        // picks for 8..127 rows with few outputs): served for Q4_K / Q6_K
        // weights by the fused verify GEMM; F32/F16 weights are not.
        for (int i = 0; i < 3; i++)
            if (!op.buf[i]) return fail(YUUKA_ERR_INVALID_ARGUMENT, "GEMM buffer %d is null", i);
        const uint64_t K = op.n[0], N = op.n[1], rows = op.n[2];
        yuuka_status st = check_verify_gemm(K, N, rows, op.u[0], 512);
        if (st != YUUKA_OK) return st;
        yuuka_op f;
        if (!fused_form(op, &f, &need->ws))
            return fail(YUUKA_ERR_UNSUPPORTED, "GEMM shape %llux%llu at %llu rows is not served",
                        (unsigned long long)N, (unsigned long long)K, (unsigned long long)rows);
        return YUUKA_OK;
    }
    default:
        return validate_model_op(op, &need->ws);
    }
}

static yuuka_status execute(const yuuka_op &op, const ExecCtx &ctx) {
    switch (op.code) {
    case YUUKA_OP_GEMM_SWIGLU:
    case YUUKA_OP_GEMM: {
        yuuka_op f;
        uint64_t ws = 0;
        if (!fused_form(op, &f, &ws)) return fail(YUUKA_ERR_INTERNAL, "GEMM op changed after validation");
        return execute_model_op(f, ctx);
    }
    case YUUKA_OP_GEMV_RESIDUAL:
    case YUUKA_OP_GEMV_PAIR: {
        yuuka_op f;
        uint64_t ws = 0;
        if (!fused_form(op, &f, &ws)) return fail(YUUKA_ERR_INTERNAL, "decode matvec op changed after validation");
        return execute_model_op(f, ctx);
    }
    case YUUKA_OP_GEMV:
    case YUUKA_OP_LM_HEAD:
    case YUUKA_OP_GEMV_BATCH: {
        yuuka_op f;
        uint64_t ws = 0;
        if (fused_form(op, &f, &ws)) return execute_model_op(f, ctx);
        return run_verify_gemm(ctx.stream, at<const uint8_t>(op, 0), op.u[0], at<const float>(op, 1),
                               at<float>(op, 2), op.n[0], op.n[1], op.code == YUUKA_OP_GEMV ? 1 : op.n[2], ctx.ws,
                               ctx.tickets);
    }
    default:
        return execute_model_op(op, ctx);
    }
}

static yuuka_status prepare(yuuka_plan *plan) {
    if (plan->ws_bytes < plan->ws_need) {
        if (plan->ws) (void)hipFree(plan->ws);
        plan->ws = nullptr;
        plan->ws_bytes = 0;
        const uint64_t want = (plan->ws_need + 0xffffull) & ~0xffffull;
        hipError_t err = hipMalloc(&plan->ws, want);
        if (err != hipSuccess) return fail(YUUKA_ERR_ALLOCATION, "plan workspace: %s", hip_error(err));
        plan->ws_bytes = want;
    }
    // split-K tickets, then the chained GEMMs' counters in the last words
    if (plan->tickets_len < plan->ticket_need + 1) {
        if (plan->tickets) (void)hipFree(plan->tickets);
        plan->tickets = nullptr;
        const uint32_t want = plan->ticket_need + 64;
        hipError_t err = hipMalloc(reinterpret_cast<void **>(&plan->tickets), (size_t)want * 4);
        if (err == hipSuccess) err = hipMemset(plan->tickets, 0, (size_t)want * 4);
        if (err != hipSuccess) return fail(YUUKA_ERR_ALLOCATION, "plan tickets: %s", hip_error(err));
        plan->tickets_len = want;
    }
    return YUUKA_OK;
}

template <typename F>
static yuuka_status guard(F &&f) {
    try {
        return f();
    } catch (const std::bad_alloc &) {
        return fail(YUUKA_ERR_ALLOCATION, "host allocation failed");
    } catch (const std::exception &e) {
        return fail(YUUKA_ERR_INTERNAL, "%s", e.what());
    } catch (...) {
        return fail(YUUKA_ERR_INTERNAL, "unknown exception");
    }
}

static yuuka_status run_ops(yuuka_plan *plan, hipStream_t stream, int32_t token, uint32_t position,
                            const int32_t *dyn, int run_tail, uint32_t *codes, uint64_t *times,
                            uint64_t capacity, uint64_t *count) {
    ExecCtx ctx{stream, token, position, dyn, plan->ws, plan->tickets, plan->ws_bytes};
    ctx.part_off = plan->chain_quant ? (plan->chain_quant + 255) & ~255ull : 0;
    uint64_t n = 0;
    hipEvent_t a = nullptr, b = nullptr;
    if (times) {
        if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess)
            return fail(YUUKA_ERR_DEVICE, "profiling events");
    }
    yuuka_status st = YUUKA_OK;
    const int nops = (int)plan->ops.size();
    for (int oi = 0; oi < nops; oi++) {
        const yuuka_op &op = plan->ops[oi];
        if ((op.flags & YUUKA_OP_FLAG_TAIL) && !run_tail) continue;
        if (!times && op.code == YUUKA_EXT_OP_GDN_COMMIT) {
            // consecutive per-layer commits go out as one launch
            int run = gdn_commit_run(&plan->ops[oi], nops - oi);
            for (int k = 1; k < run; k++)
                if ((plan->ops[oi + k].flags & YUUKA_OP_FLAG_TAIL) && !run_tail) run = k;
            for (int k = 0; k < run && st == YUUKA_OK; k++)
                for (int i = 0; i < 16; i++)
                    if (plan->ops[oi + k].buf[i] && !plan->ops[oi + k].buf[i]->ptr)
                        st = fail(YUUKA_ERR_INVALID_ARGUMENT, "plan op %u has a freed buffer", op.code);
            if (st != YUUKA_OK) break;
            if (run > 1) {
                st = execute_gdn_commit_run(&plan->ops[oi], run, ctx);
                if (st != YUUKA_OK) break;
                n += run;
                oi += run - 1;
                continue;
            }
        }
        for (int i = 0; i < 16; i++)
            if (op.buf[i] && !op.buf[i]->ptr) {
                st = fail(YUUKA_ERR_INVALID_ARGUMENT, "plan op %u has a freed buffer", op.code);
                break;
            }
        if (st != YUUKA_OK) break;
        auto usable = [&](int k) {
            if ((plan->ops[k].flags & YUUKA_OP_FLAG_TAIL) && !run_tail) return false;
            for (int i = 0; i < 16; i++)
                if (plan->ops[k].buf[i] && !plan->ops[k].buf[i]->ptr) return false;
            return true;
        };
        if (!times && ctx.part_off && gemm_chain_member(op)) {
            // a run of many-row GEMMs: split reductions inside the next
            // member's prologue (and a following RMSNorm of the last output)
            int j = 1;
            while (oi + j < nops && gemm_chain_member(plan->ops[oi + j]) && usable(oi + j)) j++;
            const yuuka_op *after = oi + j < nops && usable(oi + j) ? &plan->ops[oi + j] : nullptr;
            if (j > 1 || (after && after->code == YUUKA_OP_RMSNORM_BATCH)) {
                bool after_done = false;
                st = execute_gemm_chain(&plan->ops[oi], j, after, ctx, &after_done);
                if (st != YUUKA_OK) break;
                n += j + (after_done ? 1 : 0);
                oi += j - 1 + (after_done ? 1 : 0);
                continue;
            }
        }
        if (times) (void)hipEventRecord(a, stream);
        st = execute(op, ctx);
        if (st != YUUKA_OK) break;
        if (times) {
            (void)hipEventRecord(b, stream);
            (void)hipEventSynchronize(b);
            float ms = 0.0f;
            (void)hipEventElapsedTime(&ms, a, b);
            if (n < capacity) {
                codes[n] = op.code;
                times[n] = (uint64_t)((double)ms * 1e6);
            }
        }
        n++;
    }
    if (times) {
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
    }
    if (count) *count = n;
    return st;
}

}  // namespace yk

using namespace yk;

namespace yk {
yuuka_status verify_gemm_op_needs(const yuuka_op &op, uint64_t *ws, uint32_t *tickets) {
    Need need;
    yuuka_status st = validate(op, &need);
    *ws = need.ws;
    *tickets = need.tickets;
    return st;
}

yuuka_status run_verify_gemm_op(const yuuka_op &op, hipStream_t stream, void *ws, uint32_t *tickets) {
    ExecCtx ctx{stream, 0, 0, nullptr, ws, tickets};
    return execute(op, ctx);
}

yuuka_status plan_run_dynamic(yuuka_plan *plan, hipStream_t stream, const int32_t *dyn) {
    yuuka_status st = prepare(plan);
    if (st != YUUKA_OK) return st;
    return run_ops(plan, stream, 0, 0, dyn, 1, nullptr, nullptr, 0, nullptr);
}
}  // namespace yk

extern "C" {

yuuka_status yuuka_plan_create(yuuka_device *dev, yuuka_plan **out) {
    return guard([&]() -> yuuka_status {
        if (!dev || !out) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null device or output");
        auto *p = new yuuka_plan();
        p->dev = dev;
        *out = p;
        return YUUKA_OK;
    });
}

void yuuka_plan_destroy(yuuka_plan *plan) {
    if (!plan) return;
    (void)hipDeviceSynchronize();
    if (plan->ws) (void)hipFree(plan->ws);
    if (plan->tickets) (void)hipFree(plan->tickets);
    delete plan;
}

yuuka_status yuuka_plan_add(yuuka_plan *plan, const yuuka_op *op) {
    return guard([&]() -> yuuka_status {
        if (!plan || !op) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null plan or op");
        Need need;
        yuuka_status st = validate(*op, &need);
        if (st != YUUKA_OK) return st;
        plan->ops.push_back(*op);
        plan->ws_need = std::max(plan->ws_need, need.ws);
        uint64_t q = 0, p = 0;
        if (gemm_chain_ws(*op, &q, &p)) {  // runs of them share one layout
            plan->chain_quant = std::max(plan->chain_quant, q);
            plan->chain_part = std::max(plan->chain_part, p);
            plan->ws_need = std::max<uint64_t>(plan->ws_need, ((plan->chain_quant + 255) & ~255ull) + plan->chain_part + 256);
        }
        plan->ticket_need = std::max(plan->ticket_need, need.tickets);
        return YUUKA_OK;
    });
}

yuuka_status yuuka_plan_execute(yuuka_plan *plan, yuuka_stream *stream, int32_t token,
                                uint32_t position, int run_tail, yuuka_event *completion) {
    return guard([&]() -> yuuka_status {
        if (!plan || !stream) return fail(YUUKA_ERR_INVALID_ARGUMENT, "plan or stream is null");
        yuuka_status st = prepare(plan);
        if (st != YUUKA_OK) return st;
        st = run_ops(plan, stream->stream, token, position, nullptr, run_tail, nullptr, nullptr, 0, nullptr);
        if (st != YUUKA_OK) return st;
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "plan execute: %s", hip_error(err));
        if (completion) {
            err = hipEventRecord(completion->event, stream->stream);
            if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "event record: %s", hip_error(err));
        }
        return YUUKA_OK;
    });
}

yuuka_status yuuka_plan_execute_profiled(yuuka_plan *plan, yuuka_stream *stream, int32_t token,
                                         uint32_t position, int run_tail, uint32_t *op_codes,
                                         uint64_t *op_times_ns, uint64_t capacity,
                                         uint64_t *op_count, yuuka_event *completion) {
    return guard([&]() -> yuuka_status {
        if (!plan || !stream || !op_codes || !op_times_ns || !op_count)
            return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        yuuka_status st = prepare(plan);
        if (st != YUUKA_OK) return st;
        st = run_ops(plan, stream->stream, token, position, nullptr, run_tail, op_codes, op_times_ns,
                     capacity, op_count);
        if (st != YUUKA_OK) return st;
        if (completion) {
            hipError_t err = hipEventRecord(completion->event, stream->stream);
            if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "event record: %s", hip_error(err));
        }
        return YUUKA_OK;
    });
}

// Captures the plan into a HIP graph. Position-dependent ops read {token,
// position} from `dynamic` (written by yuuka_dynamic_set) at replay time.
yuuka_status yuuka_graph_create(yuuka_plan *plan, yuuka_stream *stream, yuuka_buffer *dynamic,
                                int run_tail, yuuka_graph **out) {
    return guard([&]() -> yuuka_status {
        if (!plan || !stream || !out) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        *out = nullptr;
        if (dynamic && dynamic->bytes < 8) return fail(YUUKA_ERR_INVALID_ARGUMENT, "dynamic buffer under 8 bytes");
        for (const yuuka_op &op : plan->ops)
            if (op_uses_position(op) && !dynamic)
                return fail(YUUKA_ERR_UNSUPPORTED, "plan op %u needs a dynamic-parameter buffer", op.code);
        yuuka_status st = prepare(plan);
        if (st != YUUKA_OK) return st;
        hipError_t err = hipStreamSynchronize(stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "pre-capture sync: %s", hip_error(err));
        err = hipStreamBeginCapture(stream->stream, hipStreamCaptureModeThreadLocal);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "begin capture: %s", hip_error(err));
        const int32_t *dyn = dynamic ? static_cast<const int32_t *>(dynamic->ptr) : nullptr;
        st = run_ops(plan, stream->stream, 0, 0, dyn, run_tail, nullptr, nullptr, 0, nullptr);
        hipGraph_t graph = nullptr;
        err = hipStreamEndCapture(stream->stream, &graph);
        if (st != YUUKA_OK) {
            if (graph) (void)hipGraphDestroy(graph);
            return st;
        }
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "end capture: %s", hip_error(err));
        hipGraphExec_t exec = nullptr;
        err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (err != hipSuccess) {
            (void)hipGraphDestroy(graph);
            return fail(YUUKA_ERR_DEVICE, "graph instantiate: %s", hip_error(err));
        }
        auto *g = new yuuka_graph();
        g->graph = graph;
        g->exec = exec;
        *out = g;
        return YUUKA_OK;
    });
}

yuuka_status yuuka_graph_replay(yuuka_graph *graph, yuuka_stream *stream, yuuka_event *completion) {
    return guard([&]() -> yuuka_status {
        if (!graph || !stream) return fail(YUUKA_ERR_INVALID_ARGUMENT, "null argument");
        hipError_t err = hipGraphLaunch(graph->exec, stream->stream);
        if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "graph launch: %s", hip_error(err));
        if (completion) {
            err = hipEventRecord(completion->event, stream->stream);
            if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "event record: %s", hip_error(err));
        }
        return YUUKA_OK;
    });
}

void yuuka_graph_destroy(yuuka_graph *graph) {
    if (!graph) return;
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
}

}  // extern "C"
