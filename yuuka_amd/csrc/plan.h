// plan.h — recorded op lists (yuuka_plan) and captured graphs (yuuka_graph).
#pragma once

#include <vector>

#include "internal.h"

struct yuuka_plan {
    yuuka_device *dev = nullptr;
    std::vector<yuuka_op> ops;
    uint64_t ws_need = 0;      // bytes of op workspace (max over ops)
    uint64_t chain_quant = 0;  // many-row GEMMs: largest quantized-row area
    uint64_t chain_part = 0;   // and largest split partial-sum area (chained layout)
    uint32_t ticket_need = 0;  // split-K tickets (max over ops)
    void *ws = nullptr;
    uint64_t ws_bytes = 0;
    uint32_t *tickets = nullptr;
    uint32_t tickets_len = 0;
};

struct yuuka_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace yk {

yuuka_status check_verify_gemm(uint64_t n_in, uint64_t n_out, uint64_t rows, uint32_t dtype,
                               uint64_t max_rows);
yuuka_status run_verify_gemm(hipStream_t stream, const void *w, uint32_t dtype, const float *x,
                             float *out, uint64_t n_in, uint64_t n_out, uint64_t rows, void *ws,
                             uint32_t *tickets);
uint64_t verify_gemm_ws_bytes(uint64_t n_in, uint64_t n_out, uint64_t rows, uint32_t dtype);
uint32_t verify_gemm_tickets(uint64_t n_in, uint64_t n_out, uint64_t rows, uint32_t dtype);

// An LM_HEAD / GEMV_BATCH op outside a plan (yuuka_lm_head, yuuka_gemv*):
// validation with its workspace and ticket needs, then execution on `stream`
// (the fused verify GEMM where it serves the shape).
yuuka_status verify_gemm_op_needs(const yuuka_op &op, uint64_t *ws, uint32_t *tickets);
yuuka_status run_verify_gemm_op(const yuuka_op &op, hipStream_t stream, void *ws, uint32_t *tickets);

// Runs the plan's ops directly on `stream` (no graph), reading {token,
// position} from the device buffer `dyn` exactly as a captured graph would.
yuuka_status plan_run_dynamic(yuuka_plan *plan, hipStream_t stream, const int32_t *dyn);

// Execution context handed to op executors.
struct ExecCtx {
    hipStream_t stream;
    int32_t token;
    uint32_t position;
    const int32_t *dyn;  // device {token, position} for graph replay, or null
    void *ws;
    uint32_t *tickets;
    uint64_t ws_bytes = 0;  // size of ws (0: unknown, no op pairs fused)
    uint64_t part_off = 0;  // many-row GEMM runs: partial sums at ws + part_off (0: not chained)
};

}  // namespace yk
