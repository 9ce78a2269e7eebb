// ops.h — validation and execution of the non-GEMM plan ops (norms, RoPE,
// embedding, paged KV write, paged attention, recurrent chunk, elementwise).
#pragma once

#include <cstdlib>

#include "plan.h"
#include "fgemm.h"

namespace yk {

// Validates a plan op other than LM_HEAD/GEMV_BATCH; *ws receives the
// workspace bytes it needs. Unknown codes fail with YUUKA_ERR_UNSUPPORTED.
yuuka_status validate_model_op(const yuuka_op &op, uint64_t *ws);
yuuka_status execute_model_op(const yuuka_op &op, const ExecCtx &ctx);
// True when the op reads the execution position (graph capture then needs
// the dynamic-parameter buffer).
bool op_uses_position(const yuuka_op &op);
// Length of the run of consecutive GDN_COMMIT ops starting at ops[0] that
// one multi-layer launch can serve (same shape, flags and acceptance
// result), 1 when there is none to merge.
int gdn_commit_run(const yuuka_op *ops, int count);
yuuka_status execute_gdn_commit_run(const yuuka_op *ops, int count, const ExecCtx &ctx);
// GEMM_FUSED over more than 8 rows (the many-row kernel), and its workspace
// in two parts (quantized rows, split partial sums).
bool gemm_chain_member(const yuuka_op &op);
bool gemm_chain_ws(const yuuka_op &op, uint64_t *quant, uint64_t *part);
// A run of n consecutive many-row GEMM_FUSED ops (launch_fused_gemm_rows_chain:
// each split reduction inside the next member's prologue where they link),
// with ctx.part_off the run's common partial-sum offset. `after` (may be
// null) is the op that follows the run: an RMSNORM_BATCH of the last
// member's residual output takes its split reduction too (*after_done).
yuuka_status execute_gemm_chain(const yuuka_op *ops, int n, const yuuka_op *after, const ExecCtx &ctx,
                                bool *after_done);

// Elementwise launchers (k_ops.hip).
hipError_t launch_copy_f32(float *dst, const float *src, uint64_t n, hipStream_t stream);
// One-row decode helpers (k_decode.hip).
hipError_t launch_scale_f32(float *x, uint64_t n, float s, hipStream_t stream);
hipError_t launch_l2norm_heads(const float *src, float *dst, int heads, int size, uint64_t stride, float eps,
                               float extra, hipStream_t stream);
// Q8_1: n values (n % 32 == 0) -> int8 digits qs[n], {d, d * sum} pairs ds[n / 32];
// with `up`, the values are SiLU(x) * up.
hipError_t launch_quant_q8_1(const float *x, const float *up, void *qs, void *ds, uint64_t n, hipStream_t stream);
hipError_t launch_dequant_q8_1(const void *qs, const void *ds, float *x, uint64_t n, hipStream_t stream);
hipError_t launch_silu_mul(const float *gate, const float *up, float *out, uint64_t n,
                           hipStream_t stream);

}  // namespace yk
