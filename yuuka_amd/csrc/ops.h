// ops.h — validation and execution of the non-GEMM plan ops (norms, RoPE,
// embedding, paged KV write, paged attention, recurrent chunk, elementwise).
#pragma once

#include <cstdlib>

#include "plan.h"

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
// Two consecutive GEMM_FUSED ops over more than 8 rows where b normalises a's
// residual output run with a's split reduction and b's prologue in one
// launch; *done is false when they do not qualify (nothing was launched).
yuuka_status execute_gemm_pair(const yuuka_op &a, const yuuka_op &b, const ExecCtx &ctx, bool *done);

// Elementwise launchers (k_ops.hip).
hipError_t launch_copy_f32(float *dst, const float *src, uint64_t n, hipStream_t stream);
hipError_t launch_silu_mul(const float *gate, const float *up, float *out, uint64_t n,
                           hipStream_t stream);

}  // namespace yk
