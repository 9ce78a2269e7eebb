// ops.cpp — plan-op validation and dispatch for the non-GEMM ops. Buffer
// layouts follow the reference header comments (yuuka_hip.h:336-476) and the
// Go builders (backend/hip/hip.go).
#include "ops.h"

namespace yk {

static bool buf_ok(const yuuka_buffer *b, uint64_t off, uint64_t bytes) {
    return b != nullptr && off <= b->bytes && bytes <= b->bytes - off;
}

template <typename T>
static T *at(const yuuka_op &op, int i) {
    return reinterpret_cast<T *>(static_cast<uint8_t *>(op.buf[i]->ptr) + op.off[i]);
}

bool op_uses_position(const yuuka_op &op) {
    switch (op.code) {
    case YUUKA_OP_ROPE_BATCH:
    case YUUKA_OP_KV_WRITE_BATCH_PAGED:
    case YUUKA_OP_ATTENTION_PREFILL_PAGED:
        return true;
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
    default:
        return fail(YUUKA_ERR_UNSUPPORTED, "plan op code %u is not served by this library", op.code);
    }
}

yuuka_status execute_model_op(const yuuka_op &op, const ExecCtx &ctx) {
    hipError_t err = hipSuccess;
    switch (op.code) {
    case YUUKA_OP_ADD:
        err = launch_add_f32(at<float>(op, 0), at<const float>(op, 0), at<const float>(op, 1), op.n[0], ctx.stream);
        break;
    case YUUKA_OP_COPY:
        err = launch_copy_f32(at<float>(op, 0), at<const float>(op, 1), op.n[0], ctx.stream);
        break;
    case YUUKA_OP_SILU_MUL:
        err = launch_silu_mul(at<const float>(op, 0), at<const float>(op, 1), at<float>(op, 2), op.n[0], ctx.stream);
        break;
    default:
        return fail(YUUKA_ERR_UNSUPPORTED, "plan op code %u is not served by this library", op.code);
    }
    if (err != hipSuccess) return fail(YUUKA_ERR_DEVICE, "op %u launch: %s", op.code, hip_error(err));
    return YUUKA_OK;
}

}  // namespace yk
