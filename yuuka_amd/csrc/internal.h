// internal.h — handle layouts, error plumbing and kernel launcher
// declarations shared by the ABI layer (bridge.cpp) and the kernel files.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/yuuka_hip.h"

struct yuuka_device {
    int index = 0;
    hipDeviceProp_t props{};
    void *noalloc_scratch = nullptr;  // this GPU's copy of the fixed accept scratch array
};

struct yuuka_buffer {
    yuuka_device *dev = nullptr;
    void *ptr = nullptr;
    uint64_t bytes = 0;
};

// Per-stream scratch: split-K partials, tickets and accept partials. Grown on
// demand outside any graph capture and released with the stream.
struct yk_scratch {
    void *ptr = nullptr;
    uint64_t bytes = 0;
};

struct yuuka_stream {
    yuuka_device *dev = nullptr;
    hipStream_t stream = nullptr;
    yk_scratch scratch;
    yk_scratch tickets;  // zero-initialised uint32 counters, self-resetting
};

struct yuuka_event {
    hipEvent_t event = nullptr;
};

namespace yk {

// Thread-local error message (reference bridge.cpp:47-57 convention).
yuuka_status fail(yuuka_status status, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
const char *hip_error(hipError_t err);

// Grows a stream scratch area to at least `bytes`; zero-fills new memory.
yuuka_status ensure_scratch(yuuka_stream *stream, yk_scratch *area, uint64_t bytes);

// GGUF row bytes for `cols` elements, or 0 when cols does not fit the block.
uint64_t row_bytes(uint32_t dtype, uint64_t cols);

// ---------------------------------------------------------------- GEMM
// Workspace needs of one verify GEMM call (bytes of partial sums and number
// of tickets), computed from the shape.
struct GemmPlan {
    int splits = 1;        // workgroups along K per 64-row block
    int sb_per_wave = 1;   // super-blocks per wave
    uint64_t xq_bytes = 0; // quantized activation block
    uint64_t part_bytes = 0;
    uint32_t tickets = 0;
};
GemmPlan gemm_plan(uint64_t n_in, uint64_t n_out, uint64_t rows, uint32_t dtype);

// Quantizes x[rows, n_in] (FP32) into the int8 hi/lo planes the GEMM reads.
hipError_t launch_quantize_x(const float *x, uint64_t n_in, uint64_t rows, void *xq,
                             hipStream_t stream);
// out[rows, n_out] = W * x using the planes written by launch_quantize_x.
hipError_t launch_gemm_q(const void *w, uint32_t dtype, const void *xq, float *out,
                         uint64_t n_in, uint64_t n_out, uint64_t rows, const GemmPlan &plan,
                         void *partials, uint32_t *tickets, hipStream_t stream,
                         const float *residual = nullptr);
hipError_t launch_dequant_f32(const void *src, uint32_t dtype, float *dst, uint64_t n_in,
                              uint64_t n_out, hipStream_t stream);
hipError_t launch_dequant_f16(const void *src, uint32_t dtype, uint16_t *dst, uint64_t n_in,
                              uint64_t n_out, hipStream_t stream);
hipError_t launch_cast_f16(const float *src, uint16_t *dst, uint64_t n, hipStream_t stream);

// --------------------------------------------------------------- accept
uint64_t accept_scratch_bytes(const yuuka_accept_params &p);
// ROUTER_NORMAL: logits [rows][E] <- i.i.d. N(0,1) (k_accept.hip).
hipError_t launch_router_normal(float *logits, int rows, int E, uint64_t seed, uint32_t layer, const uint64_t *step,
                                hipStream_t s);
hipError_t launch_verify_accept(const float *logits, const int32_t *drafts, int32_t *result,
                                double *debug, const yuuka_accept_params &p, void *scratch,
                                hipStream_t stream, const uint64_t *step_dev = nullptr, uint32_t draft_stride = 0,
                                const int32_t *forced = nullptr);

// ----------------------------------------------------------- small ops
hipError_t launch_add_f32(float *dst, const float *a, const float *b, uint64_t n,
                          hipStream_t stream);

}  // namespace yk
