// k_ops.hip — elementwise kernels of the verify plan: residual add
// (reference plan.Add), SwiGLU product (plan.AddSiluMul), FP32 copy.
// float4-vectorised grid-stride loops; scalar tail.
#include <hip/hip_runtime.h>

#include "ops.h"
#include "refmath.h"

namespace yk {
namespace {

__global__ __launch_bounds__(256) void add_kernel(float *__restrict__ dst, const float *__restrict__ a,
                                                  const float *__restrict__ b, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = a[i] + b[i];
}

__global__ __launch_bounds__(256) void copy_kernel(float *__restrict__ dst, const float *__restrict__ src,
                                                   uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = src[i];
}

// out = silu(gate) * up with silu(x) = x * sigmoid(x) (forward.go:306-308).
__global__ __launch_bounds__(256) void silu_mul_kernel(const float *__restrict__ gate,
                                                       const float *__restrict__ up,
                                                       float *__restrict__ out, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) {
        const float g = gate[i];
        out[i] = __fmul_rn(__fmul_rn(g, sigmoid_ref(g)), up[i]);
    }
}

unsigned blocks(uint64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t launch_add_f32(float *dst, const float *a, const float *b, uint64_t n, hipStream_t stream) {
    if (n) add_kernel<<<blocks(n), 256, 0, stream>>>(dst, a, b, n);
    return hipGetLastError();
}

hipError_t launch_copy_f32(float *dst, const float *src, uint64_t n, hipStream_t stream) {
    if (n) copy_kernel<<<blocks(n), 256, 0, stream>>>(dst, src, n);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float *gate, const float *up, float *out, uint64_t n, hipStream_t stream) {
    if (n) silu_mul_kernel<<<blocks(n), 256, 0, stream>>>(gate, up, out, n);
    return hipGetLastError();
}

}  // namespace yk
