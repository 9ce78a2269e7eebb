// k_decode.hip — one-row helpers of the reference's single-token decode plan
// (engine/gpu/plan.go:238-307 buildDecodePlan) that have no batched
// counterpart here: SCALE, the legacy per-head L2 norm, and the Q8_1
// activation format of the int8 decode matvec (QUANT_Q8_1,
// SILU_MUL_QUANT_Q8_1, and its dequantization feeding GEMV_Q8_1). The other
// decode ops run as one-row forms of the verify kernels (ops.cpp).
#include <hip/hip_runtime.h>

#include "ops.h"
#include "refmath.h"

namespace yk {
namespace {

__global__ __launch_bounds__(256) void scale_kernel(float *__restrict__ x, uint64_t n, float s) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = __fmul_rn(x[i], s);
}

// forward.go:484-493 l2NormHead per head: float64 sum of squares, scale =
// float32(1 / sqrt(sum + eps)) * extra. One workgroup per head.
__global__ __launch_bounds__(256) void l2norm_heads_kernel(const float *__restrict__ src, float *__restrict__ dst,
                                                           int size, uint64_t stride, float eps, float extra) {
    __shared__ double red[4];
    const float *x = src + blockIdx.x * stride;
    double s = 0.0;
    for (int c = threadIdx.x; c < size; c += 256) s += (double)x[c] * (double)x[c];
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    s = (red[0] + red[1]) + (red[2] + red[3]);
    const float scale = __fmul_rn((float)(1.0 / sqrt(s + (double)eps)), extra);
    float *y = dst + blockIdx.x * stride;
    __syncthreads();  // in place: every read of x is done
    for (int c = threadIdx.x; c < size; c += 256) y[c] = __fmul_rn(x[c], scale);
}

// Q8_1 activations (the reference's int8 decode format): per 32 values, int8
// digits q = clamp(rint(v * 127 / amax), -127, 127) and the pair {d = amax /
// 127, d * sum(q)}. One thread per 32-value block; with `up` the values are
// SiLU(gate) * up first (forward.go:306-308).
__global__ __launch_bounds__(256) void quant_q8_1_kernel(const float *__restrict__ x, const float *__restrict__ up,
                                                         int8_t *__restrict__ qs, float2 *__restrict__ ds,
                                                         uint64_t blocks) {
    const uint64_t b = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= blocks) return;
    float v[32];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        float t = x[b * 32 + i];
        if (up) t = __fmul_rn(__fmul_rn(t, sigmoid_ref(t)), up[b * 32 + i]);
        v[i] = t;
        amax = fmaxf(amax, fabsf(t));
    }
    const float d = amax / 127.0f;
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    int sum = 0;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const int q = (int)fmaxf(-127.0f, fminf(127.0f, rintf(v[i] * inv)));
        qs[b * 32 + i] = (int8_t)q;
        sum += q;
    }
    ds[b] = make_float2(d, d * (float)sum);
}

// x = q * d per Q8_1 block (exact: |q| <= 127 times an FP32 scale).
__global__ __launch_bounds__(256) void dequant_q8_1_kernel(const int8_t *__restrict__ qs, const float2 *__restrict__ ds,
                                                           float *__restrict__ x, uint64_t n) {
    const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) x[i] = __fmul_rn((float)qs[i], ds[i / 32].x);
}

unsigned grid_of(uint64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

hipError_t launch_scale_f32(float *x, uint64_t n, float s, hipStream_t stream) {
    if (n) scale_kernel<<<grid_of(n), 256, 0, stream>>>(x, n, s);
    return hipGetLastError();
}

hipError_t launch_l2norm_heads(const float *src, float *dst, int heads, int size, uint64_t stride, float eps,
                               float extra, hipStream_t stream) {
    if (heads > 0) l2norm_heads_kernel<<<(unsigned)heads, 256, 0, stream>>>(src, dst, size, stride, eps, extra);
    return hipGetLastError();
}

hipError_t launch_quant_q8_1(const float *x, const float *up, void *qs, void *ds, uint64_t n, hipStream_t stream) {
    const uint64_t blocks = n / 32;
    if (blocks)
        quant_q8_1_kernel<<<grid_of(blocks), 256, 0, stream>>>(x, up, static_cast<int8_t *>(qs),
                                                               static_cast<float2 *>(ds), blocks);
    return hipGetLastError();
}

hipError_t launch_dequant_q8_1(const void *qs, const void *ds, float *x, uint64_t n, hipStream_t stream) {
    if (n)
        dequant_q8_1_kernel<<<grid_of(n), 256, 0, stream>>>(static_cast<const int8_t *>(qs),
                                                            static_cast<const float2 *>(ds), x, n);
    return hipGetLastError();
}

}  // namespace yk
