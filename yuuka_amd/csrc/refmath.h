// refmath.h — device versions of the reference decoder's scalar functions,
// evaluated the way the Go code evaluates them (float64 exp/log, then a
// float32 result).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

namespace yk {

// 1/(1+float32(exp(float64(-x)))) as model/qwen35/forward.go:552-554.
__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + (float)exp((double)(-x))); }
__device__ __forceinline__ float silu_ref(float x) { return __fmul_rn(x, sigmoid_ref(x)); }
// SiLU with a float32 exp (the device library's expf, within 1 ulp of the
// rounded float64 exp) where the float64 exp is on a latency-critical path;
// the sigmoid then differs from sigmoid_ref by at most an ulp or two.
__device__ __forceinline__ float silu_f32(float x) { return __fmul_rn(x, 1.0f / (1.0f + expf(-x))); }
__device__ __forceinline__ float softplus_ref(float x) { return x > 20.0f ? x : (float)log1p(exp((double)x)); }

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// tensor/half.go:35-68 Float32ToFloat16 (round half up on the dropped bits,
// as the reference does; not round-to-nearest-even).
__device__ __forceinline__ uint16_t ref_f32_to_f16(float f) {
    const uint32_t b = __float_as_uint(f);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    int32_t exp = (int32_t)((b >> 23) & 0xffu) - 127;
    const uint32_t mant = b & 0x7fffffu;
    if (exp == 128) return mant ? (uint16_t)(sign | 0x7e00u) : (uint16_t)(sign | 0x7c00u);
    if (exp > 15) return (uint16_t)(sign | 0x7c00u);
    if (exp < -24) return sign;
    if (exp < -14) {
        const uint32_t shift = (uint32_t)(-exp - 14);
        const uint32_t full = mant | 0x800000u;
        const uint32_t rounded = full + (1u << (shift + 12));
        return (uint16_t)(sign | (uint16_t)(rounded >> (shift + 13)));
    }
    uint32_t rounded = mant + 0x1000u;
    if (rounded & 0x800000u) {
        exp++;
        rounded = 0;
        if (exp > 15) return (uint16_t)(sign | 0x7c00u);
    }
    return (uint16_t)(sign | (uint16_t)((exp + 15) << 10) | (uint16_t)(rounded >> 13));
}

}  // namespace yk
