// refmath.h — device versions of the reference decoder's scalar functions,
// evaluated the way the Go code evaluates them (float64 exp/log, then a
// float32 result).
#pragma once

#include <hip/hip_runtime.h>

namespace yk {

// 1/(1+float32(exp(float64(-x)))) as model/qwen35/forward.go:552-554.
__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + (float)exp((double)(-x))); }
__device__ __forceinline__ float silu_ref(float x) { return __fmul_rn(x, sigmoid_ref(x)); }
__device__ __forceinline__ float softplus_ref(float x) { return x > 20.0f ? x : (float)log1p(exp((double)x)); }

}  // namespace yk
