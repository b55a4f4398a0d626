// Correctly rounded fp32 arithmetic helpers for device code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bm {

// Correctly rounded fp32 sqrt: v_sqrt_f32 (not correctly rounded by itself)
// followed by the exact residual test of its two neighbours, the sequence
// the compiler emits for sqrtf with -fhip-fp32-correctly-rounded-divide-sqrt,
// which the build passes explicitly.
__device__ __forceinline__ float cr_sqrtf(float x) { return sqrtf(x); }

// Correctly rounded fp32 division: the IEEE sequence (v_div_scale,
// v_rcp_f32 refined by fma steps, v_div_fmas, v_div_fixup) that the compiler
// emits for `/` with -fhip-fp32-correctly-rounded-divide-sqrt, which the
// build passes explicitly; denormal operands and results are kept.
__device__ __forceinline__ float cr_divf(float a, float b) { return a / b; }

}  // namespace bm
