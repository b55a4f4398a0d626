// Correctly rounded fp32 arithmetic helpers for device code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bm {

// Correctly rounded fp32 sqrt (the device's v_sqrt_f32 is not).  The result
// is first taken from an fp64 evaluation rounded to fp32, then checked
// exactly: the two midpoints around the candidate have 25 significant bits,
// so midpoint*midpoint is exact in fp64 and decides whether the true value
// lies below, inside or above the candidate's rounding interval (a true
// value can never sit exactly on a midpoint for an fp32 operand).
__device__ __forceinline__ float next_up_pos(float v) { return __int_as_float(__float_as_int(v) + 1); }
__device__ __forceinline__ float next_dn_pos(float v) { return __int_as_float(__float_as_int(v) - 1); }

// (branch-free: both corrections are computed and selected)
__device__ __forceinline__ float cr_sqrtf(float x) {
  const float s = (float)__builtin_sqrt((double)x);
  const bool simple = !(x > 0.0f) || !(s < 3.0e38f) || !(s > 1.0e-30f);
  const double xd = (double)x;
  const float up = next_up_pos(s), dn = next_dn_pos(s);
  const double mhi = 0.5 * ((double)s + (double)up), mlo = 0.5 * ((double)s + (double)dn);
  float r = s;
  r = xd > mhi * mhi ? up : r;
  r = xd < mlo * mlo ? dn : r;
  return simple ? s : r;
}

// Correctly rounded fp32 division: the IEEE sequence (v_div_scale,
// v_rcp_f32 refined by fma steps, v_div_fmas, v_div_fixup) that the compiler
// emits for `/` with -fhip-fp32-correctly-rounded-divide-sqrt, which the
// build passes explicitly; denormal operands and results are kept.
__device__ __forceinline__ float cr_divf(float a, float b) { return a / b; }

}  // namespace bm
