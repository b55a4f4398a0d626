// Correctly rounded fp32 arithmetic helpers for device code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bm {

// Correctly rounded fp32 sqrt and division (the device's v_sqrt_f32 and
// v_rcp_f32 are not).  The result is first taken from an fp64 evaluation
// rounded to fp32, then checked exactly: the two midpoints around the
// candidate have 25 significant bits, so midpoint*midpoint and
// midpoint*|b| are exact in fp64 and decide whether the true value lies
// below, inside or above the candidate's rounding interval (a true value
// can never sit exactly on a midpoint for fp32 operands).
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

__device__ __forceinline__ float cr_divf(float a, float b) {
  const float q = (float)((double)a / (double)b);
  const float aq = fabsf(q);
  const bool simple =
      a == 0.0f || !(aq < 3.0e38f) || !(aq > 1.0e-30f) || !(fabsf(b) < 3.0e38f);
  const double ad = fabs((double)a), bd = fabs((double)b);
  const float up = next_up_pos(aq), dn = next_dn_pos(aq);
  const double mhi = 0.5 * ((double)aq + (double)up), mlo = 0.5 * ((double)aq + (double)dn);
  float r = aq;
  r = ad > mhi * bd ? up : r;  // (the two tests exclude each other)
  r = ad < mlo * bd ? dn : r;
  return simple ? q : copysignf(r, q);
}

}  // namespace bm
