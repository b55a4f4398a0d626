// Correctly rounded fp32 arithmetic helpers for device code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bm {

// Correctly rounded fp32 division and square root, written out on the
// gfx950 instructions so that the results do not depend on the compiler's
// fp32 division/sqrt options.  fp32 denormals are kept (the default mode).

// a / b: the IEEE sequence of the ISA -- both operands scaled into range
// (v_div_scale), the reciprocal refined by fma steps, the quotient refined
// twice, v_div_fmas undoing the scaling and v_div_fixup handling zeros,
// infinities, NaNs and overflow.
__device__ __forceinline__ float cr_divf(float a, float b) {
  bool den_flag, num_flag;
  const float den = __builtin_amdgcn_div_scalef(a, b, false, &den_flag);
  const float num = __builtin_amdgcn_div_scalef(a, b, true, &num_flag);
  (void)den_flag;
  const float r0 = __builtin_amdgcn_rcpf(den);
  const float e0 = __builtin_fmaf(-den, r0, 1.0f);
  const float r1 = __builtin_fmaf(e0, r0, r0);
  const float q0 = num * r1;
  const float e1 = __builtin_fmaf(-den, q0, num);
  const float q1 = __builtin_fmaf(e1, r1, q0);
  const float e2 = __builtin_fmaf(-den, q1, num);
  const float f = __builtin_amdgcn_div_fmasf(e2, r1, q1, num_flag);
  return __builtin_amdgcn_div_fixupf(f, b, a);
}

// sqrt(x): v_sqrt_f32 (inputs below 2^-96 scaled by 2^32 first), then the
// exact residual test of its two neighbours picks the correctly rounded
// one; zeros and +inf pass through, negative inputs and NaN give NaN.
__device__ __forceinline__ float cr_sqrtf(float x) {
  const bool tiny = x < 0x1p-96f;
  const float xs = tiny ? x * 0x1p32f : x;
  float s = __builtin_amdgcn_sqrtf(xs);
  const float s_dn = __int_as_float(__float_as_int(s) - 1);
  const float s_up = __int_as_float(__float_as_int(s) + 1);
  const float r_dn = __builtin_fmaf(-s_dn, s, xs);
  const float r_up = __builtin_fmaf(-s_up, s, xs);
  s = 0.0f >= r_dn ? s_dn : s;
  s = 0.0f < r_up ? s_up : s;
  s = tiny ? s * 0x1p-16f : s;
  // class mask 0x260: -0, +0, +inf
  return __builtin_amdgcn_classf(xs, 0x260) ? xs : s;
}

}  // namespace bm
