// expf / logf with the exact results of the reference's libm.
//
// The reference computes the SSM step with glibc's expf and logf
// (src/kernel.c:50-68, src/bitmamba.h:234-243; glibc 2.35 on the x86-64
// hosts used here).  glibc implements both with the published algorithms of
// Arm's optimized-routines (e_expf.c / e_logf.c, 2017-2018): a 2^(k/32)
// table plus a cubic in fp64 for expf, a 16-entry (1/c, log c) table plus a
// cubic in fp64 for logf.  On x86-64 CPUs with FMA, glibc dispatches to a
// build of the same C code in which the compiler fuses every a*b+c; the
// restatement below uses fma() at exactly those places.  It reproduces the
// installed glibc for every float input (checked exhaustively on the CPU by
// tests/test_libm.py), including glibc's rare misroundings, which a
// correctly rounded exp/log would not.
//
// Compiles as HIP device/host code and as plain C++ (the test build).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define BM_HD __host__ __device__ __forceinline__
#else
#include <cmath>
#define BM_HD inline
#endif

namespace bm {
namespace libm {

BM_HD uint64_t u64_of(double d) { uint64_t u; __builtin_memcpy(&u, &d, 8); return u; }
BM_HD double dbl_of(uint64_t u) { double d; __builtin_memcpy(&d, &u, 8); return d; }
BM_HD uint32_t u32_of(float f) { uint32_t u; __builtin_memcpy(&u, &f, 4); return u; }
BM_HD float flt_of(uint32_t u) { float f; __builtin_memcpy(&f, &u, 4); return f; }

// 2^(i/32) rounded to fp64, stored minus i << 47 so that adding the
// integer exponent bits of k/32 yields 2^(k/32) directly.
inline constexpr uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,
    0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,
    0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,
    0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,
    0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,
    0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,
    0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,
    0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,
    0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

BM_HD float expf_glibc(float x) {
  // special cases (selected at the end, no branches): overflow above
  // ~88.72, underflow to 0 below ~-103.97, NaN passes through
  const bool nan = x != x;
  const bool ovf = x > 0x1.62e42ep6f;
  const bool unf = x < -0x1.9fe368p6f;
  const double InvLn2N = 0x1.71547652b82fep+0 * 32;
  const double Shift = 0x1.8p+52;
  const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double C2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double xd = (double)((nan || ovf || unf) ? 0.0f : x);
  // x*32/ln2 = k + r, |r| <= 1/2
  double kd = __builtin_fma(InvLn2N, xd, Shift);
  const uint64_t ki = u64_of(kd);
  kd -= Shift;
  const double r = __builtin_fma(InvLn2N, xd, -kd);
  uint64_t t = kExp2Tab[ki % 32];
  t += ki << (52 - 5);
  const double s = dbl_of(t);
  const double z = __builtin_fma(C0, r, C1);
  const double r2 = r * r;
  double y = __builtin_fma(C2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  float res = (float)y;
  res = unf ? 0.0f : res;
  res = ovf ? __builtin_inff() : res;
  return nan ? x : res;
}

// (1/c, log c) for the 16 subintervals of [0x3f330000, 2 * 0x3f330000)
inline constexpr double kLogInvC[16] = {
    0x1.661ec79f8f3bep+0, 0x1.571ed4aaf883dp+0, 0x1.49539f0f010bp+0, 0x1.3c995b0b80385p+0,
    0x1.30d190c8864a5p+0, 0x1.25e227b0b8eap+0, 0x1.1bb4a4a1a343fp+0, 0x1.12358f08ae5bap+0,
    0x1.0953f419900a7p+0, 0x1p+0, 0x1.e608cfd9a47acp-1, 0x1.ca4b31f026aap-1,
    0x1.b2036576afce6p-1, 0x1.9c2d163a1aa2dp-1, 0x1.886e6037841edp-1, 0x1.767dcf5534862p-1,
};
inline constexpr double kLogC[16] = {
    -0x1.57bf7808caadep-2, -0x1.2bef0a7c06ddbp-2, -0x1.01eae7f513a67p-2, -0x1.b31d8a68224e9p-3,
    -0x1.6574f0ac07758p-3, -0x1.1aa2bc79c81p-3, -0x1.a4e76ce8c0e5ep-4, -0x1.1973c5a611cccp-4,
    -0x1.252f438e10c1ep-5, 0x0p+0, 0x1.aa5aa5df25984p-5, 0x1.c5e53aa362eb4p-4,
    0x1.526e57720db08p-3, 0x1.bc2860d22477p-3, 0x1.1058bc8a07ee1p-2, 0x1.4043057b6ee09p-2,
};

BM_HD float logf_glibc(float x) {
  // special inputs are handled by selects after the main path: 1 -> 0,
  // +-0 -> -inf, +inf -> +inf, negative or NaN -> NaN; subnormals are
  // normalized first
  const uint32_t ix0 = u32_of(x);
  const bool special = ix0 - 0x00800000u >= 0x7f800000u - 0x00800000u;
  const bool sub = special && ix0 > 0u && ix0 < 0x00800000u;
  const uint32_t ix = sub ? u32_of(x * 0x1p23f) - (23u << 23) : ix0;
  const double Ln2 = 0x1.62e42fefa39efp-1;
  const double A0 = -0x1.00ea348b88334p-2, A1 = 0x1.5575b0be00b6ap-2,
               A2 = -0x1.ffffef20a4123p-2;
  // x = 2^k z, z in [0x3f330000, 2*0x3f330000) split in 16 subintervals
  const uint32_t tmp = ix - 0x3f330000u;
  const int i = (int)((tmp >> (23 - 4)) % 16);
  const int k = (int32_t)tmp >> 23;
  const uint32_t iz = ix - (tmp & (0x1ffu << 23));
  const double invc = kLogInvC[i], logc = kLogC[i];
  const double z = (double)flt_of(iz);
  // log(x) = log1p(z/c - 1) + log(c) + k*Ln2
  const double r = __builtin_fma(z, invc, -1.0);
  const double y0 = __builtin_fma((double)k, Ln2, logc);
  const double r2 = r * r;
  double y = __builtin_fma(A1, r, A2);
  y = __builtin_fma(A0, r2, y);
  y = __builtin_fma(y, r2, y0 + r);
  float res = (float)y;
  if (special && !sub) {
    res = ix0 * 2 == 0 ? -__builtin_inff()
          : ix0 == 0x7f800000u ? x
                               : __builtin_nanf("");
  }
  return ix0 == 0x3f800000u ? 0.0f : res;
}

}  // namespace libm
}  // namespace bm
