// Compares bm::libm::expf_glibc / logf_glibc (the device restatement in
// bitmamba.c_amd/csrc/bm_libm.h, compiled here for the CPU) with the
// installed glibc expf / logf on every float input.  Prints mismatch counts.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "bm_libm.h"

int main() {
  long n_exp = 0, d_exp = 0, n_log = 0, d_log = 0;
#pragma omp parallel for schedule(dynamic, 1) reduction(+ : n_exp, d_exp, n_log, d_log)
  for (int64_t hi = 0; hi < 65536; ++hi) {
    for (uint32_t lo = 0; lo < 65536; ++lo) {
      const uint32_t u = ((uint32_t)hi << 16) | lo;
      float x;
      memcpy(&x, &u, 4);
      if (isnan(x)) continue;
      const float a = expf(x), b = bm::libm::expf_glibc(x);
      ++n_exp;
      if (memcmp(&a, &b, 4) != 0 && !(a == 0 && b == 0)) ++d_exp;
      if (x >= 0.0f) {
        const float c = logf(x), e = bm::libm::logf_glibc(x);
        ++n_log;
        if (memcmp(&c, &e, 4) != 0) ++d_log;
      }
    }
  }
  printf("expf %ld %ld\nlogf %ld %ld\n", n_exp, d_exp, n_log, d_log);
  return 0;
}
