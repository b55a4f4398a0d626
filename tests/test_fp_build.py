"""The library's correctly rounded fp32 division and square root
(csrc/bm_fp.h) are written out on the gfx950 instructions, so they must not
depend on the compiler's fp32 division/sqrt option: built with that option
off, they compile to the same instructions as `a / b` and `sqrtf(x)` built
with -fhip-fp32-correctly-rounded-divide-sqrt (the compiler's IEEE
sequences).  Their numerics are checked on the device against the host's
IEEE arithmetic in test_gpu_model.test_device_division_sqrt_and_silu."""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "bitmamba.c_amd", "csrc")
HIPCC = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")

SRC = r'''
#include "bm_fp.h"
__global__ void k_div(const float* a, const float* b, float* o) {
  const int i = threadIdx.x;
  o[i] = DIV(a[i], b[i]);
}
__global__ void k_sqrt(const float* a, float* o) {
  const int i = threadIdx.x;
  o[i] = SQRT(a[i]);
}
'''


def _isa(defs, flag, d):
    src = os.path.join(d, "k.hip")
    with open(src, "w") as f:
        f.write(SRC)
    out = os.path.join(d, "k_%d.s" % abs(hash((defs, flag))))
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-ffp-contract=off", flag, "--cuda-device-only",
           "-S", "-I", CSRC, "-o", out, src] + ["-D%s" % x for x in defs]
    subprocess.run(cmd, check=True, stdout=subprocess.PIPE, stderr=subprocess.PIPE)
    text = open(out).read()
    kernels = {}
    for name in ("k_div", "k_sqrt"):
        m = re.search(r"^(_Z\d+%sP\S*):.*?\n(.*?)s_endpgm" % name, text, re.S | re.M)
        assert m, name
        body = [l.strip() for l in m.group(2).splitlines()
                if l.strip() and not l.strip().startswith((";", "."))]
        kernels[name] = body
    return kernels


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
def test_cr_div_sqrt_match_compiler_ieee_sequences():
    d = tempfile.mkdtemp()
    try:
        ours = _isa(("DIV=bm::cr_divf", "SQRT=bm::cr_sqrtf"),
                    "-fno-hip-fp32-correctly-rounded-divide-sqrt", d)
        ieee = _isa(("DIV(a,b)=((a)/(b))", "SQRT=sqrtf"),
                    "-fhip-fp32-correctly-rounded-divide-sqrt", d)
        fast = _isa(("DIV(a,b)=((a)/(b))", "SQRT=sqrtf"),
                    "-fno-hip-fp32-correctly-rounded-divide-sqrt", d)
    finally:
        shutil.rmtree(d, ignore_errors=True)
    assert ours == ieee
    # the comparison means something: without the option the compiler's own
    # division and sqrt are other (approximate) sequences
    assert fast != ieee
