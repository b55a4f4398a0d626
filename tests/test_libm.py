"""The device's expf/logf (bitmamba.c_amd/csrc/bm_libm.h) equal the host
glibc's on every float input.  The same header is compiled here with g++;
the GPU test test_gpu_model.py::test_device_libm checks the device build of
it on a dense sample against the same glibc."""
import os
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _has_fma():
    try:
        return " fma " in open("/proc/cpuinfo").read().replace("\n", " ")
    except OSError:
        return False


@pytest.mark.skipif(not _has_fma(), reason="glibc takes its non-FMA expf/logf path on this CPU")
def test_libm_restatement_exhaustive():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "libm_check")
        subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", "-std=c++17",
                        "-I" + os.path.join(ROOT, "bitmamba.c_amd", "csrc"),
                        os.path.join(ROOT, "tests", "csrc", "libm_exhaustive.cpp"),
                        "-o", exe, "-lm"], check=True)
        out = subprocess.run([exe], check=True, stdout=subprocess.PIPE, text=True,
                             timeout=600).stdout.split()
    n_exp, d_exp, n_log, d_log = int(out[1]), int(out[2]), int(out[4]), int(out[5])
    assert n_exp > 4_000_000_000 and n_log > 2_000_000_000
    assert d_exp == 0, "%d expf mismatches" % d_exp
    assert d_log == 0, "%d logf mismatches" % d_log
