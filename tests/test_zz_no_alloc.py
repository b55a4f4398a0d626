"""The allocation-free entry point (bm_hip_bitlinear_noalloc_dev) against the
existing bm_hip_bitlinear_dev, through the C ABI: bit-identical outputs on
consecutive calls that reuse the library's scratch array (the second call
smaller than the first, so stale workspace from the first call would show),
on every product path (GEMV, few-token MFMA, GEMM, generic K), plus the
refusal of a call larger than the scratch array."""
import numpy as np
import pytest

import native
from native import bh, same_bits

pytestmark = pytest.mark.gpu
DB = bh.DeviceBuffer


def note(msg):
    print("[case] " + msg, flush=True)


def both(hip, M, K, N, seed):
    """Output of bm_hip_bitlinear_dev and of the no-alloc entry on the same
    inputs (host arrays), and the inputs."""
    r = np.random.default_rng(seed)
    packed = r.integers(0, 256, (N, (K + 3) // 4), dtype=np.uint8)
    x = r.standard_normal((M, K)).astype(np.float32)
    x[:, r.integers(0, K, 3)] *= 10.0
    g = (r.standard_normal(K) * 0.02).astype(np.float32)
    dx, dg, dw = DB.from_array(x), DB.from_array(g), DB.from_array(packed)
    d_ref, d_na = DB(4 * M * N), DB(4 * M * N)
    dq, ds, da = DB(M * K), DB(4 * M), DB(max(hip.bm_hip_act_bytes(M, K), 1))
    bh.check(hip.bm_hip_bitlinear_dev(dx.ptr, M, K, dg.ptr, dw.ptr, N, 0.02, 0, d_ref.ptr,
                                      dq.ptr, K, ds.ptr, da.ptr, None), "bitlinear_dev")
    bh.check(hip.bm_hip_bitlinear_noalloc_dev(dx.ptr, M, K, dg.ptr, dw.ptr, N, 0.02, 0,
                                              d_na.ptr, None), "bitlinear_noalloc_dev")
    bh.check(hip.bm_hip_synchronize(), "synchronize")
    return (d_ref.download((M, N), np.float32), d_na.download((M, N), np.float32),
            (x, packed, g))


# (first call, second smaller call) per product path
PAIRS = [((1, 2048, 8512), (1, 1024, 300)),      # decode GEMV
         ((24, 4096, 2048), (5, 2048, 100)),      # few-token MFMA
         ((300, 2048, 1000), (64, 1024, 333)),    # GEMM
         ((7, 1000, 77), (2, 100, 10))]           # K % 64 != 0: generic kernel


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_bitlinear_dev(hip, first, second):
    for i, (M, K, N) in enumerate((first, second)):
        note("noalloc M=%d K=%d N=%d" % (M, K, N))
        ref, got, _ = both(hip, M, K, N, 100 * i + M + K + N)
        same_bits(got, ref, "noalloc vs bitlinear_dev")


def test_noalloc_matches_oracle(hip):
    M, K, N = 3, 2048, 520
    note("noalloc vs oracle M=%d K=%d N=%d" % (M, K, N))
    ref, got, (x, packed, g) = both(hip, M, K, N, 7)
    oracle, _, _ = native.orc_bitlinear(x, packed, N, K, 0.02, g)
    same_bits(got, oracle, "noalloc vs oracle")


def test_noalloc_refuses_more_than_its_scratch(hip):
    """M = 2048 tokens of K = 4096 need ~17 MB of workspace, more than the
    8 MiB array: refused with -2 before anything is launched (the buffers
    are real and large enough all the same)."""
    limit = hip.bm_hip_noalloc_scratch_bytes()
    assert limit == 8 << 20
    M, K, N = 2048, 4096, 64
    assert M * hip.bm_hip_act_bytes(1, K) > limit
    dx, dg = DB(4 * M * K), DB(4 * K)
    dw, do = DB(N * K // 4), DB(4 * M * N)
    rc = hip.bm_hip_bitlinear_noalloc_dev(dx.ptr, M, K, dg.ptr, dw.ptr, N, 0.02, 1, do.ptr, None)
    assert rc == -2, rc
    assert "scratch" in bh.last_error()
