"""The allocation-free entry point (bm_hip_bitlinear_noalloc_dev) against the
existing bm_hip_bitlinear_dev, through the C ABI: bit-identical outputs on
consecutive calls that reuse the library's scratch array (the second call
smaller than the first, so stale workspace from the first call would show),
on every product path (GEMV, few-token MFMA, GEMM, generic K), plus the
refusal of a call larger than the scratch array; and what the entry exists
for: repeated calls leave the device's free memory unchanged, and a call
captured into a HIP graph on a caller's stream replays correctly."""
import ctypes as C

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


def _hip_runtime():
    """The HIP runtime the library itself uses (loaded once per process)."""
    rt = C.CDLL("libamdhip64.so")
    vp = C.c_void_p
    sigs = {
        "hipStreamCreateWithFlags": [C.POINTER(vp), C.c_uint],
        "hipStreamBeginCapture": [vp, C.c_int],
        "hipStreamEndCapture": [vp, C.POINTER(vp)],
        "hipGraphInstantiate": [C.POINTER(vp), vp, vp, C.c_char_p, C.c_size_t],
        "hipGraphLaunch": [vp, vp],
        "hipStreamSynchronize": [vp],
        "hipGraphExecDestroy": [vp],
        "hipGraphDestroy": [vp],
        "hipStreamDestroy": [vp],
        "hipMemGetInfo": [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)],
    }
    for name, args in sigs.items():
        f = getattr(rt, name)
        f.argtypes = args
        f.restype = C.c_int
    return rt


def _ok(rc, what):
    assert rc == 0, "%s: HIP error %d" % (what, rc)


def test_noalloc_no_allocation_and_graph_capture(hip):
    """On a stream of the caller's: (1) after a first call of each shape,
    five more calls leave hipMemGetInfo's free bytes unchanged; (2) the call
    captured between hipStreamBeginCapture and hipStreamEndCapture
    (thread-local mode: an allocation inside would fail the capture),
    instantiated and replayed three times, with eager calls on other inputs
    (which reuse the same scratch) between the replays, gives
    bm_hip_bitlinear_dev's output bit for bit on every replay."""
    rt = _hip_runtime()
    s = C.c_void_p()
    _ok(rt.hipStreamCreateWithFlags(C.byref(s), 1), "hipStreamCreateWithFlags")
    free0, free1, total = C.c_size_t(), C.c_size_t(), C.c_size_t()
    try:
        for M, K, N in ((1, 2048, 8512), (24, 4096, 2048), (64, 1024, 333)):
            note("noalloc capture M=%d K=%d N=%d" % (M, K, N))
            r = np.random.default_rng(M + K + N)
            packed = r.integers(0, 256, (N, K // 4), dtype=np.uint8)
            x = r.standard_normal((M, K)).astype(np.float32)
            x2 = r.standard_normal((M, K)).astype(np.float32)
            g = (1.0 + 0.1 * r.standard_normal(K)).astype(np.float32)
            dx, dx2, dg, dw = (DB.from_array(a) for a in (x, x2, g, packed))
            d_ref, d_na, d_other = DB(4 * M * N), DB(4 * M * N), DB(4 * M * N)
            dq, ds, da = DB(M * K), DB(4 * M), DB(max(hip.bm_hip_act_bytes(M, K), 1))
            bh.check(hip.bm_hip_bitlinear_dev(dx.ptr, M, K, dg.ptr, dw.ptr, N, 0.02, 0,
                                              d_ref.ptr, dq.ptr, K, ds.ptr, da.ptr, None),
                     "bitlinear_dev")
            bh.check(hip.bm_hip_synchronize(), "synchronize")
            ref = d_ref.download((M, N), np.float32)

            def call(src, dst):
                return hip.bm_hip_bitlinear_noalloc_dev(src.ptr, M, K, dg.ptr, dw.ptr, N, 0.02,
                                                        0, dst.ptr, s.value)

            assert call(dx, d_na) == 0
            _ok(rt.hipStreamSynchronize(s), "sync")
            _ok(rt.hipMemGetInfo(C.byref(free0), C.byref(total)), "hipMemGetInfo")
            for _ in range(5):
                assert call(dx, d_na) == 0
            _ok(rt.hipStreamSynchronize(s), "sync")
            _ok(rt.hipMemGetInfo(C.byref(free1), C.byref(total)), "hipMemGetInfo")
            assert free1.value == free0.value, (free0.value, free1.value)
            same_bits(d_na.download((M, N), np.float32), ref, "eager on the caller's stream")

            graph, exe = C.c_void_p(), C.c_void_p()
            _ok(rt.hipStreamBeginCapture(s, 1), "hipStreamBeginCapture")
            rc = call(dx, d_na)
            _ok(rt.hipStreamEndCapture(s, C.byref(graph)), "hipStreamEndCapture")
            assert rc == 0, bh.last_error()
            _ok(rt.hipGraphInstantiate(C.byref(exe), graph, None, None, 0), "instantiate")
            try:
                for rep in range(3):
                    bh.check(hip.bm_hip_memset(d_na.ptr, 0xFF, 4 * M * N), "memset")
                    assert hip.bm_hip_bitlinear_noalloc_dev(dx2.ptr, M, K, dg.ptr, dw.ptr, N,
                                                            0.02, 0, d_other.ptr, None) == 0
                    bh.check(hip.bm_hip_synchronize(), "synchronize")
                    _ok(rt.hipGraphLaunch(exe, s), "hipGraphLaunch")
                    _ok(rt.hipStreamSynchronize(s), "sync")
                    same_bits(d_na.download((M, N), np.float32), ref, "replay %d" % rep)
            finally:
                rt.hipGraphExecDestroy(exe)
                rt.hipGraphDestroy(graph)
            for b in (dx, dx2, dg, dw, d_ref, d_na, d_other, dq, ds, da):
                b.free()
    finally:
        rt.hipStreamDestroy(s)
