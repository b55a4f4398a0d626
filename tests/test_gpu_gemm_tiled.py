"""GPU parity of the prefill GEMM on tiled weights (two K-groups per block)
against the oracle, through the C ABI.

Bar: int32 totals and fp32 outputs bit-exact.  The fp32 epilogue folds the
1024-column block terms in the scalar kernel's order (src/kernel.c:255-256,
407-425); the K split between the two groups of a block falls inside a
block for K = 256 .. 1792 and 2304 .. 3072 (its two int32 partial totals
are added before the block's term is formed) and on a block boundary for
K = 2048 and 4096, and every one of these cases is covered below.
"""
import numpy as np
import pytest

import native
from native import bh, same_bits

pytestmark = pytest.mark.gpu
DB = bh.DeviceBuffer


def note(msg):
    print("[case] " + msg, flush=True)


def tile_host(packed, N, K):
    """The MFMA tile layout, restated in numpy from its definition: for each
    run of 32 rows and each 128-column stage the rows' 32 packed bytes of the
    stage, row after row; rows past N hold code 01 (weight 0); code 11 -> 10."""
    p = np.asarray(packed, np.uint8)
    rows = (N + 31) // 32 * 32
    full = np.full((rows, K // 4), 0x55, np.uint8)
    full[:N] = p
    # field 11 -> 10: clear the low bit where both bits are set
    full = full - (((full >> 1) & full) & 0x55)
    t = full.reshape(rows // 32, 32, K // 128, 32).transpose(0, 2, 1, 3)
    return np.ascontiguousarray(t).reshape(-1)


def gpu_tile(hip, packed, N, K, canonical=0):
    dw = DB.from_array(packed)
    dt = DB(hip.bm_hip_tiled_bytes(N, K))
    bh.check(hip.bm_hip_tile_weights_dev(dw.ptr, N, K, canonical, dt.ptr, None), "tile")
    return dw, dt


def gpu_gemm_i32_tiled(hip, xq, packed, N, K):
    M = xq.shape[0]
    dw, dt = gpu_tile(hip, packed, N, K)
    dx = DB.from_array(xq)
    do, da = DB(4 * M * N), DB(hip.bm_hip_i8_act_bytes(M, K))
    bh.check(hip.bm_hip_ternary_gemm_i32_tiled_dev(dx.ptr, M, K, dt.ptr, N, K, do.ptr, da.ptr,
                                                   None), "gemm_i32_tiled")
    hip.bm_hip_synchronize()
    return do.download((M, N), np.int32)


def gpu_bitlinear_tiled(hip, x, packed, N, K, scale, g):
    """quantize (bm_hip_quantize_dev) + the tiled GEMM; also returns the
    row-major GEMM's output on the same workspace (the other GPU path)."""
    M = x.shape[0]
    dw, dt = gpu_tile(hip, packed, N, K)
    dx, dg = DB.from_array(x), DB.from_array(g)
    dq, ds = DB(M * K), DB(4 * M)
    da = DB(hip.bm_hip_act_bytes(M, K))
    do = DB(4 * M * N)
    bh.check(hip.bm_hip_quantize_dev(dx.ptr, M, K, K, dg.ptr, None, dq.ptr, K, ds.ptr, da.ptr,
                                     None), "quantize")
    bh.check(hip.bm_hip_bitlinear_tiled_dev(da.ptr, ds.ptr, M, dt.ptr, N, K, scale, do.ptr, None),
             "bitlinear_tiled")
    hip.bm_hip_synchronize()
    return do.download((M, N), np.float32), dq.download((M, K), np.int8)


@pytest.mark.parametrize("N,K", [(32, 128), (100, 256), (8512, 2048), (33, 4096), (2048, 4096)])
def test_tile_layout(hip, N, K):
    note("tile layout N=%d K=%d" % (N, K))
    r = np.random.default_rng(N + K)
    packed = r.integers(0, 256, (N, K // 4), dtype=np.uint8)  # codes 11 included
    _, dt = gpu_tile(hip, packed, N, K)
    got = dt.download(hip.bm_hip_tiled_bytes(N, K), np.uint8)
    np.testing.assert_array_equal(got, tile_host(packed, N, K))


I32_SHAPES = [(1, 256, 100), (63, 512, 384), (65, 1024, 385), (100, 2048, 1000),
              (257, 4096, 256), (130, 8192, 768), (64, 16384, 130), (200, 3072, 500),
              (70, 1280, 300), (128, 2304, 640)]


@pytest.mark.parametrize("M,K,N", I32_SHAPES)
def test_tiled_i32_exact(hip, M, K, N):
    note("tiled i32 M=%d K=%d N=%d" % (M, K, N))
    r = np.random.default_rng(M * 7 + K + N)
    packed = r.integers(0, 256, (N, K // 4), dtype=np.uint8)
    xq = r.integers(-128, 128, (M, K), dtype=np.int8)
    got = gpu_gemm_i32_tiled(hip, xq, packed, N, K)
    np.testing.assert_array_equal(got, native.orc_gemm_i32(xq, packed, N, K))


# every K-split case of the fp32 fold (see the module docstring)
FP_SHAPES = [(64, 256, 384), (70, 512, 100), (33, 1024, 777), (65, 1280, 300),
             (64, 1536, 256), (100, 1792, 130), (128, 2048, 1000), (96, 2304, 384),
             (64, 2560, 256), (64, 2816, 200), (130, 3072, 260), (128, 4096, 512),
             (1, 2048, 8512), (257, 4096, 2048), (200, 2048, 8384)]


@pytest.mark.parametrize("M,K,N", FP_SHAPES)
def test_tiled_fp32_exact(hip, M, K, N):
    note("tiled fp32 M=%d K=%d N=%d" % (M, K, N))
    r = np.random.default_rng(M + 3 * K + N)
    packed = r.integers(0, 256, (N, K // 4), dtype=np.uint8)
    x = r.standard_normal((M, K)).astype(np.float32)
    x[:, r.integers(0, K, 3)] *= 10.0
    g = (r.standard_normal(K) * 0.02).astype(np.float32)
    out, xq = gpu_bitlinear_tiled(hip, x, packed, N, K, 0.02, g)
    ref, _, rq = native.orc_bitlinear(x, packed, N, K, 0.02, g)
    np.testing.assert_array_equal(xq, rq)
    same_bits(out, ref, "out")


def test_prefill_shapes_tiled(hip):
    """The M=2048 prefill products (K=2048 -> N=8512, K=4096 -> N=2048) on
    tiled weights: 40 token rows (first and last tile rows included) against
    the oracle, and every output against the row-major GEMM (the other GPU
    path, itself checked against the oracle by test_gpu_kernels)."""
    r = np.random.default_rng(2048)
    L = hip
    for M, K, N, seed in ((2048, 2048, 8512, 11), (2048, 4096, 2048, 12)):
        note("prefill tiled M=%d K=%d N=%d" % (M, K, N))
        packed = bh.synth_ternary(seed, 1, N, K, bh.SYNTH_UNIFORM)
        x = bh.synth_normal(seed, 2, (M, K), 1.0)
        x[r.random((M, K)) < 0.01] *= 10.0
        g = np.ones(K, np.float32)
        out, xq = gpu_bitlinear_tiled(hip, x, packed, N, K, 0.02, g)
        rows = np.unique(np.concatenate([[0, 1, 63, 64, 127, 128, M - 1], r.integers(0, M, 33)]))
        ref, _, rq = native.orc_bitlinear(x[rows], packed, N, K, 0.02, g)
        np.testing.assert_array_equal(xq[rows], rq)
        same_bits(out[rows], ref, "out[rows]")
        # every output against the row-major GEMM
        dx, dg, dw = DB.from_array(x), DB.from_array(g), DB.from_array(packed)
        do, dq, ds = DB(4 * M * N), DB(M * K), DB(4 * M)
        da = DB(L.bm_hip_act_bytes(M, K))
        bh.check(L.bm_hip_bitlinear_dev(dx.ptr, M, K, dg.ptr, dw.ptr, N, 0.02, 1, do.ptr, dq.ptr,
                                        K, ds.ptr, da.ptr, None), "bitlinear_dev")
        L.bm_hip_synchronize()
        same_bits(out, do.download((M, N), np.float32), "tiled vs row-major GEMM")


def test_stress_m4096_tiled(hip):
    """K = N = 8192, p(0) = 0.6, M = 4096 on tiled weights: 64 x 64 sampled
    entries exactly against the closed form, one full row against the
    oracle, and linearity in the activations."""
    K = N = 8192
    M = 4096
    note("stress tiled M=4096")
    packed = bh.synth_ternary(5, 1, N, K, bh.SYNTH_P0_60)
    xq = bh.synth_int8(5, 3, (M, K))
    got = gpu_gemm_i32_tiled(hip, xq, packed, N, K)
    r = np.random.default_rng(19)
    ms, ns = r.integers(0, M, 64), r.integers(0, N, 64)
    w = native.decode_dense(packed[ns], K).astype(np.int64)
    np.testing.assert_array_equal(got[np.ix_(ms, ns)], xq[ms].astype(np.int64) @ w.T)
    np.testing.assert_array_equal(got[M - 1], native.orc_gemm_i32(xq[M - 1:], packed, N, K)[0])
    a = (xq[:256] // 2).astype(np.int8)
    b = (xq[:256] - a).astype(np.int8)
    np.testing.assert_array_equal(gpu_gemm_i32_tiled(hip, a, packed, N, K) +
                                  gpu_gemm_i32_tiled(hip, b, packed, N, K), got[:256])


def test_tiled_rejects_uncovered_k(hip):
    """K outside the kernel's cover (K % 256 != 0; fp32 with K > 4096 or
    K = 3328..3840) is refused with -2 before anything is launched (the
    buffers are real and large enough all the same)."""
    M = N = 64
    for K, mode in ((384, "fp32"), (8192, "fp32"), (3584, "fp32"), (384, "i32")):
        note("tiled reject K=%d %s" % (K, mode))
        da, ds = DB(hip.bm_hip_act_bytes(M, K)), DB(4 * M)
        dt, do, dx = DB(N * K), DB(4 * M * N), DB(M * K)
        if mode == "fp32":
            rc = hip.bm_hip_bitlinear_tiled_dev(da.ptr, ds.ptr, M, dt.ptr, N, K, 1.0, do.ptr,
                                                None)
        else:
            rc = hip.bm_hip_ternary_gemm_i32_tiled_dev(dx.ptr, M, K, dt.ptr, N, K, do.ptr,
                                                       da.ptr, None)
        assert rc == -2, (K, mode, rc)
