"""GPU parity of the gfx950 kernels against the oracle and the golden
fixtures, through the C ABI.

Bar: int8, int32 and fp32 outputs bit-exact (the fp32 epilogue follows the
scalar kernel's 1024-column block order, so no tolerance is needed; the
stated 1e-4 relative tolerance is asserted as a second, looser line in the
fp32 tests so a failure shows how far off it is).
"""
import ctypes as C
import os

import numpy as np
import pytest

import native
from native import bh, ptr, same_bits

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DB = bh.DeviceBuffer


def rnd(seed):
    return np.random.default_rng(seed)


def note(msg):
    print("[case] " + msg, flush=True)


def rel_err(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


# ------------------------------------------------------------ helpers
def gpu_quantize(hip, x, g, act=True):
    M, n = x.shape
    dx, dg = DB.from_array(x), DB.from_array(g)
    dn, dq, ds = DB(x.nbytes), DB(M * n), DB(4 * M)
    da = DB(bh.lib().bm_hip_act_bytes(M, n)) if act else None
    bh.check(hip.bm_hip_quantize_dev(dx.ptr, M, n, n, dg.ptr, dn.ptr, dq.ptr, n, ds.ptr,
                                     da.ptr if da else None, None), "quantize")
    hip.bm_hip_synchronize()
    return (dn.download((M, n), np.float32), dq.download((M, n), np.int8),
            ds.download(M, np.float32))


def gpu_bitlinear(hip, x, packed, N, K, scale, g, canonical=0):
    M = x.shape[0]
    dx, dg, dw = DB.from_array(x), DB.from_array(g), DB.from_array(packed)
    do, dq, ds = DB(4 * M * N), DB(M * K), DB(4 * M)
    da = DB(hip.bm_hip_act_bytes(M, K))
    bh.check(hip.bm_hip_bitlinear_dev(dx.ptr, M, K, dg.ptr, dw.ptr, N, scale, canonical, do.ptr,
                                      dq.ptr, K, ds.ptr, da.ptr, None), "bitlinear_dev")
    hip.bm_hip_synchronize()
    return do.download((M, N), np.float32), dq.download((M, K), np.int8)


def gpu_gemm_i32(hip, xq, packed, N, K, canonical=0):
    M = xq.shape[0]
    dx, dw = DB.from_array(xq), DB.from_array(packed)
    do, da = DB(4 * M * N), DB(hip.bm_hip_i8_act_bytes(M, K))
    bh.check(hip.bm_hip_ternary_gemm_i32_dev(dx.ptr, M, K, dw.ptr, N, K, canonical, do.ptr,
                                             da.ptr, None), "gemm_i32")
    hip.bm_hip_synchronize()
    return do.download((M, N), np.int32)


# ------------------------------------------------------------ quantizer
def test_quantize_golden(hip):
    z = np.load(os.path.join(GOLD, "quant_vectors.npz"))
    for n in (1024, 4096, 4099, 100):
        note("quantize golden n=%d" % n)
        x, g = z["x_%d" % n], z["g_%d" % n]
        xn, xq, _ = gpu_quantize(hip, x, g, act=(n % 16 == 0))
        same_bits(xn, z["xn_%d" % n], "xn")
        np.testing.assert_array_equal(xq, z["xq_%d" % n])


@pytest.mark.parametrize("n", [1024, 2048, 4096, 8192, 1040])
def test_quantize_random_vs_oracle(hip, n):
    note("quantize random n=%d" % n)
    r = rnd(n)
    M = 96
    scales = 10.0 ** r.uniform(-4, 4, (M, 1))
    x = (r.standard_normal((M, n)) * scales).astype(np.float32)
    x[::7, r.integers(0, n, 5)] *= 100.0
    g = (r.standard_normal(n) * 0.02).astype(np.float32)
    xn, xq, sc = gpu_quantize(hip, x, g)
    on, oq, osc, _ = native.orc_quantize_rows(x, g)
    same_bits(xn, on, "xn")
    np.testing.assert_array_equal(xq, oq)
    same_bits(sc, osc, "sc")


def _chain_rows(n, seed):
    """Rows whose sums of squares stress an exact sequential fp32 sum: ties
    of the running sum's rounding (1 and 4096 mixed: x^2 = 1 is half an ulp
    once the sum passes 2^24), powers of two, denormal squares, zeros, an
    overflow to inf, and outliers in normal data."""
    r = rnd(seed)
    rows = [
        np.where(r.random(n) < 0.02, 4096.0, 1.0),
        np.ldexp(1.0, r.integers(-20, 20, n)) * r.choice([-1.0, 1.0], n),
        r.integers(-3, 4, n).astype(np.float64),
        r.standard_normal(n) * 1e-23,
        np.zeros(n),
        np.where(np.arange(n) == n // 3, 3.0, 0.0),
        np.where(np.arange(n) == n // 2, 1e20, r.standard_normal(n)),
        r.standard_normal(n) * np.where(r.random(n) < 0.01, 1e4, 1.0),
        np.where(r.random(n) < 0.5, 2048.0, r.integers(1, 64, n).astype(np.float64)),
    ]
    return np.ascontiguousarray(np.stack(rows).astype(np.float32))


@pytest.mark.parametrize("n", [1024, 2048, 4096, 8192, 1040, 300])
def test_quantize_chain_edge_rows(hip, n):
    """The generic per-token quantizer (a row stride that is not a multiple
    of 4 selects it at every n) on rows built to break an inexact sum of
    squares, bit-exact against the oracle."""
    note("quantize chain edge rows n=%d" % n)
    x = _chain_rows(n, 40 + n)
    M = x.shape[0]
    g = (rnd(n).standard_normal(n) * 0.02).astype(np.float32)
    xs = np.zeros((M, n + 1), np.float32)
    xs[:, :n] = x
    dx, dg = DB.from_array(xs), DB.from_array(g)
    dn, dq, ds = DB(4 * M * n), DB(M * n), DB(4 * M)
    bh.check(hip.bm_hip_quantize_dev(dx.ptr, M, n, n + 1, dg.ptr, dn.ptr, dq.ptr, n, ds.ptr,
                                     None, None), "quantize")
    hip.bm_hip_synchronize()
    on, oq, osc, _ = native.orc_quantize_rows(x, g)
    same_bits(dn.download((M, n), np.float32), on, "xn")
    np.testing.assert_array_equal(dq.download((M, n), np.int8), oq)
    same_bits(ds.download(M, np.float32), osc, "sc")
    for i in range(M):
        out = np.empty(n, np.float32)
        hip.hip_rms_norm(ptr(x[i]), n, ptr(g), ptr(out))
        ref = np.empty(n, np.float32)
        native.oracle().orc_rms_norm(ptr(np.ascontiguousarray(x[i])), n, ptr(g), ptr(ref))
        same_bits(out, ref, "rms_norm row %d" % i)


def test_rms_norm_dropin(hip):
    r = rnd(3)
    for n in (1024, 2048, 777):
        note("hip_rms_norm n=%d" % n)
        x = r.standard_normal(n).astype(np.float32)
        g = r.standard_normal(n).astype(np.float32)
        out = np.empty(n, np.float32)
        mx = hip.hip_rms_norm(ptr(x), n, ptr(g), ptr(out))
        ref = np.empty(n, np.float32)
        rmx = native.oracle().orc_rms_norm(ptr(x), n, ptr(g), ptr(ref))
        same_bits(out, ref, "out")
        assert np.float32(mx) == np.float32(rmx)


# ------------------------------------------------------------ int32 products
GEMV_SHAPES = [(1024, 4384), (2048, 8512), (4096, 2048), (8192, 1000), (1024, 50257),
               (512, 100), (1536, 77), (2560, 33), (16384, 40)]


@pytest.mark.parametrize("K,N", GEMV_SHAPES)
@pytest.mark.parametrize("canonical", [0, 1])
def test_gemv_i32_exact(hip, K, N, canonical):
    note("gemv i32 K=%d N=%d canonical=%d" % (K, N, canonical))
    r = rnd(K + N + canonical)
    if canonical:
        packed = bh.synth_ternary(K, N, N, K, bh.SYNTH_UNIFORM)
    else:
        packed = r.integers(0, 256, (N, K // 4), dtype=np.uint8)
    xq = r.integers(-128, 128, (1, K), dtype=np.int8)
    got = gpu_gemm_i32(hip, xq, packed, N, K, canonical)
    np.testing.assert_array_equal(got, native.orc_gemm_i32(xq, packed, N, K))


@pytest.mark.parametrize("M,K,N", [(32, 1024, 128), (100, 2048, 200), (256, 1024, 333),
                                   (64, 4096, 64), (40, 8192, 129), (16, 8192, 512),
                                   (3, 1024, 50), (300, 1152, 260), (700, 2048, 1100),
                                   (1100, 1024, 700), (48, 16384, 96), (2, 2048, 77),
                                   (31, 4096, 300), (5, 8192, 33), (97, 4096, 200),
                                   (256, 2048, 64),
                                   # few tokens with a short last 1024-column slice
                                   # (1, 3 and 1 blocks of 128 columns)
                                   (7, 1152, 100), (20, 1408, 70), (9, 3200, 40),
                                   # up to 16 tokens on 8 MB of weights and more
                                   # (nontemporal weight loads)
                                   (11, 4096, 8192), (6, 2048, 16384),
                                   # GEMM tiles 32x128 (700x2048x1100, 1100x1024x700), 64x128
                                   # (300x1152x260 and 2100x128x2048 in 128-deep stages,
                                   # 1233x256x8512 and 1920x256x8512 in 256-deep ones);
                                   # 128x256 tiles (K >= 8192 or four per CU) run in the
                                   # M=4096 stress tests and test_gemm_128x256_ragged
                                   (1233, 256, 8512), (2100, 128, 2048), (1920, 256, 8512),
                                   # GEMM stage counts: 3 and 5 stages of 128 (the ring's
                                   # prologue and tail waits), 64 stages of 256
                                   (320, 384, 300), (513, 640, 1000), (600, 16384, 130),
                                   # 32x128 tiles (64x128 would leave CUs idle), ragged
                                   # last row and column tiles
                                   (520, 256, 3000),
                                   # 64x256 tiles (two 64x128 tiles per CU), ragged
                                   (1100, 256, 3000)])
def test_gemm_i32_exact(hip, M, K, N):
    note("gemm i32 M=%d K=%d N=%d" % (M, K, N))
    r = rnd(M * 3 + K + N)
    packed = r.integers(0, 256, (N, K // 4), dtype=np.uint8)
    xq = r.integers(-128, 128, (M, K), dtype=np.int8)
    got = gpu_gemm_i32(hip, xq, packed, N, K)
    np.testing.assert_array_equal(got, native.orc_gemm_i32(xq, packed, N, K))


@pytest.mark.parametrize("M,K,N,off,ldx", [(1, 1024, 300, 1, 1024), (1, 8192, 70, 3, 8192),
                                            (5, 2048, 200, 0, 2056), (16, 1024, 100, 8, 1032),
                                            (12, 1152, 90, 0, 1160)])
def test_gemm_i32_unaligned_rows(hip, M, K, N, off, ldx):
    """int8 rows that do not start on 16 bytes (a byte offset, or a row
    stride that is not a multiple of 16): the one-token GEMV reads them byte
    by byte, the few-token product falls back to the preparation launch;
    int32 totals exact against the oracle (src/kernel.c:159-316)."""
    note("gemm i32 unaligned M=%d K=%d N=%d off=%d ldx=%d" % (M, K, N, off, ldx))
    r = rnd(M * 7 + K + N + off)
    packed = r.integers(0, 256, (N, K // 4), dtype=np.uint8)
    xq = r.integers(-128, 128, (M, K), dtype=np.int8)
    buf = np.zeros(off + M * ldx + 16, np.int8)
    for m in range(M):
        buf[off + m * ldx: off + m * ldx + K] = xq[m]
    dx, dw = DB.from_array(buf), DB.from_array(packed)
    do, da = DB(4 * M * N), DB(hip.bm_hip_i8_act_bytes(M, K))
    bh.check(hip.bm_hip_ternary_gemm_i32_dev(dx.ptr + off, M, ldx, dw.ptr, N, K, 0, do.ptr,
                                             da.ptr, None), "gemm_i32")
    hip.bm_hip_synchronize()
    got = do.download((M, N), np.int32)
    np.testing.assert_array_equal(got, native.orc_gemm_i32(xq, packed, N, K))


@pytest.mark.parametrize("M", [1, 16])
def test_stress_exact_small_m(hip, M):
    """Stress shape K = N = 8192, p(0)=0.6, int8 activations, full check."""
    K = N = 8192
    note("stress M=%d" % M)
    packed = bh.synth_ternary(5, 1, N, K, bh.SYNTH_P0_60)
    xq = bh.synth_int8(5, 2, (M, K))
    got = gpu_gemm_i32(hip, xq, packed, N, K, canonical=1)
    np.testing.assert_array_equal(got, native.orc_gemm_i32(xq, packed, N, K))


def test_stress_m4096_sampled_and_linear(hip):
    """M=4096 at full size: 4096 sampled entries checked exactly, plus
    linearity in the activations (size-independent)."""
    K = N = 8192
    M = 4096
    note("stress M=4096")
    packed = bh.synth_ternary(5, 1, N, K, bh.SYNTH_P0_60)
    xq = bh.synth_int8(5, 3, (M, K))
    got = gpu_gemm_i32(hip, xq, packed, N, K, canonical=1)
    r = rnd(9)
    ms = r.integers(0, M, 64)
    ns = r.integers(0, N, 64)
    w = native.decode_dense(packed[ns], K).astype(np.int64)
    expect = xq[ms].astype(np.int64) @ w.T
    np.testing.assert_array_equal(got[np.ix_(ms, ns)], expect)
    # every row of the last tile and a full column
    np.testing.assert_array_equal(got[M - 1], native.orc_gemm_i32(xq[M - 1:], packed, N, K)[0])
    # linearity: (a + b) with |a|,|b| <= 63 stays in int8
    a = (xq[:256] // 2).astype(np.int8)
    b = (xq[:256] - a).astype(np.int8)
    ga = gpu_gemm_i32(hip, a, packed, N, K, 1)
    gb = gpu_gemm_i32(hip, b, packed, N, K, 1)
    np.testing.assert_array_equal(ga + gb, got[:256])


def test_gemm_128x256_ragged(hip):
    """128x256 tiles (K = 8192) with ragged last row and column tiles
    (M = N = 2100): every total of the last row tile and of the last column
    tile exact, plus sampled entries."""
    M, K, N = 2100, 8192, 2100
    note("gemm 128x256 ragged M=%d K=%d N=%d" % (M, K, N))
    packed = bh.synth_ternary(11, 1, N, K, bh.SYNTH_P0_60)
    xq = bh.synth_int8(11, 3, (M, K))
    got = gpu_gemm_i32(hip, xq, packed, N, K, canonical=1)
    w = native.decode_dense(packed, K).astype(np.int64)
    np.testing.assert_array_equal(got[2048:], xq[2048:].astype(np.int64) @ w.T)
    np.testing.assert_array_equal(got[:, 2048:], xq.astype(np.int64) @ w[2048:].T)
    r = rnd(12)
    ms = r.integers(0, M, 64)
    ns = r.integers(0, N, 64)
    np.testing.assert_array_equal(got[np.ix_(ms, ns)], xq[ms].astype(np.int64) @ w[ns].T)


def test_stress_m4096_full_exact(hip):
    """M=4096 at full size, every one of the 4096 x 8192 int32 totals against
    the brute-force product Σ x·decode(W) (float32 BLAS is exact here: every
    partial sum is an integer below 127 · 8192 < 2^24)."""
    K = N = 8192
    M = 4096
    note("stress M=4096 full")
    packed = bh.synth_ternary(5, 1, N, K, bh.SYNTH_P0_60)
    xq = bh.synth_int8(5, 3, (M, K))
    got = gpu_gemm_i32(hip, xq, packed, N, K, canonical=1)
    w = native.decode_dense(packed, K).astype(np.float32)
    expect = xq.astype(np.float32) @ w.T
    np.testing.assert_array_equal(got, expect.astype(np.int32))


def _epilogue_ref(xq, sc, packed, N, K, w_scale):
    """The fp32 outputs of src/kernel.c:388-428 from exact slice totals:
    out = 0; out += (float)total_s * inv per 1024-column slice in order,
    inv = 1/(scale_x * w_scale); totals by float32 BLAS (exact: below 2^24)."""
    f = np.float32
    w = native.decode_dense(packed, K).astype(f)
    x = xq.astype(f)
    inv = f(1.0) / (sc.astype(f) * f(w_scale))
    out = np.zeros((x.shape[0], N), f)
    for s0 in range(0, K, 1024):
        t = x[:, s0:s0 + 1024] @ w[:, s0:s0 + 1024].T
        out = (out + (t.astype(f) * inv[:, None]).astype(f)).astype(f)
    return out


def test_prefill_full_exact(hip):
    """The two M=2048 prefill products at full size: every int8 activation
    against the oracle's quantizer and every fp32 output against the
    reference's slice epilogue on brute-force totals."""
    r = rnd(4096)
    for M, K, N, seed in ((2048, 2048, 8512, 11), (2048, 4096, 2048, 12)):
        note("prefill full M=%d K=%d N=%d" % (M, K, N))
        packed = bh.synth_ternary(seed, 1, N, K, bh.SYNTH_UNIFORM)
        x = bh.synth_normal(seed, 2, (M, K), 1.0)
        x[r.random((M, K)) < 0.01] *= 10.0
        g = np.ones(K, np.float32)
        out, xq = gpu_bitlinear(hip, x, packed, N, K, 0.02, g, canonical=1)
        _, oq, osc, _ = native.orc_quantize_rows(x, g)
        np.testing.assert_array_equal(xq, oq)
        same_bits(out, _epilogue_ref(oq, osc, packed, N, K, 0.02), "out")


# ------------------------------------------------------------ fp32 BitLinear
FP_SHAPES = [(1, 1024, 4384), (1, 2048, 8512), (1, 4096, 2048), (1, 2048, 50257),
             (3, 1024, 300), (1, 1000, 77), (2, 1026, 33), (1, 100, 10),
             (48, 2048, 520), (40, 4096, 260),
             # few tokens on MFMA: 1, 2, 3, 4, 5 and 16 slices of 1024 columns
             (7, 2048, 8512), (16, 4096, 2048), (12, 3072, 100), (9, 5120, 64), (31, 1024, 70),
             (30, 16384, 40),
             # up to 16 tokens on 8 MB of weights and more (nontemporal weight loads)
             (4, 8192, 4096), (13, 2048, 16384),
             # several token tiles of 32 (ragged last tile), and past the few-token range
             (64, 2048, 8384), (100, 4096, 2048), (256, 4096, 2048), (77, 3072, 96),
             (128, 2048, 8384),
             # the MFMA GEMM with partial last slices (K = 1.5, 3 and 5 slices of 1024)
             (300, 1536, 520), (400, 3072, 200), (260, 5120, 130),
             # 32x128 tiles (at most one 64x128 tile per CU), ragged last tiles
             (700, 1024, 2000),
             # 64x256 tiles (two 64x128 tiles per CU), ragged last tiles
             (1000, 2048, 3100)]


@pytest.mark.parametrize("M,K,N", FP_SHAPES)
def test_bitlinear_fp32_exact(hip, M, K, N):
    note("bitlinear fp32 M=%d K=%d N=%d" % (M, K, N))
    r = rnd(M + K * 3 + N)
    packed = r.integers(0, 256, (N, (K + 3) // 4), dtype=np.uint8)
    x = r.standard_normal((M, K)).astype(np.float32)
    x[:, r.integers(0, K, 3)] *= 10.0
    g = (r.standard_normal(K) * 0.02).astype(np.float32)
    out, xq = gpu_bitlinear(hip, x, packed, N, K, 0.02, g)
    ref, _, rq = native.orc_bitlinear(x, packed, N, K, 0.02, g)
    np.testing.assert_array_equal(xq, rq)
    assert rel_err(out, ref) <= 1e-4
    same_bits(out, ref, "out")


@pytest.mark.parametrize("K,N", [(1024, 4384), (2048, 8384), (4096, 2048), (8192, 1000),
                                 (1088, 300), (3072, 130), (5120, 64), (64, 7)])
def test_bitlinear_dev_one_token_fused(hip, K, N):
    """bm_hip_bitlinear_dev at one token on canonical weights (one launch of
    the decode's fused kernel, every block running the RMSNorm/int8
    prologue, block 0 writing x_quant and scale_x): out, x_quant and
    scale_x bit-exact against the oracle."""
    note("bitlinear_dev one token K=%d N=%d" % (K, N))
    r = rnd(7 * K + N)
    packed = bh.synth_ternary(K, N, N, K, bh.SYNTH_UNIFORM)
    x = r.standard_normal((1, K)).astype(np.float32)
    x[:, r.integers(0, K, 3)] *= 10.0
    g = (r.standard_normal(K) * 0.02).astype(np.float32)
    dx, dg, dw = DB.from_array(x), DB.from_array(g), DB.from_array(packed)
    do, dq, ds = DB(4 * N), DB(K), DB(4)
    da = DB(hip.bm_hip_act_bytes(1, K))
    bh.check(hip.bm_hip_bitlinear_dev(dx.ptr, 1, K, dg.ptr, dw.ptr, N, 0.02, 1, do.ptr, dq.ptr,
                                      K, ds.ptr, da.ptr, None), "bitlinear_dev")
    hip.bm_hip_synchronize()
    ref, _, rq = native.orc_bitlinear(x, packed, N, K, 0.02, g)
    _, oq, osc, _ = native.orc_quantize_rows(x, g)
    np.testing.assert_array_equal(dq.download((1, K), np.int8), rq)
    np.testing.assert_array_equal(dq.download((1, K), np.int8), oq)
    same_bits(ds.download(1, np.float32), osc.astype(np.float32), "scale_x")
    same_bits(do.download((1, N), np.float32), ref, "out")


def test_prefill_shapes_sampled(hip):
    """Prefill GEMM shapes M=2048: K=2048->N=8512 and K=4096->N=2048 (and
    M=1233, 1024 of the 1B prefill, which take the other tile shapes), fp32,
    activations N(0,1) with 1% outliers x10; 40 token rows (first/last tile
    included) checked bit-exactly against the oracle."""
    r = rnd(2048)
    for M, K, N, seed in ((2048, 2048, 8512, 11), (2048, 4096, 2048, 12),
                          (1233, 2048, 8512, 13), (1024, 2048, 8384, 14)):
        note("prefill M=%d K=%d N=%d" % (M, K, N))
        packed = bh.synth_ternary(seed, 1, N, K, bh.SYNTH_UNIFORM)
        x = bh.synth_normal(seed, 2, (M, K), 1.0)
        mask = r.random((M, K)) < 0.01
        x[mask] *= 10.0
        g = np.ones(K, np.float32)
        out, xq = gpu_bitlinear(hip, x, packed, N, K, 0.02, g, canonical=1)
        rows = np.unique(np.concatenate([[0, 1, 63, 64, 127, 128, M - 1], r.integers(0, M, 35)]))
        ref, _, rq = native.orc_bitlinear(x[rows], packed, N, K, 0.02, g)
        np.testing.assert_array_equal(xq[rows], rq)
        same_bits(out[rows], ref, "out[rows]")


# ------------------------------------------------------------ drop-in ABI
def test_dropin_cfg1_golden(hip):
    from golden.make_golden import cfg1_inputs, sha, CFG1
    z = np.load(os.path.join(GOLD, "bitlinear_k1024_n4384.npz"))
    packed, x, g = cfg1_inputs()
    assert sha(packed) == str(z["packed_sha256"]) and sha(x) == str(z["x_sha256"])
    K, N = CFG1["K"], CFG1["N"]
    w = bh.make_tensor(packed, N, K, CFG1["scale"])
    nw = bh.make_tensor(data=g)
    out = np.empty(N, np.float32)
    xn = np.empty(K, np.float32)
    xq = np.zeros(K + 32, np.int8)
    hip.hip_bitlinear_forward(ptr(x), K, C.byref(w), C.byref(nw), ptr(out), ptr(xn), ptr(xq))
    same_bits(out, z["out"][0], "out")
    same_bits(xn, z["x_norm"], "xn")
    np.testing.assert_array_equal(xq[:K], z["x_quant"][0])


def test_dropin_reused_host_buffers(hip):
    """The same host arrays refilled with other weights and norm between
    calls (as when an allocator reuses freed memory): every call must see the
    current contents, checked against the oracle."""
    K, N = 2048, 300
    packed = np.empty((N, K // 4), np.uint8)
    g = np.empty(K, np.float32)
    O = native.oracle()
    for seed in (21, 22, 23):
        note("drop-in reused buffers seed=%d" % seed)
        r = rnd(seed)
        packed[:] = r.integers(0, 256, packed.shape, dtype=np.uint8)
        g[:] = r.standard_normal(K).astype(np.float32)
        x = r.standard_normal(K).astype(np.float32)
        w = bh.make_tensor(packed, N, K, 0.03)
        nw = bh.make_tensor(data=g)
        out = np.empty(N, np.float32)
        xn = np.empty(K, np.float32)
        xq = np.zeros(K + 32, np.int8)
        hip.hip_bitlinear_forward(ptr(x), K, C.byref(w), C.byref(nw), ptr(out), ptr(xn), ptr(xq))
        ref = np.empty(N, np.float32)
        rxn = np.empty(K, np.float32)
        rxq = np.zeros(K + 32, np.int8)
        O.orc_bitlinear_forward(ptr(x), K, ptr(packed), N, K, C.c_float(0.03), ptr(g), ptr(ref),
                                ptr(rxn), ptr(rxq))
        same_bits(out, ref, "out seed %d" % seed)


# images registered with bm_hip_set_mmap stay registered for the process:
# they are kept alive here so that no later array reuses their addresses
_REGISTERED = []


def _dropin_call(hip, x, w, nw, N, K):
    out = np.full(N, np.nan, np.float32)
    xn = np.full(K, np.nan, np.float32)
    xq = np.full(K + 32, 77, np.int8)
    hip.hip_bitlinear_forward(ptr(x), K, C.byref(w), C.byref(nw), ptr(out), ptr(xn), ptr(xq))
    return out, xn, xq


def _dropin_ref(x, packed, N, K, scale, g):
    O = native.oracle()
    ref = np.empty(N, np.float32)
    rxn = np.empty(K, np.float32)
    rxq = np.zeros(K + 32, np.int8)
    O.orc_bitlinear_forward(ptr(x), K, ptr(packed), N, K, C.c_float(scale), ptr(g), ptr(ref),
                            ptr(rxn), ptr(rxq))
    return ref, rxn, rxq


# one token: the single-launch path (K % 64 == 0, outputs within the mapped
# buffer, at most 2048 blocks: the 50257-row LM heads take 786 and 1571)
# and the two-launch path (K = 1000, and an output too large for the mapped
# buffer); calls alternate shapes so that each one must see its own
# completion words
DROPIN_SHAPES = [(64, 1), (128, 3), (1024, 4192), (1000, 77), (1536, 65), (2048, 8384),
                 (3072, 130), (4096, 2048), (8192, 300), (2048, 50257), (1024, 70000),
                 (64, 2), (1024, 50257), (1024, 4384)]


def test_dropin_single_token_shapes(hip):
    """hip_bitlinear_forward at one token, out / x_norm / x_quant bit-exact
    against the oracle's bitlinear_forward (src/kernel.c:388-447) for each
    shape, on weights uploaded per call (codes 11 included)."""
    for i, (K, N) in enumerate(DROPIN_SHAPES):
        note("drop-in one token K=%d N=%d" % (K, N))
        r = rnd(400 + i)
        packed = r.integers(0, 256, (N, (K + 3) // 4), dtype=np.uint8)
        g = (1.0 + 0.1 * r.standard_normal(K)).astype(np.float32)
        x = r.standard_normal(K).astype(np.float32)
        x[r.integers(0, K, 2)] *= 8.0
        w = bh.make_tensor(packed, N, K, 0.025)
        nw = bh.make_tensor(data=g)
        out, xn, xq = _dropin_call(hip, x, w, nw, N, K)
        ref, rxn, rxq = _dropin_ref(x, packed, N, K, 0.025, g)
        same_bits(out, ref, "out K=%d N=%d" % (K, N))
        same_bits(xn, rxn, "x_norm K=%d N=%d" % (K, N))
        np.testing.assert_array_equal(xq[:K], rxq[:K])


def test_dropin_single_token_registered(hip):
    """The same entry on weights of a registered model image (1B and 255M
    widths: in_proj 2048 -> 8384 and 1024 -> 4192, out_proj 4096 -> 2048 and
    2048 -> 1024), several tokens in a row through each tensor."""
    for dm, nh in ((2048, 64), (1024, 32)):
        blob = bh.synth_model(1000, dm, 1, nh, 9, bh.SYNTH_UNIFORM)
        _REGISTERED.append(blob)
        assert hip.bm_hip_set_mmap(ptr(blob), blob.nbytes)
        for which, norm in ((bh.BM_L_IN_PROJ, bh.BM_L_IN_NORM),
                            (bh.BM_L_OUT_PROJ, bh.BM_L_OUT_NORM)):
            w = bh.image_tensors(blob, 0, which)
            nw = bh.image_tensors(blob, 0, norm)
            K, N = w.cols, w.rows
            packed = np.ctypeslib.as_array(C.cast(w.packed_data, C.POINTER(C.c_uint8)),
                                           (N * (K // 4),)).reshape(N, K // 4)
            g = np.ctypeslib.as_array(C.cast(nw.data, C.POINTER(C.c_float)), (K,))
            for t in range(3):
                note("drop-in registered dm=%d K=%d N=%d token %d" % (dm, K, N, t))
                x = rnd(500 + t).standard_normal(K).astype(np.float32)
                out, xn, xq = _dropin_call(hip, x, w, nw, N, K)
                ref, rxn, rxq = _dropin_ref(x, packed, N, K, w.scale, g)
                same_bits(out, ref, "out")
                same_bits(xn, rxn, "x_norm")
                np.testing.assert_array_equal(xq[:K], rxq[:K])


def test_dropin_batch_golden_shapes(hip):
    z = np.load(os.path.join(GOLD, "bitlinear_shapes.npz"))
    for key in sorted(k[4:] for k in z.files if k.startswith("out_")):
        K, N = map(int, key.split("_"))
        note("drop-in batch golden K=%d N=%d" % (K, N))
        p, x, g = z["packed_" + key], z["x_" + key], z["g_" + key]
        M = x.shape[0]
        w = bh.make_tensor(p, N, K, 0.037)
        nw = bh.make_tensor(data=g)
        out = np.empty((M, N), np.float32)
        xn = np.empty(K, np.float32)
        xq = np.zeros((M, K + 32), np.int8)
        hip.hip_bitlinear_forward_batch(ptr(x), M, K, C.byref(w), C.byref(nw), ptr(out),
                                        ptr(xn), ptr(xq), K + 32)
        same_bits(out, z["out_" + key], "out")
        np.testing.assert_array_equal(xq[:, :K], z["xq_" + key])


def test_register_table(hip):
    t = bh.Dispatch()
    t.ssm_inner = 1234
    assert hip.bm_hip_register(C.byref(t))
    assert t.name == b"hip" and t.bitlinear_prepare is None and t.bitlinear_row_worker is None
    assert t.ssm_inner == 1234 and t.bitlinear_forward and t.rms_norm


def test_set_mmap_registers_model(hip):
    blob = bh.synth_model(1000, 128, 2, 4, 5, bh.SYNTH_RAW_BYTES)
    _REGISTERED.append(blob)
    assert hip.bm_hip_set_mmap(ptr(blob), blob.nbytes)
