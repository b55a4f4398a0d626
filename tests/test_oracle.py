"""The oracle (oracle/bm_oracle.c) pinned three ways:

* against the reference's own C compiled here (oracle/_ref, scalar kernels
  forced): bit-exact for every fp32 and int8 output;
* against closed forms in numpy (decode table, int32 brute force);
* against invariants the scalar path must satisfy (scale invariance of the
  int8 vector, the largest element quantizing to +-127, ties away from zero).
"""
import ctypes as C

import numpy as np
import pytest

import native
from native import bh, ptr, same_bits


def rnd(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- a1 decode
def test_decode_closed_form():
    O = native.oracle()
    assert [O.orc_decode_weight(b) for b in range(4)] == [-1, 0, 1, 1]
    unpack = np.empty((256, 4), np.int8)
    pm = np.empty(256, np.uint8)
    nm = np.empty(256, np.uint8)
    O.orc_luts(ptr(unpack), ptr(pm), ptr(nm))
    b = np.arange(256, dtype=np.uint8)[:, None]
    expect = native.decode_dense(b, 4)
    np.testing.assert_array_equal(unpack, expect)
    np.testing.assert_array_equal(pm, ((expect == 1) * (1 << np.arange(4))).sum(1))
    np.testing.assert_array_equal(nm, ((expect == -1) * (1 << np.arange(4))).sum(1))


def test_decode_vs_reference(ref_lib):
    O = native.oracle()
    ref_lib.bmref_init(1, 0)
    tabs = [np.empty((256, 4), np.int8), np.empty(256, np.uint8), np.empty(256, np.uint8)]
    rtabs = [np.empty_like(t) for t in tabs]
    O.orc_luts(*(ptr(t) for t in tabs))
    ref_lib.bmref_lut(*(ptr(t) for t in rtabs))
    for a, b in zip(tabs, rtabs):
        np.testing.assert_array_equal(a, b)


def test_prng_vs_reference(ref_lib):
    import ctypes as C
    O = native.oracle()
    for seed in (1, 42, 0xDEADBEEF):
        ref_lib.bmref_rng_seed(seed)
        st = C.c_uint64(seed)
        for _ in range(100):
            assert O.orc_rng_next(C.byref(st)) == ref_lib.bmref_rng_next()


# ------------------------------------------------------- a3/a4 rms + quant
@pytest.mark.parametrize("n", [1, 3, 4, 7, 64, 1000, 1024, 2048, 4096, 4099])
def test_rms_norm_vs_reference(ref_lib, n):
    ref_lib.bmref_init(1, 0)
    O = native.oracle()
    r = rnd(n)
    for trial in range(5):
        x = (r.standard_normal(n) * (10.0 ** r.integers(-3, 3))).astype(np.float32)
        g = r.standard_normal(n).astype(np.float32)
        a = np.empty(n, np.float32)
        b = np.empty(n, np.float32)
        ma = O.orc_rms_norm(ptr(x), n, ptr(g), ptr(a))
        mb = ref_lib.bmref_rms_norm(ptr(x), n, ptr(g), ptr(b))
        same_bits(np.float32(ma), np.float32(mb), "np.float32(ma)")
        same_bits(a, b, "a")


def test_quantize_invariants():
    r = rnd(7)
    n = 2048
    g = np.ones(n, np.float32)
    x = r.standard_normal((20, n)).astype(np.float32)
    xn, xq, sc, mx = native.orc_quantize_rows(x, g)
    # the element of largest magnitude maps to +-127 (v*scale just under 127)
    for m in range(20):
        i = np.argmax(np.abs(xn[m]))
        assert abs(int(xq[m, i])) == 127
    assert np.all(np.abs(xq.astype(int)) <= 127)
    # RMSNorm makes the int8 vector invariant to a power-of-two input scale
    _, xq2, _, _ = native.orc_quantize_rows(x * np.float32(8.0), g)
    np.testing.assert_array_equal(xq, xq2)
    # ties go away from zero: v = k + 0.5 exactly
    O = native.oracle()
    v = np.array([0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -0.49], np.float32)
    q = np.empty(v.size, np.int8)
    # max_abs chosen so that scale_x == 1.0f exactly: 127/(126+1e-5) != 1,
    # so quantize with max such that 127/(max+1e-5f) rounds to 1.0f
    mx = np.float32(127.0) - np.float32(1e-5)
    sc = O.orc_quantize(ptr(v), v.size, float(mx), ptr(q))
    assert sc == 1.0
    assert q.tolist() == [1, -1, 2, -2, 3, -3, 127, 0]


# ------------------------------------------------- a5-a8 bitlinear forward
SHAPES = [(1024, 64), (1024, 4384), (2048, 257), (4096, 96), (1000, 33), (1026, 17),
          (64, 5), (3, 4), (8192, 40)]


@pytest.mark.parametrize("K,N", SHAPES)
def test_bitlinear_vs_reference(ref_lib, K, N):
    ref_lib.bmref_init(1, 0)
    r = rnd(K * 131 + N)
    packed = r.integers(0, 256, (N, (K + 3) // 4), dtype=np.uint8)  # codes 11 included
    M = 3
    x = r.standard_normal((M, K)).astype(np.float32)
    x[1] *= 50
    g = (r.standard_normal(K) * 0.5).astype(np.float32)
    a = native.orc_bitlinear(x, packed, N, K, 0.02, g)
    b = native.ref_bitlinear(x, packed, N, K, 0.02, g)
    for u, v in zip(a, b):
        same_bits(u, v, "u")


@pytest.mark.parametrize("K,N", [(1024, 50), (2048, 31), (1030, 9), (4096, 12)])
def test_slice_totals_closed_form(K, N):
    r = rnd(K + N)
    packed = r.integers(0, 256, (N, (K + 3) // 4), dtype=np.uint8)
    xq = r.integers(-128, 128, K, dtype=np.int8)
    st, rt = native.orc_slice_totals(xq, packed, N, K)
    w = native.decode_dense(packed, K).astype(np.int64)
    x = xq.astype(np.int64)
    ng = K // 4
    for s in range(st.shape[1]):
        c0, c1 = 1024 * s, min(1024 * (s + 1), 4 * ng)
        np.testing.assert_array_equal(st[:, s], w[:, c0:c1] @ x[c0:c1])
    np.testing.assert_array_equal(rt, w[:, 4 * ng:] @ x[4 * ng:])
    full = native.orc_gemm_i32(xq[None, :], packed, N, K)[0]
    np.testing.assert_array_equal(full, w @ x)


def test_rows_epilogue_order():
    """fp32 out = sum over 1024-blocks of fl(total*inv) in block order: a
    dropped or reordered block changes the low bits."""
    r = rnd(3)
    K, N = 4096, 64
    packed = r.integers(0, 256, (N, K // 4), dtype=np.uint8)
    xq = r.integers(-128, 128, K, dtype=np.int8)
    inv = np.float32(0.0123457)
    out = np.empty(N, np.float32)
    native.oracle().orc_tmac_rows_f32(ptr(xq), ptr(packed), N, K, float(inv), ptr(out))
    st, _ = native.orc_slice_totals(xq, packed, N, K)
    acc = np.zeros(N, np.float32)
    for s in range(4):
        acc = (acc + (st[:, s].astype(np.float32) * inv).astype(np.float32)).astype(np.float32)
    same_bits(out, acc, "out")


# ----------------------------------------------------------- a15 SSM step
def test_ssm_inner_vs_reference(ref_lib):
    import ctypes as C
    ref_lib.bmref_init(1, 0)

    class Args(C.Structure):
        _fields_ = [(n, C.c_void_p) for n in
                    ("z", "x", "B", "C", "dt", "dt_bias", "A", "cw", "cb", "cs0", "cs1", "cs2",
                     "csw", "state", "D", "y")] + [("head_dim", C.c_int), ("d_inner", C.c_int),
                                                   ("n_heads", C.c_int)]

    ref_lib.bmref_ssm_inner.argtypes = [C.POINTER(Args), C.c_int, C.c_int]
    r = rnd(11)
    di, nh = 512, 8
    proj = (r.standard_normal(2 * di + 3 * nh) * 3).astype(np.float32)
    dtb = r.standard_normal(nh).astype(np.float32)
    A = -np.exp(r.standard_normal(nh)).astype(np.float32)
    cw = r.standard_normal((4, di)).astype(np.float32)
    cb = r.standard_normal(di).astype(np.float32)
    D = r.standard_normal(di).astype(np.float32)
    cs = r.standard_normal((3, di)).astype(np.float32)
    st = r.standard_normal(di).astype(np.float32)
    proj[2 * di + 2 * nh] = 30.0  # softplus linear branch

    outs = []
    for who in ("orc", "ref"):
        cs_ = cs.copy()
        st_ = st.copy()
        y = np.empty(di, np.float32)
        p_ = proj.copy()
        if who == "orc":
            native.oracle().orc_ssm_inner(ptr(p_), di, nh, ptr(dtb), ptr(A), ptr(cw), ptr(cb),
                                          ptr(cs_[0]), ptr(cs_[1]), ptr(cs_[2]), ptr(st_),
                                          ptr(D), ptr(y), 0, di)
        else:
            base = p_.ctypes.data
            a = Args(base, base + 4 * di, base + 8 * di, base + 8 * di + 4 * nh,
                     base + 8 * di + 8 * nh, dtb.ctypes.data, A.ctypes.data, cw.ctypes.data,
                     cb.ctypes.data, cs_[0].ctypes.data, cs_[1].ctypes.data, cs_[2].ctypes.data,
                     cs_[0].ctypes.data, st_.ctypes.data, D.ctypes.data, y.ctypes.data,
                     di // nh, di, nh)
            ref_lib.bmref_ssm_inner(C.byref(a), 0, di)
        outs.append((cs_, st_, y))
    for u, v in zip(*outs):
        same_bits(u, v, "u")


# --------------------------------------------------- end-to-end (model)
def _tiny_model(seed, dist=bh.SYNTH_UNIFORM, vocab=1000, d_model=128, n_layers=2, n_heads=4):
    return bh.synth_model(vocab, d_model, n_layers, n_heads, seed, dist)


def _ref_stream(ref_lib, path, prompt, steps):
    h = ref_lib.bmref_model_load(path.encode())
    assert h
    try:
        if len(prompt) > 1:
            p = np.ascontiguousarray(prompt[:-1], np.int32)
            ref_lib.bmref_model_prefill(h, ptr(p), len(p))
        hist = list(prompt)
        cur = int(prompt[-1])
        toks, logits = [], []
        V = ref_lib.bmref_model_vocab(h)
        for _ in range(steps):
            harr = np.array(hist[-256:], np.int32)
            cur = ref_lib.bmref_model_step(h, cur, ptr(harr), len(harr), 1.0)
            toks.append(cur)
            logits.append(np.ctypeslib.as_array(ref_lib.bmref_model_logits(h), (V,)).copy())
            hist.append(cur)
        return toks, logits
    finally:
        ref_lib.bmref_model_free(h)


def orc_stream(blob, prompt, steps):
    O = native.oracle()
    h = O.orc_model_load(ptr(blob), blob.nbytes)
    assert h
    try:
        if len(prompt) > 1:
            p = np.ascontiguousarray(prompt[:-1], np.int32)
            O.orc_model_prefill(h, ptr(p), len(p))
        hist = list(prompt)
        cur = int(prompt[-1])
        V = O.orc_model_config(h, 0)
        toks, logits = [], []
        for _ in range(steps):
            harr = np.array(hist[-256:], np.int32)
            cur = O.orc_model_step(h, cur, ptr(harr), len(harr), 1.0)
            toks.append(cur)
            logits.append(np.ctypeslib.as_array(O.orc_model_logits(h), (V,)).copy())
            hist.append(cur)
        return toks, logits
    finally:
        O.orc_model_free(h)


@pytest.mark.parametrize("seed,dist", [(5, bh.SYNTH_UNIFORM), (6, bh.SYNTH_P0_40)])
def test_model_vs_reference(ref_lib, tmp_path, seed, dist):
    ref_lib.bmref_init(2, 0)
    blob = _tiny_model(seed, dist)
    path = tmp_path / "m.bin"
    blob.tofile(path)
    prompt = bh.synth_prompt(seed, 1000, 8)
    t1, l1 = orc_stream(blob, prompt, 12)
    t2, l2 = _ref_stream(ref_lib, str(path), prompt, 12)
    assert t1 == t2
    for a, b in zip(l1, l2):
        same_bits(a, b, "a")


def test_model_loader_rejects_malformed():
    O = native.oracle()
    blob = _tiny_model(1)
    assert O.orc_model_load(ptr(blob), blob.nbytes)  # sanity (leaks a handle: tiny)
    bad = blob.copy()
    bad[:4] = 0
    assert not O.orc_model_load(ptr(bad), bad.nbytes)
    trunc = blob[: blob.nbytes // 2].copy()
    assert not O.orc_model_load(ptr(trunc), trunc.nbytes)


# --------------------------------------------------- sampler
# (temp, min_p, top_p, top_k, penalty, seed): every branch of
# sample_advanced (src/model.c:132-361) on the tiny model's logits
SAMPLER_CASES = [
    (0.8, 0.05, 0.9, 40, 1.0, 42),    # top-k heap, sorted for top_p
    (1.0, 0.0, 1.0, 40, 1.0, 7),      # top-k heap, CDF in heap order
    (1.2, 0.0, 0.95, 256, 1.3, 9),    # k = 256 with the repetition penalty
    (0.7, 0.0, 0.9, 0, 1.0, 11),      # no top-k: top-256 partial sort
    (10.0, 0.0, 0.99, 0, 1.0, 13),    # flat: the partial sort falls short, full sort
    (1.0, 0.1, 1.0, 0, 1.0, 17),      # min_p, CDF in index order
    (10.0, 0.0, 1.0, 300, 1.0, 19),   # top_k > 256: full sort, then top_k
    (1.0, 1.0, 1.0, 0, 1.0, 23),      # min_p = 1: only the maximum survives
    (0.9, 0.0, 1.0, 1, 1.0, 29),      # top_k = 1
    (0.01, 0.0, 1.0, 0, 1.0, 31),     # temp < 0.05: greedy
]
SAMPLER_MODEL = dict(vocab=5000, d_model=128, n_layers=2, n_heads=4, seed=21)


def sampler_model():
    c = SAMPLER_MODEL
    blob = bh.synth_model(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["seed"],
                          bh.SYNTH_UNIFORM)
    return blob, bh.synth_prompt(c["seed"], c["vocab"], 8)


def sampler_branch(logits, temp, min_p, top_p, top_k):
    """Which branch of sample_advanced these logits take (numpy, float32
    like the reference); used to show the cases cover all of them."""
    if temp < 0.05:
        return "greedy"
    z = (logits * np.float32(1.0 / np.float32(temp))).astype(np.float32)
    mx = z.max()
    thr = np.float32(-1e30)
    if min_p >= 1.0:
        thr = mx
    elif min_p > 0.0:
        thr = np.float32(mx + np.float32(np.log(np.float32(min_p))))
    if 0 < top_k <= 256:
        return "topk_heap" if (z >= thr).sum() > top_k else "topk"
    n = int((z >= thr).sum())
    if top_p >= 1.0 and (top_k <= 0 or top_k >= n):
        return "direct"
    if top_p < 1.0 and n > 256:
        p = np.exp((z[z >= thr] - mx).astype(np.float64))
        p /= p.sum()
        return "partial" if np.sort(p)[::-1][:256].sum() >= top_p * (1 - 1e-6) else "full"
    return "full"


def sampler_ref_stream(ref_lib, path, prompt, steps, case):
    """The reference's sampled stream with, in lockstep, a greedy instance
    that exposes the logits each draw sees."""
    temp, min_p, top_p, top_k, penalty, seed = case
    hs = ref_lib.bmref_model_load(path.encode())
    hg = ref_lib.bmref_model_load(path.encode())
    assert hs and hg
    try:
        p = np.ascontiguousarray(prompt[:-1], np.int32)
        ref_lib.bmref_model_prefill(hs, ptr(p), len(p))
        ref_lib.bmref_model_prefill(hg, ptr(p), len(p))
        ref_lib.bmref_rng_seed(seed)
        V = ref_lib.bmref_model_vocab(hs)
        hist, cur = list(prompt), int(prompt[-1])
        toks, seen = [], []
        for _ in range(steps):
            harr = np.array(hist[-256:], np.int32)
            ref_lib.bmref_model_step(hg, cur, ptr(harr), len(harr), penalty)
            seen.append(np.ctypeslib.as_array(ref_lib.bmref_model_logits(hg), (V,)).copy())
            cur = ref_lib.bmref_model_step_sample(hs, cur, ptr(harr), len(harr), penalty, temp,
                                                  min_p, top_p, top_k)
            toks.append(cur)
            hist.append(cur)
        return toks, seen
    finally:
        ref_lib.bmref_model_free(hs)
        ref_lib.bmref_model_free(hg)


def test_sampler_vs_reference(ref_lib, tmp_path):
    """orc_sample draws the reference's token from the same logits and
    generator state on every branch; min_p = 1 and top_k = 1 reduce to the
    first maximum."""
    ref_lib.bmref_init(2, 0)
    blob, prompt = sampler_model()
    path = tmp_path / "s.bin"
    blob.tofile(path)
    O = native.oracle()
    branches = set()
    for case in SAMPLER_CASES:
        temp, min_p, top_p, top_k, penalty, seed = case
        toks, seen = sampler_ref_stream(ref_lib, str(path), prompt, 16, case)
        rng = C.c_uint64(seed if seed else 0x853C49E6748FEA9B)
        for t, lg in zip(toks, seen):
            branches.add(sampler_branch(lg, temp, min_p, top_p, top_k))
            work = lg.copy()
            got = O.orc_sample(ptr(work), lg.size, temp, min_p, top_p, top_k, C.byref(rng))
            assert got == t, case
            if min_p >= 1.0 or top_k == 1 or temp < 0.05:
                assert t == int(np.argmax(lg)), case
    assert branches >= {"greedy", "topk", "topk_heap", "direct", "partial", "full"}, branches
