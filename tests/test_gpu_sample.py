"""GPU parity of the device sampler on its own (bm_hip_sample_advanced)
against the oracle's restatement of sample_advanced (src/model.c:132-361).

Bar: bit-exact token, scaled logits and generator state, over every branch
of the sampler, vocabulary sizes that are not multiples of the kernel's
4-wide loads (1, 3, 7, 4999, 50257), vocabularies past 65535 (whose
histogram pass walks several rows per block and whose full sort needs
32-bit offsets) up to the loader's limit of 256000 (src/bitmamba.h:55),
and logits with ties, infinities and a long tail far below the maximum.
"""
import numpy as np
import pytest

import native
from native import bh, ptr

pytestmark = pytest.mark.gpu

# (temp, min_p, top_p, top_k): the branches of sample_advanced
PARAMS = [
    (0.8, 0.05, 0.9, 40),      # histogram + heap + top_p sort (the CLI's sampled default)
    (1.0, 0.0, 1.0, 40),       # histogram without min_p: the far tail counted too
    (1.2, 0.0, 0.95, 256),     # largest heap
    (0.9, 0.0, 1.0, 1),        # top-1
    (0.7, 0.0, 0.9, 0),        # partial top-256 sort
    (10.0, 0.0, 0.99, 0),      # full sort
    (1.0, 0.1, 1.0, 0),        # direct CDF walk in index order
    (10.0, 0.0, 1.0, 300),     # top_k above the heap limit
    (1.0, 1.0, 1.0, 0),        # only the maximum survives min_p
    (0.01, 0.0, 1.0, 0),       # greedy
]
VOCABS = [1, 3, 7, 4999, 50257, 65535, 65536, 100003, 256000]


def _logits(kind, V, seed):
    r = np.random.default_rng(seed)
    if kind == "normal":
        return (r.standard_normal(V) * 3.0).astype(np.float32)
    if kind == "ties":       # few distinct values: ties everywhere
        return (np.round(r.standard_normal(V) * 2.0) * 0.5).astype(np.float32)
    # a long tail far below the maximum, and infinities
    x = (r.standard_normal(V) * 40.0).astype(np.float32)
    if V > 8:
        x[r.integers(0, V, size=max(1, V // 100))] = -np.inf
    return x


def _check(V, kind, params, seed, draws=2):
    temp, min_p, top_p, top_k = params
    lg = _logits(kind, V, seed)
    rng = 0x853c49e6748fea9b ^ seed
    for d in range(draws):
        t_dev, l_dev, r_dev = bh.sample_advanced(lg, temp, min_p, top_p, top_k, rng)
        ref = lg.copy()
        st = native.C.c_uint64(rng)
        t_orc = native.oracle().orc_sample(ptr(ref), V, temp, min_p, top_p, top_k,
                                           native.C.byref(st))
        case = (V, kind, params, seed, d)
        assert t_dev == t_orc, case
        assert r_dev == st.value, case
        assert l_dev.view(np.uint32).tolist() == ref.view(np.uint32).tolist(), case
        rng = st.value
        lg = ref  # the next draw starts from the scaled logits, as a caller reusing them


@pytest.mark.parametrize("V", VOCABS)
@pytest.mark.parametrize("kind", ["normal", "ties", "tail"])
def test_sample_advanced_vs_oracle(hip, V, kind):
    for i, params in enumerate(PARAMS):
        _check(V, kind, params, seed=1000 * i + V % 997)


def test_sample_advanced_rejects(hip):
    L = hip
    buf = bh.DeviceBuffer(bh.lib().bm_hip_sample_workspace_bytes(65535) + 64)
    try:
        p = buf.ptr
        for V in (0, -1, 256001):
            assert L.bm_hip_sample_advanced(p, V, 1.0, 0.0, 1.0, 0, p, p, p, None) == -1
        assert L.bm_hip_sample_advanced(p + 4, 8, 1.0, 0.0, 1.0, 0, p, p, p, None) == -1
        assert "aligned" in bh.last_error()
        assert L.bm_hip_sample_advanced(None, 8, 1.0, 0.0, 1.0, 0, p, p, p, None) == -1
    finally:
        buf.free()
