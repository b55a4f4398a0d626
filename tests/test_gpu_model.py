"""GPU parity of the device-resident model (bm_hip_model_*) against the
oracle and the reference's greedy streams.

Bar: every logit and every recurrent-state value bit-exact at sizes the
oracle runs in seconds; identical greedy token streams at the full 255M- and
1B-shape configurations (streams written by the reference's own scalar
build, tests/golden/stream_*.json).
"""
import json
import os

import numpy as np
import pytest

import native
from native import bh, ptr, same_bits

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def note(msg):
    print("[case] " + msg, flush=True)


def gold(name):
    with open(os.path.join(GOLD, "stream_%s.json" % name)) as f:
        return json.load(f)


def model_image(g):
    c = g["config"]
    blob = bh.synth_model(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["seed"],
                          c["dist"])
    assert blob.nbytes == g["blob_bytes"]
    return blob, np.array(g["prompt"], np.int32), c["steps"]


def test_device_libm(hip):
    """Device expf/logf vs the host glibc on 2^24 inputs: every float bit
    pattern with a stride, plus dense samples of the SSM's ranges."""
    note("device libm")
    r = np.random.default_rng(1)
    strided = (np.arange(1 << 23, dtype=np.uint64) * 512 + 7).astype(np.uint32).view(np.float32)
    dense = np.concatenate([r.uniform(-30, 30, 1 << 22), r.uniform(-1, 1, 1 << 22),
                            r.uniform(0, 50, 1 << 21)]).astype(np.float32)
    x = np.concatenate([strided, dense]).astype(np.float32)
    x = x[~np.isnan(x)]
    dx = bh.DeviceBuffer.from_array(x)
    dy = bh.DeviceBuffer(x.nbytes)
    for fn, name in ((0, "expf"), (1, "logf")):
        bh.check(hip.bm_hip_libm_eval_dev(fn, dx.ptr, dy.ptr, x.size, None), name)
        hip.bm_hip_synchronize()
        got = dy.download(x.shape, np.float32)
        ref = np.empty_like(x)
        getattr(native.oracle(), "orc_%s_array" % name)(ptr(x), ptr(ref), x.size)
        both_nan = np.isnan(got) & np.isnan(ref)
        got[both_nan] = 0
        ref[both_nan] = 0
        same_bits(got, ref, name)


def test_device_division_sqrt_and_silu(hip):
    """Device fp32 division, sqrt and silu against the host's IEEE float
    arithmetic (numpy float32, and the oracle's glibc expf inside silu): 2^24
    pairs of every-exponent bit patterns (zeros, subnormals, infinities
    included) and of the ranges the sampler, the norms and the SSM use."""
    note("device division and silu")
    r = np.random.default_rng(2)
    bits = r.integers(0, 1 << 32, 1 << 23, dtype=np.uint64).astype(np.uint32).view(np.float32)
    specials = np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 1.1754942e-38,
                         1.1754944e-38, 3.4028235e38, -3.4028235e38, 1.0, -1.0, 127.0,
                         1e-5, 20.0, 255.0], np.float32)
    pairs = np.stack(np.meshgrid(specials, specials), -1).reshape(-1)
    dense = np.concatenate([r.uniform(-30, 30, 1 << 22), r.uniform(1e-6, 100, 1 << 22),
                            r.uniform(-1, 1, 1 << 21)]).astype(np.float32)
    x = np.concatenate([pairs, bits, dense]).astype(np.float32)
    x = x[: x.size // 2 * 2]
    x = x[~np.isnan(x).reshape(-1, 2).any(1).repeat(2)]
    dx = bh.DeviceBuffer.from_array(x)
    dy = bh.DeviceBuffer(x.nbytes)
    O = native.oracle()
    with np.errstate(all="ignore"):
        partner = x.reshape(-1, 2)[:, ::-1].reshape(-1)
        ref_div = (x / partner).astype(np.float32)
        e = np.empty_like(x)
        O.orc_expf_array(ptr(np.ascontiguousarray(-x)), ptr(e), x.size)
        ref_silu = (x / (np.float32(1.0) + e)).astype(np.float32)
        ref_sqrt = np.sqrt(x).astype(np.float32)
    for fn, name, ref in ((2, "division", ref_div), (3, "silu", ref_silu), (4, "sqrt", ref_sqrt)):
        bh.check(hip.bm_hip_libm_eval_dev(fn, dx.ptr, dy.ptr, x.size, None), name)
        hip.bm_hip_synchronize()
        got = dy.download(x.shape, np.float32)
        ref = ref.copy()
        both_nan = np.isnan(got) & np.isnan(ref)
        got[both_nan] = 0
        ref[both_nan] = 0
        same_bits(got, ref, name)
    assert hip.bm_hip_libm_eval_dev(5, dx.ptr, dy.ptr, x.size, None) == -1


def _oracle_model(blob):
    O = native.oracle()
    h = O.orc_model_load(ptr(blob), blob.nbytes)
    assert h
    return O, h


@pytest.mark.parametrize("penalty", [1.0, 1.3])
def test_tiny_model_logits_and_state(hip, penalty):
    """Prefill state, then every step's logits (after the penalty) and the
    greedy token, bit-exact against the oracle."""
    g = gold("tiny")
    blob, prompt, steps = model_image(g)
    note("tiny model penalty=%g" % penalty)
    m = bh.Model(blob)
    O, h = _oracle_model(blob)
    try:
        p = prompt[:-1].copy()
        m.prefill(p)
        O.orc_model_prefill(h, ptr(p), p.size)
        for layer in range(m.n_layers):
            cs, ss, pos = m.layer_state(layer)
            ocs = np.empty((3, m.d_inner), np.float32)
            oss = np.empty(m.d_inner, np.float32)
            opos = O.orc_model_layer_state(h, layer, ptr(ocs), ptr(oss))
            assert pos == opos
            same_bits(cs, ocs, "conv_state[%d]" % layer)
            same_bits(ss, oss, "ssm_state[%d]" % layer)
        hist = [int(t) for t in prompt]
        cur = int(prompt[-1])
        for s in range(steps):
            harr = np.array(hist[-256:], np.int32)
            a = m.step(cur, harr, penalty)
            b = O.orc_model_step(h, cur, ptr(harr), harr.size, penalty)
            same_bits(m.logits(), np.ctypeslib.as_array(O.orc_model_logits(h), (m.vocab,)),
                      "logits step %d" % s)
            assert a == b
            hist.append(a)
            cur = a
        if penalty == 1.0:
            assert hist[len(prompt):] == g["tokens"]
    finally:
        O.orc_model_free(h)
        m.free()


@pytest.mark.parametrize("d_model,n_heads,penalty", [(1024, 32, 1.0), (2048, 64, 1.3)])
def test_wide_model_logits_vs_oracle(hip, d_model, n_heads, penalty):
    """Two-layer models at the 255M and 1B widths (2000-token vocabulary):
    the prefill state and every step's logits bit-exact against the oracle.
    At these widths (K = 1024, 2048, 4096) the decode kernels keep their
    input in registers and run the register-resident sums of squares."""
    note("wide model d_model=%d penalty=%g" % (d_model, penalty))
    blob = bh.synth_model(2000, d_model, 2, n_heads, 77 + d_model, bh.SYNTH_UNIFORM)
    prompt = bh.synth_prompt(77, 2000, 8)
    m = bh.Model(blob)
    O, h = _oracle_model(blob)
    try:
        p = prompt[:-1].copy()
        m.prefill(p)
        O.orc_model_prefill(h, ptr(p), p.size)
        for layer in range(m.n_layers):
            cs, ss, pos = m.layer_state(layer)
            ocs = np.empty((3, m.d_inner), np.float32)
            oss = np.empty(m.d_inner, np.float32)
            assert pos == O.orc_model_layer_state(h, layer, ptr(ocs), ptr(oss))
            same_bits(cs, ocs, "conv_state[%d]" % layer)
            same_bits(ss, oss, "ssm_state[%d]" % layer)
        hist, cur = [int(t) for t in prompt], int(prompt[-1])
        for s in range(6):
            harr = np.array(hist[-256:], np.int32)
            a = m.step(cur, harr, penalty)
            b = O.orc_model_step(h, cur, ptr(harr), harr.size, penalty)
            same_bits(m.logits(), np.ctypeslib.as_array(O.orc_model_logits(h), (m.vocab,)),
                      "logits step %d" % s)
            assert a == b
            hist.append(a)
            cur = a
    finally:
        O.orc_model_free(h)
        m.free()


# Shapes the loader accepts that the fused decode kernels do not cover:
# d_model % 64 != 0 (in_proj and LM head through the generic quantize +
# product kernels), a head dim that is not a multiple of 16 (in_proj + the
# per-head SSM kernel), d_inner > 8192 with head dims past 1024 (out_proj
# through the generic kernels, several SSM blocks per head), and a vocabulary
# past 65535 under the sampler.
ODD_SHAPES = [  # (vocab, d_model, n_heads, penalty, sampler)
    (300, 96, 4, 1.0, None),
    (300, 96, 4, 1.3, None),
    (257, 128, 32, 1.0, None),
    (100, 4160, 5, 1.0, None),
    (70001, 64, 2, 1.0, (0.9, 0.0, 0.95, 0)),
    (70001, 64, 2, 1.2, (1.1, 0.05, 0.9, 40)),
]


@pytest.mark.parametrize("vocab,d_model,n_heads,penalty,sampler", ODD_SHAPES)
def test_odd_shapes_vs_oracle(hip, vocab, d_model, n_heads, penalty, sampler):
    """One-layer models of the shapes above: the prefill state, then every
    step's logits (after the penalty; divided by the temperature when
    sampled) and token bit-exact against the oracle (orc_sample for the
    sampled ones), through single steps and through the captured graph of
    bm_hip_model_generate."""
    note("odd shape vocab=%d d_model=%d heads=%d penalty=%g sampler=%s"
         % (vocab, d_model, n_heads, penalty, sampler))
    blob = bh.synth_model(vocab, d_model, 1, n_heads, 5 + d_model + vocab, bh.SYNTH_UNIFORM)
    prompt = bh.synth_prompt(5 + d_model, vocab, 8)
    m = bh.Model(blob)
    O, h = _oracle_model(blob)
    try:
        p = prompt[:-1].copy()
        m.prefill(p)
        O.orc_model_prefill(h, ptr(p), p.size)
        cs, ss, pos = m.layer_state(0)
        ocs = np.empty((3, m.d_inner), np.float32)
        oss = np.empty(m.d_inner, np.float32)
        assert pos == O.orc_model_layer_state(h, 0, ptr(ocs), ptr(oss))
        same_bits(cs, ocs, "conv_state")
        same_bits(ss, oss, "ssm_state")
        rng = native.C.c_uint64(0x853c49e6748fea9b)
        if sampler:
            m.set_sampler(*sampler)
            m.seed(0x853c49e6748fea9b)
        hist, cur = [int(t) for t in prompt], int(prompt[-1])
        for i in range(5):
            harr = np.array(hist[-256:], np.int32)
            t_dev = m.step(cur, harr, penalty)
            t_orc = O.orc_model_step(h, cur, ptr(harr), harr.size, penalty)
            lg = np.ctypeslib.as_array(O.orc_model_logits(h), (vocab,)).copy()
            if sampler:
                t_orc = O.orc_sample(ptr(lg), vocab, sampler[0], sampler[1], sampler[2],
                                     sampler[3], native.C.byref(rng))
            same_bits(m.logits(), lg, "logits step %d" % i)
            assert t_dev == t_orc, i
            hist.append(t_dev)
            cur = t_dev
        # the same steps as one captured graph each, from the prompt again
        m.reset()
        if sampler:
            m.seed(0x853c49e6748fea9b)
        toks, _ = m.generate(prompt, 5, penalty)
        assert [int(t) for t in toks] == hist[len(prompt):]
    finally:
        O.orc_model_free(h)
        m.free()


# GEMM tiles of the 1B width: 300 tokens 64x128, 1220 in_proj 128x128, 2100
# 128x256 (three SSM chunks); 255M width, 1030 tokens: in_proj 128x256,
# out_proj 64x128, two SSM chunks; d_model 320: out_proj (K=640 -> N=320)
# in 64x128 tiles with 128-deep stages, its residual add over ragged last
# row and column tiles; 1600 tokens: out_proj in 64x256 tiles
@pytest.mark.parametrize("d_model,n_heads,n_tokens", [(1024, 32, 1030), (2048, 64, 300),
                                                      (2048, 64, 1220), (2048, 64, 2100),
                                                      (320, 10, 300), (2048, 64, 1600)])
def test_wide_model_long_prefill_vs_oracle(hip, d_model, n_heads, n_tokens):
    """Long prompts at the 255M and 1B widths (two layers, 2000-token
    vocabulary): the batched path with MFMA GEMM tiles, the quantize kernels
    at K = 1024 .. 4096 and, at 1030 tokens, two chunks of the three-phase
    SSM with 64-channel heads.  Every state value and the next step's logits
    bit-exact against the oracle's token-serial prefill."""
    note("wide model long prefill d_model=%d tokens=%d" % (d_model, n_tokens))
    blob = bh.synth_model(2000, d_model, 2, n_heads, 91 + d_model, bh.SYNTH_UNIFORM)
    prompt = bh.synth_prompt(91, 2000, n_tokens + 1)
    m = bh.Model(blob)
    O, h = _oracle_model(blob)
    try:
        p = prompt[:-1].copy()
        m.prefill(p)
        O.orc_model_prefill(h, ptr(p), p.size)
        for layer in range(m.n_layers):
            cs, ss, pos = m.layer_state(layer)
            ocs = np.empty((3, m.d_inner), np.float32)
            oss = np.empty(m.d_inner, np.float32)
            assert pos == O.orc_model_layer_state(h, layer, ptr(ocs), ptr(oss))
            same_bits(cs, ocs, "conv_state[%d]" % layer)
            same_bits(ss, oss, "ssm_state[%d]" % layer)
        harr = np.array(prompt[-256:], np.int32)
        a = m.step(int(prompt[-1]), harr, 1.0)
        b = O.orc_model_step(h, int(prompt[-1]), ptr(harr), harr.size, 1.0)
        same_bits(m.logits(), np.ctypeslib.as_array(O.orc_model_logits(h), (m.vocab,)), "logits")
        assert a == b
    finally:
        O.orc_model_free(h)
        m.free()


def test_prefill_lengths_vs_oracle(hip):
    """Prefill in one call and in several (the conv ring and the state carry
    over), with 1 to 2050 tokens (several 1024-token chunks of the
    three-phase SSM, counts that are not whole 4-token quads): every layer's
    state and the next step's logits bit-exact against the oracle's
    token-serial prefill."""
    g = gold("tiny")
    blob, _, _ = model_image(g)
    c = g["config"]
    m = bh.Model(blob)
    O, h = _oracle_model(blob)
    try:
        for parts in ([1], [2], [3], [5], [12], [16], [300], [600], [100, 200], [1, 2, 257],
                      [1025], [2050], [7, 1030]):
            note("prefill parts %s" % parts)
            m.reset()
            O.orc_model_free(h)
            h = O.orc_model_load(ptr(blob), blob.nbytes)
            toks = bh.synth_prompt(sum(parts) + 11, c["vocab"], sum(parts) + 1)
            at = 0
            for n in parts:
                p = toks[at:at + n].copy()
                m.prefill(p)
                O.orc_model_prefill(h, ptr(p), p.size)
                at += n
            for layer in range(m.n_layers):
                cs, ss, pos = m.layer_state(layer)
                ocs = np.empty((3, m.d_inner), np.float32)
                oss = np.empty(m.d_inner, np.float32)
                assert pos == O.orc_model_layer_state(h, layer, ptr(ocs), ptr(oss))
                same_bits(cs, ocs, "conv_state[%d]" % layer)
                same_bits(ss, oss, "ssm_state[%d]" % layer)
            harr = np.array(toks[-256:], np.int32)
            a = m.step(int(toks[-1]), harr, 1.0)
            b = O.orc_model_step(h, int(toks[-1]), ptr(harr), harr.size, 1.0)
            same_bits(m.logits(), np.ctypeslib.as_array(O.orc_model_logits(h), (m.vocab,)),
                      "logits after prefill %s" % parts)
            assert a == b
    finally:
        O.orc_model_free(h)
        m.free()


def test_generate_stops_at_end_token(hip):
    """generate with stop_on_eos against the reference's loop, which stops
    stepping at the end token (src/main.c:473-500): the returned tokens end
    with it, and the recurrent state, ring position and logits are those of
    the step that picked it, although the device replayed the step graph for
    all n_steps.  A device-resident continuation (decode) then goes on from
    the end token as the reference would.  Model: vocabulary 64, d_model
    128, 2 layers, 4 heads (seed 3), whose greedy stream picks token 0, an
    end token, at step 8."""
    blob = bh.synth_model(64, 128, 2, 4, 3, bh.SYNTH_UNIFORM)
    prompt = bh.synth_prompt(3, 64, 6)
    note("generate stop_on_eos, vocab 64 d_model 128")
    O, h = _oracle_model(blob)
    m = bh.Model(blob)
    try:
        toks, _ = m.generate(prompt, 24, stop_on_eos=True)
        p = np.ascontiguousarray(prompt[:-1], np.int32)
        O.orc_model_prefill(h, ptr(p), p.size)
        hist, cur, ref = [int(t) for t in prompt], int(prompt[-1]), []
        while len(ref) < 24:
            harr = np.array(hist[-256:], np.int32)
            cur = O.orc_model_step(h, cur, ptr(harr), harr.size, 1.0)
            ref.append(cur)
            hist.append(cur)
            if cur in (0, 50256):
                break
        assert ref[-1] == 0 and len(ref) == 9, ref
        assert toks.tolist() == ref
        for layer in range(m.n_layers):
            cs, ss, pos = m.layer_state(layer)
            ocs = np.empty((3, m.d_inner), np.float32)
            oss = np.empty(m.d_inner, np.float32)
            assert pos == O.orc_model_layer_state(h, layer, ptr(ocs), ptr(oss))
            same_bits(cs, ocs, "conv_state[%d]" % layer)
            same_bits(ss, oss, "ssm_state[%d]" % layer)
        same_bits(m.logits(), np.ctypeslib.as_array(O.orc_model_logits(h), (m.vocab,)),
                  "logits of the end token's step")
        m.decode(4)
        cont = []
        for _ in range(4):
            harr = np.array(hist[-256:], np.int32)
            cur = O.orc_model_step(h, cur, ptr(harr), harr.size, 1.0)
            cont.append(cur)
            hist.append(cur)
        assert m.tokens(4).tolist() == cont
        same_bits(m.logits(), np.ctypeslib.as_array(O.orc_model_logits(h), (m.vocab,)),
                  "logits after the continuation")
    finally:
        O.orc_model_free(h)
        m.free()


def test_tiny_generate_matches_reference(hip):
    g = gold("tiny")
    blob, prompt, steps = model_image(g)
    m = bh.Model(blob)
    toks, ms = m.generate(prompt, steps)
    m.free()
    assert toks.tolist() == g["tokens"]


def _stream_check(hip, name):
    g = gold(name)
    note("%s-shape generation (%d steps)" % (name, g["config"]["steps"]))
    blob, prompt, steps = model_image(g)
    import hashlib
    assert hashlib.sha256(blob).hexdigest() == g["blob_sha256"]
    m = bh.Model(blob)
    del blob
    toks, ms = m.generate(prompt, steps)
    m.free()
    ref = g["tokens"]
    if toks.tolist() != ref:
        first = next(i for i, (a, b) in enumerate(zip(toks.tolist(), ref)) if a != b)
        raise AssertionError("%s: first divergence at step %d (ref top-2 margin %.3g)"
                             % (name, first, g["top2_margin"][first]))
    print("[%s] %d tokens identical, %.1f tok/s" % (name, steps, steps / (ms / 1e3)))


def test_255m_stream_matches_reference(hip):
    _stream_check(hip, "255m")


def test_1b_stream_matches_reference(hip):
    _stream_check(hip, "1b")


def _sample_fixture():
    with open(os.path.join(GOLD, "stream_sample.json")) as f:
        g = json.load(f)
    c = g["config"]
    blob = bh.synth_model(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["seed"],
                          c["dist"])
    assert blob.nbytes == g["blob_bytes"]
    return g, blob, np.array(g["prompt"], np.int32), c["steps"]


def test_sampled_streams_match_reference(hip):
    """Device sampler (every branch of sample_advanced, the repetition
    penalty, greedy below temp 0.05) against the reference's own sampled
    streams (tests/golden/stream_sample.json), each case from a reset model
    and a freshly seeded generator, as one captured graph per step."""
    g, blob, prompt, steps = _sample_fixture()
    m = bh.Model(blob)
    try:
        for s in g["streams"]:
            note("sampled stream temp=%g min_p=%g top_p=%g top_k=%d penalty=%g seed=%d"
                 % (s["temp"], s["min_p"], s["top_p"], s["top_k"], s["penalty"], s["seed"]))
            m.reset()
            m.set_sampler(s["temp"], s["min_p"], s["top_p"], s["top_k"])
            m.seed(s["seed"])
            toks, _ = m.generate(prompt, steps, s["penalty"])
            assert [int(t) for t in toks] == s["tokens"], s
    finally:
        m.free()


def test_sampled_steps_logits_vs_oracle(hip):
    """bm_hip_model_step with the sampler: each step's token and its logits
    (penalty applied, divided by the temperature in place as the reference
    leaves them) bit-exact against the oracle model + orc_sample."""
    g, blob, prompt, steps = _sample_fixture()
    O, h = _oracle_model(blob)
    m = bh.Model(blob)
    try:
        for s in (g["streams"][2], g["streams"][4]):
            note("sampled steps temp=%g top_k=%d penalty=%g" % (s["temp"], s["top_k"],
                                                                s["penalty"]))
            m.reset()
            O.orc_model_free(h)
            h = O.orc_model_load(ptr(blob), blob.nbytes)
            p = prompt[:-1].copy()
            m.prefill(p)
            O.orc_model_prefill(h, ptr(p), p.size)
            m.set_sampler(s["temp"], s["min_p"], s["top_p"], s["top_k"])
            m.seed(s["seed"])
            rng = native.C.c_uint64(s["seed"])
            V = O.orc_model_config(h, 0)
            hist, cur = [int(t) for t in prompt], int(prompt[-1])
            for i in range(8):
                harr = np.array(hist[-256:], np.int32)
                t_dev = m.step(cur, harr, s["penalty"])
                O.orc_model_step(h, cur, ptr(harr), harr.size, s["penalty"])
                lg = np.ctypeslib.as_array(O.orc_model_logits(h), (V,)).copy()
                t_orc = O.orc_sample(ptr(lg), V, s["temp"], s["min_p"], s["top_p"], s["top_k"],
                                     native.C.byref(rng))
                assert t_dev == t_orc == s["tokens"][i], (i, s)
                same_bits(m.logits(), lg, "scaled logits")
                hist.append(t_dev)
                cur = t_dev
    finally:
        m.free()
        O.orc_model_free(h)


def _bmst(layers, pos, d_inner):
    """A BMST image as src/chat.c:1160-1207 writes it: magic, n_layers,
    d_inner, d_conv, then per layer conv_state, ssm_state, conv_pos."""
    parts = [np.array([0x424D5354, len(layers), d_inner, 4], np.uint32).tobytes()]
    for cs, ss in layers:
        parts += [np.ascontiguousarray(cs, np.float32).tobytes(),
                  np.ascontiguousarray(ss, np.float32).tobytes(), np.int32(pos).tobytes()]
    return b"".join(parts)


def test_state_save_load(hip):
    """BMST images: the device's saved state equals the image built from the
    oracle's state after the same tokens; a device model loaded from the
    oracle's image continues with bit-exact logits; bad images are rejected
    with the reference's outcome (untouched on a bad magic or dimensions,
    reset on a truncated image or a bad ring position)."""
    g = gold("tiny")
    blob, prompt, _ = model_image(g)
    note("BMST save/load")
    O, h = _oracle_model(blob)
    m = bh.Model(blob)
    m2 = bh.Model(blob)
    try:
        p = prompt[:-1].copy()
        m.prefill(p)
        O.orc_model_prefill(h, ptr(p), p.size)
        hist, cur = [int(t) for t in prompt], int(prompt[-1])
        for _ in range(5):
            harr = np.array(hist[-256:], np.int32)
            cur = m.step(cur, harr)
            assert cur == O.orc_model_step(h, hist[-1], ptr(harr), harr.size, 1.0)
            hist.append(cur)
        nl, di = m.n_layers, m.d_inner
        layers, pos = [], None
        for layer in range(nl):
            cs = np.empty((3, di), np.float32)
            ss = np.empty(di, np.float32)
            pos = O.orc_model_layer_state(h, layer, ptr(cs), ptr(ss))
            layers.append((cs, ss))
        image = _bmst(layers, pos, di)
        assert m.state_save() == image
        # a fresh model continues from the oracle's image
        assert m2.state_load(image)
        for _ in range(4):
            harr = np.array(hist[-256:], np.int32)
            t2 = m2.step(cur, harr)
            t_o = O.orc_model_step(h, cur, ptr(harr), harr.size, 1.0)
            V = O.orc_model_config(h, 0)
            same_bits(m2.logits(), np.ctypeslib.as_array(O.orc_model_logits(h), (V,)), "logits")
            assert t2 == t_o
            hist.append(t2)
            cur = t2
        saved = m2.state_save()
        zero = _bmst([(np.zeros((3, di)), np.zeros(di))] * nl, 0, di)
        bad_magic = b"XXXX" + saved[4:]
        bad_dims = np.array([0x424D5354, nl + 1, di, 4], np.uint32).tobytes() + saved[16:]
        bad_pos = _bmst(layers, 3, di)
        for img, outcome in ((bad_magic, saved), (bad_dims, saved), (saved[:-5], zero),
                             (bad_pos, zero)):
            assert m2.state_load(saved)
            assert not m2.state_load(img)
            assert m2.state_save() == outcome
    finally:
        m.free()
        m2.free()
        O.orc_model_free(h)
