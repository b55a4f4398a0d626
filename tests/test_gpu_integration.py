"""The drop-in as the reference itself drives it: the reference's own
model_load / model_prefill / model_forward_step / block_step, compiled from
its sources into oracle/_ref, with its plugin table handed to this library's
bm_hip_register after bm_hip_set_mmap registered the model file the
reference mapped (the wiring of src/dispatch.c:15-52 and src/model.c:840-851
under HAS_HIP).  Every BitLinear and RMSNorm of the decode then runs through
hip_bitlinear_forward / hip_bitlinear_forward_batch / hip_rms_norm, and the
SSM step stays on the CPU (scalar ssm_inner).

Bar: the 255M-shape greedy stream (128 steps) gives the scalar reference's
tokens, and every step's logits hash to the same SHA-256 as in the golden
record written by the scalar build (tests/golden/stream_255m.json).
"""
import ctypes as C
import json
import os
import tempfile
import time

import numpy as np
import pytest

import native
from native import bh, ptr
from golden.make_golden import sha

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not native.ref_available(),
                                 reason="oracle/_ref not built (reference sources absent)")]


def test_reference_decode_through_hip_table(hip):
    gold = json.load(open(os.path.join(GOLD, "stream_255m.json")))
    c = gold["config"]
    blob = bh.synth_model(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["seed"],
                          c["dist"])
    assert sha(blob) == gold["blob_sha256"]
    prompt = bh.synth_prompt(c["seed"], c["vocab"], c["prompt"])
    assert [int(t) for t in prompt] == gold["prompt"]
    R = native.ref()
    V = c["vocab"]
    with tempfile.NamedTemporaryFile(suffix=".bin") as f:
        blob.tofile(f.name)
        del blob
        R.bmref_init(4, 0)  # CPU slots the table keeps: the scalar kernels
        h = R.bmref_model_load(f.name.encode())
        assert h, "reference model_load rejected the image"
        try:
            addr, size = C.c_void_p(), C.c_size_t()
            assert R.bmref_model_image(h, C.byref(addr), C.byref(size))
            assert hip.bm_hip_set_mmap(addr, size.value), bh.last_error()
            assert R.bmref_use_hip(C.cast(hip.bm_hip_register, C.c_void_p)) == 1
            assert R.bmref_kernels_name() == b"hip"
            print("[case] reference decode through the HIP table, 255M shape", flush=True)
            p = np.ascontiguousarray(prompt[:-1], np.int32)
            R.bmref_model_prefill(h, ptr(p), len(p))
            hist, cur = [int(t) for t in prompt], int(prompt[-1])
            toks, bad, dt = [], [], []
            for i in range(c["steps"]):
                harr = np.array(hist[-256:], np.int32)
                t0 = time.perf_counter()
                cur = R.bmref_model_step(h, cur, ptr(harr), len(harr), 1.0)
                dt.append(time.perf_counter() - t0)
                lg = np.ctypeslib.as_array(R.bmref_model_logits(h), (V,)).copy()
                if sha(lg)[:16] != gold["logits_sha256_16"][i]:
                    bad.append(i)
                toks.append(int(cur))
                hist.append(cur)
            print("[info] reference model_forward_step on the HIP table: median %.3f ms per "
                  "token (%.1f tok/s)" % (np.median(dt) * 1e3, 1.0 / np.median(dt)), flush=True)
            assert toks == gold["tokens"]
            assert not bad, "steps whose logits differ from the scalar reference: %s" % bad[:8]
        finally:
            R.bmref_model_free(h)
            R.bmref_init(4, 0)  # the CPU table again for the tests that follow
            hip.bm_hip_cleanup()


def _hook_prefill(R, hip, h, g, tokens, n_layers, di):
    """The prefill hook at the Metal spot of model_prefill
    (src/model.c:1050-1055): push the reference blocks' recurrent state into
    the device model, prefill there, pull the state back."""
    cs = np.empty(3 * di, np.float32)
    ss = np.empty(di, np.float32)
    for layer in range(n_layers):
        pos = R.bmref_model_layer_state(h, layer, ptr(cs), ptr(ss))
        assert hip.bm_hip_model_set_layer_state(g, layer, ptr(cs), ptr(ss), pos) == 0
    t = np.ascontiguousarray(tokens, np.int32)
    assert hip.bm_hip_model_prefill(g, ptr(t), t.size) == 0, bh.last_error()
    for layer in range(n_layers):
        pos = hip.bm_hip_model_layer_state(g, layer, ptr(cs), ptr(ss))
        R.bmref_model_set_layer_state(h, layer, ptr(cs), ptr(ss), pos)


def _session(R, h, prompt, turn2, steps, hook=None):
    """Two turns of a chat-like session on the reference model h: prefill
    the prompt but its last token, `steps` greedy steps, prefill a second
    user turn (carried state), `steps` more; tokens and logits hashes."""
    V = R.bmref_model_vocab(h)
    prefill = hook or (lambda toks: R.bmref_model_prefill(
        h, ptr(np.ascontiguousarray(toks, np.int32)), len(toks)))
    out, hashes = [], []
    hist = [int(t) for t in prompt]
    prefill(prompt[:-1])
    cur = int(prompt[-1])
    for turn in range(2):
        for _ in range(steps):
            harr = np.array(hist[-256:], np.int32)
            cur = R.bmref_model_step(h, cur, ptr(harr), len(harr), 1.0)
            lg = np.ctypeslib.as_array(R.bmref_model_logits(h), (V,)).copy()
            out.append(int(cur))
            hashes.append(sha(lg)[:16])
            hist.append(cur)
        if turn == 0:
            prefill(turn2[:-1])
            hist += [int(t) for t in turn2]
            cur = int(turn2[-1])
    return out, hashes


def test_reference_prefill_hook_two_turns(hip):
    """The reference's own session (model_prefill, model_forward_step, a
    second prefill on the carried state) with every prefill replaced by the
    device prefill through the state hook and every BitLinear on the HIP
    table, against the same session on the reference's scalar CPU kernels."""
    c = dict(vocab=5000, d_model=1024, n_layers=4, n_heads=32, dist=0, seed=77)
    blob = bh.synth_model(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["seed"],
                          c["dist"])
    prompt = bh.synth_prompt(c["seed"], c["vocab"], 40)
    turn2 = bh.synth_prompt(c["seed"] + 1, c["vocab"], 33)
    R = native.ref()
    di = 2 * c["d_model"]
    with tempfile.NamedTemporaryFile(suffix=".bin") as f:
        blob.tofile(f.name)
        R.bmref_init(4, 0)
        h = R.bmref_model_load(f.name.encode())
        assert h
        try:
            ref_toks, ref_hash = _session(R, h, prompt, turn2, 24)
        finally:
            R.bmref_model_free(h)
        h = R.bmref_model_load(f.name.encode())
        assert h
        g = None
        try:
            addr, size = C.c_void_p(), C.c_size_t()
            assert R.bmref_model_image(h, C.byref(addr), C.byref(size))
            assert hip.bm_hip_set_mmap(addr, size.value), bh.last_error()
            assert R.bmref_use_hip(C.cast(hip.bm_hip_register, C.c_void_p)) == 1
            g = hip.bm_hip_model_load(addr, size.value)
            assert g, bh.last_error()
            print("[case] reference session with the prefill hook, 2 turns", flush=True)
            toks, hashes = _session(R, h, prompt, turn2, 24,
                                    hook=lambda t: _hook_prefill(R, hip, h, g, t,
                                                                 c["n_layers"], di))
        finally:
            if g:
                hip.bm_hip_model_free(g)
            R.bmref_model_free(h)
            R.bmref_init(4, 0)
            hip.bm_hip_cleanup()
    assert toks == ref_toks
    assert hashes == ref_hash
