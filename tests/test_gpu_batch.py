"""The batch context: the Metal backend's prefill batching
(src/metal/bm_metal.h:57-99, src/metal/bm_metal.c:610-960) on this library,
bm_hip_batch_begin / _ptr / bm_hip_encode_bitlinear / _residual /
bm_hip_submit_and_wait / bm_hip_batch_end.

Bars:
  - the reference's own model, prefilled in model_prefill_metal's order
    (src/model.c:934-1041; oracle/ref_harness.c bmref_model_prefill_batch:
    BitLinears and residual adds on the GPU, block_ssm_scan on the CPU),
    ends in exactly the recurrent state of the reference's CPU model_prefill
    (scalar kernels, one thread) on the same tokens;
  - one encoded BitLinear equals the oracle's scalar_bitlinear_forward_batch
    bit for bit, steps chained in one submit see each other's results, and
    only the regions the steps write change;
  - the calls Metal refuses are refused (bad ids, cols % 16 != 0, tensors
    outside the registered image), and so are dimensions that would run past
    the buffers.
"""
import ctypes as C
import json
import os
import tempfile

import numpy as np
import pytest

import native
from native import bh, ptr

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
X, PROJ, Y, OUT = 0, 1, 2, 3

pytestmark = pytest.mark.gpu


class BatchApi(C.Structure):
    """bmref_batch_api_t (oracle/ref_harness.c): the six entry points."""
    _fields_ = [(n, C.c_void_p) for n in ("begin", "ptr", "encode_bitlinear",
                                          "encode_residual", "submit_and_wait", "end")]


def api_of(hip):
    return BatchApi(*[C.cast(getattr(hip, "bm_hip_" + n), C.c_void_p).value
                      for n in ("batch_begin", "batch_ptr", "encode_bitlinear",
                                "encode_residual", "submit_and_wait", "batch_end")])


def host_view(hip, ctx, buf, n):
    addr = hip.bm_hip_batch_ptr(ctx, buf)
    assert addr, "batch_ptr returned NULL for buffer %d" % buf
    return np.ctypeslib.as_array((C.c_float * n).from_address(addr))


def layer_states(R, h, n_layers, d_inner):
    cs = np.empty(3 * d_inner, np.float32)
    ss = np.empty(d_inner, np.float32)
    out = []
    for layer in range(n_layers):
        pos = R.bmref_model_layer_state(h, layer, ptr(cs), ptr(ss))
        out.append((pos, cs.view(np.uint32).copy(), ss.view(np.uint32).copy()))
    return out


@pytest.mark.skipif(not native.ref_available(),
                    reason="oracle/_ref not built (reference sources absent)")
@pytest.mark.parametrize("shape,n", [("tiny", 37), ("255m", 16)])
def test_reference_prefill_through_batch_context(hip, shape, n):
    c = json.load(open(os.path.join(GOLD, "stream_%s.json" % shape)))["config"]
    blob = bh.synth_model(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["seed"],
                          c["dist"])
    tokens = np.ascontiguousarray(bh.synth_prompt(c["seed"] + 7, c["vocab"], n), np.int32)
    d_inner = 2 * c["d_model"]
    R = native.ref()
    api = api_of(hip)
    with tempfile.NamedTemporaryFile(suffix=".bin") as f:
        blob.tofile(f.name)
        del blob
        R.bmref_init(1, 0)  # scalar kernels, one thread: the sequential SSM scan
        ha = R.bmref_model_load(f.name.encode())
        hb = R.bmref_model_load(f.name.encode())
        assert ha and hb, "reference model_load rejected the image"
        try:
            addr, size = C.c_void_p(), C.c_size_t()
            assert R.bmref_model_image(ha, C.byref(addr), C.byref(size))
            assert hip.bm_hip_set_mmap(addr, size.value), bh.last_error()
            print("[case] batch-context prefill, %s shape, %d tokens" % (shape, n), flush=True)
            assert R.bmref_model_prefill_batch(ha, ptr(tokens), n, C.byref(api)) == 0, \
                bh.last_error()
            R.bmref_model_prefill(hb, ptr(tokens), n)
            got = layer_states(R, ha, c["n_layers"], d_inner)
            want = layer_states(R, hb, c["n_layers"], d_inner)
            for layer, ((pa, ca, sa), (pb, cb, sb)) in enumerate(zip(got, want)):
                assert pa == pb, "layer %d conv_pos" % layer
                np.testing.assert_array_equal(ca, cb, err_msg="layer %d conv_state" % layer)
                np.testing.assert_array_equal(sa, sb, err_msg="layer %d ssm_state" % layer)
        finally:
            R.bmref_model_free(ha)
            R.bmref_model_free(hb)
            R.bmref_init(4, 0)
            hip.bm_hip_cleanup()
            assert hip.bm_hip_init()


def _image(r, tensors):
    """One uint8 buffer holding the given arrays at 256-byte aligned offsets
    (registered as the model image); returns the buffer and the addresses."""
    offs, total = [], 0
    for a in tensors:
        offs.append(total)
        total += (a.nbytes + 255) // 256 * 256
    img = np.zeros(total + 256, np.uint8)
    for a, o in zip(tensors, offs):
        img[o:o + a.nbytes] = np.frombuffer(a.tobytes(), np.uint8)
    base = img.ctypes.data
    return img, [base + o for o in offs]


def test_batch_context_steps(hip):
    r = np.random.default_rng(41)
    T, d_model, d_inner, max_proj = 5, 256, 512, 384
    w_in = r.integers(0, 256, (300, d_model // 4), dtype=np.uint8)    # X -> PROJ, 300 rows
    w_out = r.integers(0, 256, (d_model, d_inner // 4), dtype=np.uint8)  # Y -> OUT
    g_in = (1.0 + 0.1 * r.standard_normal(d_model)).astype(np.float32)
    g_out = (1.0 + 0.1 * r.standard_normal(d_inner)).astype(np.float32)
    w_odd = r.integers(0, 256, (8, 250 // 4 + 1), dtype=np.uint8)
    img, (a_in, a_out, a_gin, a_gout, a_odd) = _image(r, [w_in, w_out, g_in, g_out, w_odd])
    assert hip.bm_hip_set_mmap(img.ctypes.data, img.nbytes), bh.last_error()
    ctx = hip.bm_hip_batch_begin(T, d_model, max_proj, d_inner, d_inner + 32)
    assert ctx, bh.last_error()
    try:
        x = host_view(hip, ctx, X, T * d_model)
        proj = host_view(hip, ctx, PROJ, T * max_proj)
        y = host_view(hip, ctx, Y, T * d_inner)
        out = host_view(hip, ctx, OUT, T * d_model)
        assert not np.any(proj), "buffers start zeroed"
        assert hip.bm_hip_batch_ptr(ctx, 4) is None and hip.bm_hip_batch_ptr(ctx, -1) is None

        # one BitLinear X -> PROJ; the rest of PROJ keeps what the host wrote
        x[:] = r.standard_normal(T * d_model).astype(np.float32)
        proj[:] = -7.0
        print("[case] batch: one BitLinear X -> PROJ", flush=True)
        assert hip.bm_hip_encode_bitlinear(ctx, X, d_model, a_in, 300, d_model, 0.03, a_gin, PROJ)
        hip.bm_hip_submit_and_wait(ctx)
        want, _, _ = native.orc_bitlinear(x.reshape(T, d_model), w_in, 300, d_model, 0.03, g_in)
        np.testing.assert_array_equal(proj[:T * 300].view(np.uint32),
                                      want.reshape(-1).view(np.uint32))
        assert np.all(proj[T * 300:] == -7.0)

        # out_proj, residual and the next in_proj in one submit (the Metal
        # prefill's per-layer submit)
        y[:] = r.standard_normal(T * d_inner).astype(np.float32)
        x0 = x.copy()
        print("[case] batch: Y -> OUT, X += OUT, X -> PROJ in one submit", flush=True)
        assert hip.bm_hip_encode_bitlinear(ctx, Y, d_inner, a_out, d_model, d_inner, 0.05, a_gout,
                                           OUT)
        hip.bm_hip_encode_residual(ctx, T * d_model)
        assert hip.bm_hip_encode_bitlinear(ctx, X, d_model, a_in, 300, d_model, 0.03, a_gin, PROJ)
        hip.bm_hip_submit_and_wait(ctx)
        o_want, _, _ = native.orc_bitlinear(y.reshape(T, d_inner), w_out, d_model, d_inner, 0.05,
                                            g_out)
        o_want = o_want.reshape(-1)
        np.testing.assert_array_equal(out.view(np.uint32), o_want.view(np.uint32))
        x1 = (x0 + o_want).astype(np.float32)
        np.testing.assert_array_equal(x.view(np.uint32), x1.view(np.uint32))
        p_want, _, _ = native.orc_bitlinear(x1.reshape(T, d_model), w_in, 300, d_model, 0.03, g_in)
        np.testing.assert_array_equal(proj[:T * 300].view(np.uint32),
                                      p_want.reshape(-1).view(np.uint32))

        # a residual over part of X: only that part changes
        x2 = x.copy()
        hip.bm_hip_encode_residual(ctx, 100)
        hip.bm_hip_submit_and_wait(ctx)
        np.testing.assert_array_equal(x[:100], (x2[:100] + out[:100]).astype(np.float32))
        np.testing.assert_array_equal(x[100:], x2[100:])

        # refused, as Metal refuses them, or as running past the buffers
        print("[case] batch: refused steps", flush=True)
        outside = np.zeros_like(w_in)
        assert not hip.bm_hip_encode_bitlinear(ctx, PROJ, d_model, a_in, 300, d_model, 0.03, a_gin,
                                               PROJ)  # source must be X or Y
        assert not hip.bm_hip_encode_bitlinear(ctx, X, d_model, a_in, 300, d_model, 0.03, a_gin,
                                               Y)  # destination must be PROJ or OUT
        assert not hip.bm_hip_encode_bitlinear(ctx, X, 250, a_odd, 8, 250, 0.03, a_gin, PROJ)
        assert not hip.bm_hip_encode_bitlinear(ctx, X, d_model, outside.ctypes.data, 300, d_model,
                                               0.03, a_gin, PROJ)  # outside the image
        assert not hip.bm_hip_encode_bitlinear(ctx, X, d_model, a_in, 400, d_model, 0.03, a_gin,
                                               PROJ)  # 400 rows > max_proj
        assert not hip.bm_hip_encode_bitlinear(ctx, Y, d_inner, a_in, 300, d_model, 0.03, a_gin,
                                               PROJ)  # input_dim != cols
        assert not hip.bm_hip_encode_bitlinear(None, X, d_model, a_in, 300, d_model, 0.03, a_gin,
                                               PROJ)
        # nothing was queued by the refused calls: a submit changes nothing
        before = [v.copy() for v in (x, proj, y, out)]
        hip.bm_hip_submit_and_wait(ctx)
        for v, b in zip((x, proj, y, out), before):
            np.testing.assert_array_equal(v, b)
    finally:
        hip.bm_hip_batch_end(ctx)
        hip.bm_hip_cleanup()
        assert hip.bm_hip_init()
        del img
