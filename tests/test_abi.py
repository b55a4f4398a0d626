"""CPU-side checks of the product library: it loads, exports every entry
point include/bm_hip.h declares (and the binding knows them all), and the
synthetic generator is bit-reproducible (its bytes match the SHA-256 the
golden fixtures recorded when the reference produced its streams)."""
import json
import os
import re

import numpy as np

import native
from native import bh

ROOT = native.ROOT


def header_functions():
    src = open(os.path.join(ROOT, "include", "bm_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"\b([a-z_][a-z0-9_]*)\s*\(", src)
    skip = {"if", "for", "while", "sizeof", "return"}
    return sorted(set(n for n in names if n not in skip and (n.startswith("bm_") or
                                                            n.startswith("hip_"))))


def test_exports_every_declared_symbol():
    L = bh.lib()
    names = header_functions()
    assert len(names) >= 25
    for n in names:
        assert hasattr(L, n), n
        assert n in bh.SIGNATURES, "binding misses " + n


def test_synthetic_generator_reproducible():
    gold = json.load(open(os.path.join(ROOT, "tests", "golden", "stream_tiny.json")))
    c = gold["config"]
    blob = bh.synth_model(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["seed"],
                          c["dist"])
    import hashlib
    assert blob.nbytes == gold["blob_bytes"]
    assert hashlib.sha256(blob).hexdigest() == gold["blob_sha256"]
    assert list(bh.synth_prompt(c["seed"], c["vocab"], c["prompt"])) == gold["prompt"]


def test_synthetic_distributions():
    p = bh.synth_ternary(3, 1, 200, 1024, bh.SYNTH_P0_40)
    w = native.decode_dense(p, 1024)
    frac0 = np.mean(w == 0)
    assert abs(frac0 - 0.4) < 0.01 and abs(np.mean(w == 1) - 0.3) < 0.01
    assert not np.any(((p >> 0) & 3) == 3)
    x = bh.synth_normal(3, 2, (256, 1024), 1.0)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    q = bh.synth_int8(3, 4, (64, 1024))
    assert q.min() >= -127 and q.max() <= 127


def test_synth_image_size_matches_bit2_layout():
    # the synthetic writer's image size against the BIT2 record layout
    # (src/model.c:367-475: float records type, ndim, dims, data; ternary
    # records type, rows, cols, scale, packed bytes)
    blob = bh.synth_model(1000, 128, 2, 4, 5)
    dm, di, nh, V = 128, 256, 4, 1000
    fl = lambda nd, n: 8 + 4 * nd + 4 * n
    tern = lambda r, c: 16 + r * ((c + 3) // 4)
    layer = (fl(1, dm) + tern(2 * di + 3 * nh, dm) + fl(2, di * 4) + fl(1, di) + 2 * fl(1, nh)
             + 2 * fl(1, di) + tern(dm, di))
    assert blob.nbytes == 20 + fl(2, V * dm) + 2 * layer + 2 * fl(1, dm) + tern(V, dm)


def test_batch_context_null_handling():
    """The batch context's entry points (src/metal/bm_metal.h:57-99) on a
    NULL context do nothing and refuse, and bm_hip_batch_begin returns NULL
    while the backend is not initialized (no GPU here), as Metal's does
    before bm_metal_init; none of these calls touches the GPU."""
    L = bh.lib()
    assert L.bm_hip_batch_ptr(None, 0) is None
    assert not L.bm_hip_encode_bitlinear(None, 0, 64, None, 8, 64, 1.0, None, 1)
    L.bm_hip_encode_residual(None, 16)
    L.bm_hip_submit_and_wait(None)
    L.bm_hip_batch_end(None)
    if not L.bm_hip_available():
        assert L.bm_hip_batch_begin(4, 64, 128, 128, 160) is None
        assert "not initialized" in bh.last_error()
