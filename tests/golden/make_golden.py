"""Writes the golden fixtures under tests/golden/ from the reference's own C
sources (oracle/_ref/libbmref.so, scalar kernels forced, as
src/kernel.c computes them).  Run in a container that has the reference
sources built:  python tests/golden/make_golden.py [--skip-1b]

Fixtures are data only: inputs (or the seeds that regenerate them through
the deterministic synthetic generator, with a SHA-256 of the bytes) and the
reference's outputs.
"""
import argparse
import hashlib
import json
import os
import sys
import tempfile
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import native  # noqa: E402
from native import bh, ptr  # noqa: E402

# synthetic workloads (shared with bench.py and the GPU tests)
CFG1 = dict(K=1024, N=4384, seed=1, scale=0.02)          # single GEMV
E2E = {
    "tiny": dict(vocab=1000, d_model=128, n_layers=2, n_heads=4, dist=0, seed=5,
                 prompt=8, steps=24),
    "255m": dict(vocab=50257, d_model=1024, n_layers=24, n_heads=32, dist=0, seed=255,
                 prompt=8, steps=128),
    "1b": dict(vocab=50257, d_model=2048, n_layers=24, n_heads=64, dist=1, seed=1000,
               prompt=8, steps=256),
}


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).view(np.uint8)).hexdigest()


def cfg1_inputs():
    K, N, seed = CFG1["K"], CFG1["N"], CFG1["seed"]
    packed = bh.synth_ternary(seed, 1, N, K, bh.SYNTH_UNIFORM)
    x = bh.synth_normal(seed, 2, (1, K), 1.0)
    gamma = np.ones(K, np.float32)
    return packed, x, gamma


def make_quant(R):
    out = {}
    for n in (1024, 4096, 4099, 100):
        r = np.random.default_rng(n)
        x = (r.standard_normal((3, n)) * np.array([[1.0], [1e-3], [1.0]])).astype(np.float32)
        x[2, r.integers(0, n, 8)] *= 10.0
        g = (r.standard_normal(n) * 0.02).astype(np.float32)
        xn = np.empty((3, n), np.float32)
        mx = np.empty(3, np.float32)
        for m in range(3):
            row = np.ascontiguousarray(x[m])
            o = np.empty(n, np.float32)
            mx[m] = R.bmref_rms_norm(ptr(row), n, ptr(g), ptr(o))
            xn[m] = o
        # the int8 vector as scalar_bitlinear_forward leaves it
        packed = np.zeros((1, (n + 3) // 4), np.uint8)
        _, _, xq = native.ref_bitlinear(x, packed, 1, n, 1.0, g)
        out.update({"x_%d" % n: x, "g_%d" % n: g, "xn_%d" % n: xn, "max_%d" % n: mx,
                    "xq_%d" % n: xq})
    np.savez_compressed(os.path.join(HERE, "quant_vectors.npz"), **out)


def make_bitlinear(R):
    packed, x, gamma = cfg1_inputs()
    o, xn, xq = native.ref_bitlinear(x, packed, CFG1["N"], CFG1["K"], CFG1["scale"], gamma)
    np.savez_compressed(os.path.join(HERE, "bitlinear_k1024_n4384.npz"), out=o, x_norm=xn,
                        x_quant=xq, packed_sha256=np.array(sha(packed)),
                        x_sha256=np.array(sha(x)))
    # odd shapes with every 2-bit code (11 included) and K % 4 != 0
    out = {}
    for K, N in ((1026, 11), (64, 7), (2048, 9), (1000, 5), (4096, 5)):
        r = np.random.default_rng(K * 7 + N)
        p = r.integers(0, 256, (N, (K + 3) // 4), dtype=np.uint8)
        xx = r.standard_normal((3, K)).astype(np.float32)
        g = r.standard_normal(K).astype(np.float32)
        o, xn, xq = native.ref_bitlinear(xx, p, N, K, 0.037, g)
        key = "%d_%d" % (K, N)
        out.update({"packed_" + key: p, "x_" + key: xx, "g_" + key: g, "out_" + key: o,
                    "xq_" + key: xq})
    np.savez_compressed(os.path.join(HERE, "bitlinear_shapes.npz"), **out)


def make_stream(R, name, threads):
    c = E2E[name]
    t0 = time.time()
    blob = bh.synth_model(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["seed"],
                          c["dist"])
    prompt = bh.synth_prompt(c["seed"], c["vocab"], c["prompt"])
    with tempfile.NamedTemporaryFile(suffix=".bin", dir="/tmp") as f:
        blob.tofile(f.name)
        R.bmref_init(threads, 0)
        h = R.bmref_model_load(f.name.encode())
        assert h, "reference model_load rejected the synthetic image"
        p = np.ascontiguousarray(prompt[:-1], np.int32)
        R.bmref_model_prefill(h, ptr(p), len(p))
        hist = [int(t) for t in prompt]
        cur = int(prompt[-1])
        V = c["vocab"]
        toks, margins, lsha = [], [], []
        for _ in range(c["steps"]):
            harr = np.array(hist[-256:], np.int32)
            cur = R.bmref_model_step(h, cur, ptr(harr), len(harr), 1.0)
            lg = np.ctypeslib.as_array(R.bmref_model_logits(h), (V,)).copy()
            top = np.sort(lg)[-2:]
            toks.append(int(cur))
            margins.append(float(top[1] - top[0]))
            lsha.append(sha(lg)[:16])
            hist.append(cur)
        R.bmref_model_free(h)
    rec = dict(config=c, blob_bytes=int(blob.nbytes), blob_sha256=sha(blob),
               prompt=[int(t) for t in prompt], tokens=toks, top2_margin=margins,
               logits_sha256_16=lsha, stop_token_seen=any(t in (0, 50256) for t in toks),
               generator="reference scalar kernels (oracle/_ref, %d threads)" % threads,
               seconds=round(time.time() - t0, 1))
    with open(os.path.join(HERE, "stream_%s.json" % name), "w") as f:
        json.dump(rec, f, indent=1)
    print(name, "done in %.1fs" % (time.time() - t0), toks[:16])


# sampled decoding: (temp, min_p, top_p, top_k, penalty, seed), each branch
# of sample_advanced (src/model.c:132-361) on this model's logits
SAMPLE = dict(model=dict(vocab=5000, d_model=128, n_layers=2, n_heads=4, dist=0, seed=21,
                         prompt=8, steps=24),
              cases=[(0.8, 0.05, 0.9, 40, 1.0, 42), (1.0, 0.0, 1.0, 40, 1.0, 7),
                     (1.2, 0.0, 0.95, 256, 1.3, 9), (0.7, 0.0, 0.9, 0, 1.0, 11),
                     (10.0, 0.0, 0.99, 0, 1.0, 13), (1.0, 0.1, 1.0, 0, 1.0, 17),
                     (10.0, 0.0, 1.0, 300, 1.0, 19), (1.0, 1.0, 1.0, 0, 1.0, 23),
                     (0.9, 0.0, 1.0, 1, 1.0, 29), (0.01, 0.0, 1.0, 0, 1.0, 31)])


def make_sample_streams(R, threads):
    c = SAMPLE["model"]
    t0 = time.time()
    blob = bh.synth_model(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["seed"],
                          c["dist"])
    prompt = bh.synth_prompt(c["seed"], c["vocab"], c["prompt"])
    streams = []
    with tempfile.NamedTemporaryFile(suffix=".bin", dir="/tmp") as f:
        blob.tofile(f.name)
        R.bmref_init(threads, 0)
        for case in SAMPLE["cases"]:
            temp, min_p, top_p, top_k, penalty, seed = case
            h = R.bmref_model_load(f.name.encode())
            assert h, "reference model_load rejected the synthetic image"
            p = np.ascontiguousarray(prompt[:-1], np.int32)
            R.bmref_model_prefill(h, ptr(p), len(p))
            R.bmref_rng_seed(seed)
            hist, cur, toks = [int(t) for t in prompt], int(prompt[-1]), []
            for _ in range(c["steps"]):
                harr = np.array(hist[-256:], np.int32)
                cur = R.bmref_model_step_sample(h, cur, ptr(harr), len(harr), penalty, temp,
                                                min_p, top_p, top_k)
                toks.append(int(cur))
                hist.append(cur)
            R.bmref_model_free(h)
            streams.append(dict(temp=temp, min_p=min_p, top_p=top_p, top_k=top_k,
                                penalty=penalty, seed=seed, tokens=toks))
    rec = dict(config=c, blob_bytes=int(blob.nbytes), blob_sha256=sha(blob),
               prompt=[int(t) for t in prompt], streams=streams,
               generator="reference scalar kernels + sample_advanced (oracle/_ref, %d threads)"
                         % threads,
               seconds=round(time.time() - t0, 1))
    with open(os.path.join(HERE, "stream_sample.json"), "w") as f:
        json.dump(rec, f, indent=1)
    print("sample streams done in %.1fs" % (time.time() - t0))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--skip-1b", action="store_true")
    ap.add_argument("--only-sample", action="store_true")
    ap.add_argument("--threads", type=int, default=8)
    a = ap.parse_args()
    if not native.ref_available():
        sys.exit("oracle/_ref/libbmref.so is not built")
    R = native.ref()
    R.bmref_init(1, 0)
    if not a.only_sample:
        make_quant(R)
        make_bitlinear(R)
        for name in ("tiny", "255m") + (() if a.skip_1b else ("1b",)):
            make_stream(R, name, a.threads)
    make_sample_streams(R, a.threads)
    R.bmref_shutdown()


if __name__ == "__main__":
    main()
