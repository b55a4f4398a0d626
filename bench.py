"""Benchmark of the MI355X BitLinear hot path (one GPU).

Workload (the metric's configuration): synthetic 1B-shape BitMamba-2 greedy
decode, bs=1 -- 24 layers, d_model 2048, d_inner 4096, 64 heads of 64,
in_proj 2048x8384 (the width the reference's loader accepts,
src/model.c:683-701), out_proj 4096x2048, vocab 50257, ternary p(0)=0.4,
fp32 parts N(0, 0.02), 8-token prompt.  A step is one decoded token, run as
one replay of the captured per-token hipGraph with inputs already in HBM.

Prints ONE JSON line.  Legs (all by default):
  decode    W untimed steps, then K timed steps -> tok/s (the value) and
            packed-weight GB/s; then the device prefill of a 1024-token
            prompt on the same model (prefill_1b: time to first token)
  sampled   the same model decoding with the device sampler (temp 0.8,
            min_p 0.05, top_p 0.9, top_k 40): tok/s of up to 128 steps
  fast      opt-in fast mode (sums of squares as a pairwise tree): the same
            greedy decode and 1024-token prefill, its first divergence from
            the reference's stream, the 255M decode, and the quantizer
            against parity at K = 1024, 2048, 4096 (4096 tokens each)
  roofline  the decode GEMV kernel (K=2048 in_proj shape) streaming 512 MiB
            of distinct weight rows in one launch, timed with HIP events on
            the library stream -> achieved GB/s vs 8 TB/s
  prefill   int8-MFMA GEMM at M=2048: 2048->8512 and 4096->2048, TOP/s
  cpu       the reference's own AVX2 build (oracle/_ref) on the host cores,
            at one thread fewer than the box grants (at most 15) and at one thread,
            in a child process before the GPU starts: bounded samples of the
            1B and 255M decodes, the 1024-token 1B prefill, the two M=2048
            prefill products (bitlinear_forward_batch) and the K = N = 8192
            int8 products at M = 1, 16 and 4096 (the row kernel per token);
            each GPU sub-object carries its CPU figures under "cpu"
  gemv1     the single K=1024 -> N=4384 BitLinear (uniform ternary, N(0,1)
            input): device call time (warm, cache-resident), the host-pointer
            drop-in call (PCIe included), and the reference's own CPU build
            (AVX2 with the leg's thread count, scalar on 1 thread)
  d255m     255M-shape greedy decode, 128 steps (tok/s, stream identity)
  stress    int8-input ternary products at K = N = 8192, p(0) = 0.6, exact
            int32 outputs: M = 1, 16 (weight GB/s, warm) and 4096 (TOP/s)
  vendor    the vendor library's dense int8 GEMM (torch._int_mm on hipBLASLt)
            at the prefill and stress shapes: a reference point without the
            ternary decode or the fp32 epilogue
  mfma      the int8 MFMA ceiling: 2 waves per SIMD of back-to-back
            v_mfma_i32_32x32x32_i8, fixed operands and then hashed int8
            activations against codes 0..2 (the GEMM's data; the sustained
            rate depends on the data through the clock under load)
  copy      (on request only) a plain 512 MiB device copy: the calibration
            run for the HBM traffic counters
The roofline's `traffic` (HBM bytes per launch of the GEMV) is read from
profiles/gemv_k2048_traffic.txt, which holds the FETCH_SIZE / WRITE_SIZE
counter runs of this same leg and their copy-kernel calibration.
"""
import argparse
import ctypes as C
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "bitmamba.c_amd"))
import bitmamba_hip as bh  # noqa: E402

METRIC = "packed-weight GB/s + tok/s (1B-shape decode, bs=1); prefill ternary GEMM TOPS"
CFG_1B = dict(vocab=50257, d_model=2048, n_layers=24, n_heads=64, dist=bh.SYNTH_P0_40,
              seed=1000, prompt=8)
CFG_255M = dict(vocab=50257, d_model=1024, n_layers=24, n_heads=32, dist=bh.SYNTH_UNIFORM,
                seed=255, prompt=8, steps=128)
HBM_PEAK_GBPS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_k2048_traffic.txt")
I8_PEAK_TOPS = 5000.0


def packed_bytes_per_token(c):
    dm, di, nh = c["d_model"], 2 * c["d_model"], c["n_heads"]
    pd = 2 * di + 3 * nh
    return c["n_layers"] * (pd * dm // 4 + dm * di // 4) + c["vocab"] * dm // 4


def log(msg):
    print("[bench] " + msg, file=sys.stderr, flush=True)


class Events:
    def __init__(self, L):
        self.L = L
        self.a, self.b = L.bm_hip_event_create(), L.bm_hip_event_create()

    def start(self):
        self.L.bm_hip_event_record(self.a, None)

    def stop_ms(self):
        self.L.bm_hip_event_record(self.b, None)
        return self.L.bm_hip_event_elapsed_ms(self.a, self.b)


SAMPLED = dict(temp=0.8, min_p=0.05, top_p=0.9, top_k=40, seed=42)


def divergence(toks, ref):
    """First step where two greedy streams differ (None if they agree over
    their common length), and the reference record's top-2 margin there."""
    n = min(len(toks), len(ref["tokens"]))
    i = next((k for k in range(n) if int(toks[k]) != ref["tokens"][k]), None)
    return i, (None if i is None else round(ref["top2_margin"][i], 5))


def leg_decode(L, steps, warmup, sampled=False, fast=False):
    c = CFG_1B
    t0 = time.time()
    blob = bh.synth_model(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["seed"],
                          c["dist"])
    prompt = bh.synth_prompt(c["seed"], c["vocab"], c["prompt"])
    log("1B-shape image %.0f MB built in %.1fs" % (blob.nbytes / 1e6, time.time() - t0))
    m = bh.Model(blob)
    del blob
    first, _ = m.generate(prompt, warmup)           # prefill + warmup steps (untimed)
    L.bm_hip_synchronize()
    t0 = time.perf_counter()
    dev_ms = m.decode(steps)                         # K graph replays
    L.bm_hip_synchronize()
    wall = time.perf_counter() - t0
    toks = np.concatenate([first, m.tokens(steps)])
    # the step's kernels one kind at a time, launched back to back on the
    # model's stream between events (the layers in turn, 240 launches, so
    # that each reads weights the previous launches did not, as in a step;
    # the one LM head 200 times): the roofline's live durations
    ktimes = {name: round(m.time_kernel(which, layer, reps), 3) for name, which, layer, reps in
              (("k_inproj_ssm", 0, -1, 240), ("out_proj", 1, -1, 240), ("lm_head", 2, 0, 200))}
    m.reset()
    samp = None
    if sampled:
        # the same model and prompt with the device sampler
        m.reset()
        m.set_sampler(SAMPLED["temp"], SAMPLED["min_p"], SAMPLED["top_p"], SAMPLED["top_k"])
        m.seed(SAMPLED["seed"])
        m.generate(prompt, warmup)
        L.bm_hip_synchronize()
        n = min(steps, 128)
        t1 = time.perf_counter()
        sms = m.decode(n)
        L.bm_hip_synchronize()
        sw = time.perf_counter() - t1
        samp = dict(SAMPLED, steps=n, tok_s=round(n / sw, 2), ms_per_step=round(sw * 1e3 / n, 4),
                    device_ms_per_step=round(sms / n, 4))
    # time to first token: the device prefill of a 1024-token prompt
    m.reset()
    long_prompt = bh.synth_prompt(c["seed"] + 1, c["vocab"], 1024)
    m.prefill(long_prompt)  # sizes the prefill buffers (untimed)
    pf = 1e9
    for _ in range(3):
        m.reset()
        L.bm_hip_synchronize()
        t2 = time.perf_counter()
        m.prefill(long_prompt)
        L.bm_hip_synchronize()
        pf = min(pf, time.perf_counter() - t2)
    prefill = dict(tokens=1024, ms=round(pf * 1e3, 3), tok_s=round(1024 / pf, 1))
    gold_path = os.path.join(ROOT, "tests", "golden", "stream_1b.json")
    gold = json.load(open(gold_path)) if os.path.exists(gold_path) else None
    fres = None
    if fast:
        # fast mode (pairwise-tree sums of squares) on the same model, greedy
        m.reset()
        m.set_sampler()
        m.set_fast(1)
        ffirst, _ = m.generate(prompt, warmup)
        L.bm_hip_synchronize()
        t3 = time.perf_counter()
        fms = m.decode(steps)
        L.bm_hip_synchronize()
        fw = time.perf_counter() - t3
        ftoks = np.concatenate([ffirst, m.tokens(steps)])
        fpf = 1e9
        for _ in range(3):
            m.reset()
            L.bm_hip_synchronize()
            t2 = time.perf_counter()
            m.prefill(long_prompt)
            L.bm_hip_synchronize()
            fpf = min(fpf, time.perf_counter() - t2)
        m.set_fast(0)
        fres = dict(tok_s=round(steps / fw, 2), ms_per_step=round(fw * 1e3 / steps, 4),
                    device_ms_per_step=round(fms / steps, 4), steps=steps,
                    tokens_identical_to_parity=ftoks.tolist() == toks.tolist(),
                    prefill_1024_ms=round(fpf * 1e3, 3))
        if gold:
            i, mg = divergence(ftoks, gold)
            fres.update(first_divergence_from_reference=i, reference_top2_margin_there=mg,
                        compared_steps=min(len(ftoks), len(gold["tokens"])))
    m.free()
    match = None
    if gold:
        ref = gold["tokens"]
        n = min(len(ref), len(toks))
        match = toks[:n].tolist() == ref[:n]
    return wall, dev_ms, match, samp, prefill, fres, ktimes


def leg_d255m(L, fast=False):
    c = CFG_255M
    blob = bh.synth_model(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["seed"],
                          c["dist"])
    prompt = bh.synth_prompt(c["seed"], c["vocab"], c["prompt"])
    m = bh.Model(blob)
    del blob
    m.generate(prompt, 4)                            # warm the step graph
    m.reset()
    toks, ms = m.generate(prompt, c["steps"])        # device time of the decode steps
    fres = None
    gold_path = os.path.join(ROOT, "tests", "golden", "stream_255m.json")
    gold = json.load(open(gold_path)) if os.path.exists(gold_path) else None
    if fast:
        m.set_fast(1)
        m.reset()
        m.generate(prompt, 4)
        m.reset()
        ftoks, fms = m.generate(prompt, c["steps"])
        fres = dict(tok_s=round(c["steps"] / (fms * 1e-3), 1),
                    ms_per_step=round(fms / c["steps"], 4),
                    tokens_identical_to_parity=ftoks.tolist() == toks.tolist())
        if gold:
            i, mg = divergence(ftoks, gold)
            fres.update(first_divergence_from_reference=i, reference_top2_margin_there=mg)
    m.free()
    match = None
    if gold:
        match = toks.tolist() == gold["tokens"]
    bpt = packed_bytes_per_token(c)
    tok_s = c["steps"] / (ms * 1e-3)
    r = dict(tok_s=round(tok_s, 1), ms_per_step=round(ms / c["steps"], 4),
             packed_weight_GBps=round(tok_s * bpt / 1e9, 1), packed_bytes_per_token=bpt,
             tokens_match_reference=match, steps=c["steps"])
    if fres:
        r["fast_mode"] = fres
    return r


def _dropin_run(L, R, native, path, c, threads, kind, hip, tag="255M"):
    """One greedy decode of config c through the reference's own
    model_prefill / model_forward_step, its CPU table of `kind` (0 scalar,
    1 the dispatch_init choice: AVX2) at `threads` pool threads, with the
    BitLinear / RMSNorm entries handed to this library when `hip`."""
    name = R.bmref_init(threads, kind).decode()
    R.bmref_set_poll(100)
    h = R.bmref_model_load(path.encode())
    if not h:
        raise RuntimeError("reference model_load failed")
    try:
        if hip:
            addr, size = C.c_void_p(), C.c_size_t()
            if not R.bmref_model_image(h, C.byref(addr), C.byref(size)):
                raise RuntimeError("reference model not mapped")
            if not L.bm_hip_set_mmap(addr, size.value):
                raise RuntimeError("bm_hip_set_mmap: " + bh.last_error())
            if R.bmref_use_hip(C.cast(L.bm_hip_register, C.c_void_p)) != 1:
                raise RuntimeError("bm_hip_register refused the table")
            name = "%s + hip" % name
        what = "drop-in %s [%s]" % (tag, name)
        beat("%s: model loaded" % what)
        prompt = bh.synth_prompt(c["seed"], c["vocab"], c["prompt"])
        p = np.ascontiguousarray(prompt[:-1], np.int32)
        t0 = time.perf_counter()
        R.bmref_model_prefill(h, native.ptr(p), p.size)
        pf_ms = (time.perf_counter() - t0) * 1e3
        beat("%s: prompt prefilled (%.1f ms)" % (what, pf_ms))
        hist, cur = [int(t) for t in prompt], int(prompt[-1])
        toks, times = [], []
        for _ in range(c["steps"]):
            harr = np.array(hist[-256:], np.int32)
            t0 = time.perf_counter()
            cur = R.bmref_model_step(h, cur, native.ptr(harr), harr.size, 1.0)
            times.append(time.perf_counter() - t0)
            toks.append(int(cur))
            hist.append(cur)
            if len(toks) % 32 == 0:
                beat("%s: step %d %.3f ms" % (what, len(toks), times[-1] * 1e3))
    finally:
        R.bmref_model_free(h)
    t = np.array(times)
    return toks, dict(tok_s=round(len(t) / t.sum(), 1), ms_per_step=round(t.mean() * 1e3, 4),
                      median_ms_per_step=round(float(np.median(t)) * 1e3, 4),
                      prefill_ms=round(pf_ms, 2), kernels=name, threads=threads)


def leg_dropin(L, threads, c, tag, gold_file, calls):
    """The drop-in as a user of the reference runs it: the reference's own
    model_load / model_prefill / model_forward_step (oracle/_ref, built from
    its sources, with its spin-wait thread pool) with its plugin table handed
    to bm_hip_register after bm_hip_set_mmap registered the mapped model
    file (src/dispatch.c:15-52, src/model.c:840-851): every BitLinear (48
    per token plus the LM head) and the final RMSNorm run through this
    library, one launch each, while ssm_inner, the embedding and the sampler
    stay on the CPU.  c["steps"] greedy steps of config c, three runs:
      value: the reference's AVX2 table (its ssm_inner) + this library;
      cpu_same_kernels: the same reference, all on its AVX2 table (its AVX2
        BitLinear differs from its own scalar kernel, which this library
        reproduces, in the last bit of most outputs, so the two streams
        drift apart: first_divergence says where);
      scalar_ssm: the scalar table + this library, whose tokens must be the
        scalar reference's stream (tests/golden/<gold_file>).
    The pool gets one thread fewer than the CPU baseline's: this process's
    main thread also spins (it polls the GPU's completion words), and a
    spin-wait pool that shares its last CPU stalls (see cpu_threads)."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import native
    R = native.ref()
    gold_path = os.path.join(ROOT, "tests", "golden", gold_file)
    gold = json.load(open(gold_path)) if os.path.exists(gold_path) else None
    try:
        with tempfile.TemporaryDirectory(dir=tempfile.gettempdir()) as d:
            path = _ref_model_file(c, d)
            beat("drop-in %s: model file written" % tag)
            toks, r = _dropin_run(L, R, native, path, c, threads, 1, True, tag)
            ctoks, cr = _dropin_run(L, R, native, path, c, threads, 1, False, tag)
            stoks, sr = _dropin_run(L, R, native, path, c, threads, 0, True, tag)
    finally:
        R.bmref_shutdown()
    div = next((i for i, (a, b) in enumerate(zip(toks, ctoks)) if a != b), None)
    r.update(steps=c["steps"],
             tokens_match_cpu_same_kernels=toks == ctoks, first_divergence_from_cpu=div,
             cpu_same_kernels=cr,
             scalar_ssm=dict(sr, tokens_match_reference=(stoks == gold["tokens"][:len(stoks)])
                             if gold else None),
             calls_per_token=calls)
    return r


def leg_dropin_255m(L, threads):
    """leg_dropin at the 255M shape (128 steps)."""
    return leg_dropin(L, threads, CFG_255M, "255M", "stream_255m.json",
                      "48 BitLinear (in_proj 1024->4192, out_proj 2048->1024) + LM head "
                      "1024->50257 + final RMSNorm on the GPU; ssm_inner on the CPU")


def leg_dropin_1b(L, threads):
    """leg_dropin at the 1B shape (64 steps): twice the rows and columns of
    the 255M shape per BitLinear, so the CPU's time per call grows about
    fourfold while the GPU's stays near its launch and bus floor."""
    return leg_dropin(L, threads, dict(CFG_1B, steps=64), "1B", "stream_1b.json",
                      "48 BitLinear (in_proj 2048->8384, out_proj 4096->2048) + LM head "
                      "2048->50257 + final RMSNorm on the GPU; ssm_inner on the CPU")


def leg_fast_quant(L, M=4096):
    """Fast against parity quantization on the same rows (the parity kernel
    is bit-exact with the reference's scalar quantizer): int8 mismatch rate,
    scale_x drift, the fp32 BitLinear outputs' largest difference relative
    to the output scale, and both quantizers' kernel time."""
    out = {}
    ev = Events(L)
    r = np.random.default_rng(17)
    for K, N in ((1024, 4192), (2048, 8384), (4096, 2048)):
        x = r.standard_normal((M, K)).astype(np.float32)
        g = (1.0 + 0.1 * r.standard_normal(K)).astype(np.float32)
        w = bh.synth_ternary(K, 1, N, K, bh.SYNTH_P0_40)
        dx, dg, dW = (bh.DeviceBuffer.from_array(a) for a in (x, g, w))
        res = {}
        for name, fn in (("parity", L.bm_hip_quantize_dev), ("fast", L.bm_hip_quantize_fast_dev)):
            dq, ds = bh.DeviceBuffer(M * K), bh.DeviceBuffer(4 * M)
            da = bh.DeviceBuffer(L.bm_hip_act_bytes(M, K))
            do = bh.DeviceBuffer(4 * M * N)
            q = lambda: bh.check(fn(dx.ptr, M, K, K, dg.ptr, None, dq.ptr, K, ds.ptr, da.ptr,
                                    None), name)
            q()
            ev.start()
            for _ in range(5):
                q()
            us = ev.stop_ms() * 1e3 / 5
            bh.check(L.bm_hip_bitlinear_act_dev(da.ptr, ds.ptr, M, dW.ptr, N, K, 0.02, 0, do.ptr,
                                                None), "product")
            L.bm_hip_synchronize()
            res[name] = (dq.download((M, K), np.int8), ds.download(M, np.float32),
                         do.download((M, N), np.float32), us)
            for b in (dq, ds, da, do):
                b.free()
        for b in (dx, dg, dW):
            b.free()
        (pq, ps, po, pus), (fq, fs, fo, fus) = res["parity"], res["fast"]
        d = fq.astype(np.int32) - pq.astype(np.int32)
        out["K%d" % K] = dict(
            tokens=M, int8_mismatch_rate=float("%.3g" % (np.count_nonzero(d) / d.size)),
            int8_max_abs_diff=int(np.abs(d).max()),
            scale_x_max_rel_diff=float("%.3g" % np.max(np.abs(fs / ps - 1.0))),
            out_max_abs_diff_over_max_abs=float("%.3g" % (np.max(np.abs(fo - po)) /
                                                          np.max(np.abs(po)))),
            quantize_us_parity=round(pus, 1), quantize_us_fast=round(fus, 1))
    return out


def gemv1_inputs():
    K, N = 1024, 4384
    return (bh.synth_ternary(1, 1, N, K, bh.SYNTH_UNIFORM), bh.synth_normal(1, 2, (1, K), 1.0),
            np.ones(K, np.float32), K, N, 0.02)


def leg_gemv1(L, reps=200, cpu=True):
    packed, x, g, K, N, scale = gemv1_inputs()
    dW, dx, dg = (bh.DeviceBuffer.from_array(a) for a in (packed, x, g))
    dout, dq, ds = bh.DeviceBuffer(4 * N), bh.DeviceBuffer(K), bh.DeviceBuffer(4)
    da = bh.DeviceBuffer(L.bm_hip_act_bytes(1, K))
    call = lambda: bh.check(L.bm_hip_bitlinear_dev(dx.ptr, 1, K, dg.ptr, dW.ptr, N, scale, 1,
                                                   dout.ptr, dq.ptr, K, ds.ptr, da.ptr, None),
                            "bitlinear")
    for _ in range(5):
        call()
    ev = Events(L)
    ev.start()
    for _ in range(reps):
        call()
    dev_us = ev.stop_ms() * 1e3 / reps
    # cold: 460 distinct copies of the weights (516 MB, more than the 256 MB
    # last-level cache), one per call in turn
    n_copies = 460
    wbytes = N * K // 4
    cold = [bh.DeviceBuffer(wbytes) for _ in range(n_copies)]
    for c in cold:
        bh.check(L.bm_hip_copy_dev(c.ptr, dW.ptr, wbytes, None), "copy")
    cold_call = lambda c: bh.check(L.bm_hip_bitlinear_dev(dx.ptr, 1, K, dg.ptr, c.ptr, N, scale,
                                                          1, dout.ptr, dq.ptr, K, ds.ptr, da.ptr,
                                                          None), "bitlinear")
    for c in cold[:20]:
        cold_call(c)
    ev.start()
    for c in cold:
        cold_call(c)
    cold_us = ev.stop_ms() * 1e3 / n_copies
    for c in cold:
        c.free()
    for b in (dW, dx, dg, dout, dq, ds, da):
        b.free()
    # the drop-in entry with host buffers (PCIe and a synchronisation per call)
    w = bh.make_tensor(packed, N, K, scale)
    nw = bh.make_tensor(data=g)
    out = np.empty(N, np.float32)
    xn = np.empty(K, np.float32)
    xq = np.zeros(K + 32, np.int8)
    for _ in range(5):
        L.hip_bitlinear_forward(bh.ptr(x), K, C.byref(w), C.byref(nw), bh.ptr(out), bh.ptr(xn),
                                bh.ptr(xq))
    t = []
    for _ in range(50):
        t0 = time.perf_counter()
        L.hip_bitlinear_forward(bh.ptr(x), K, C.byref(w), C.byref(nw), bh.ptr(out), bh.ptr(xn),
                                bh.ptr(xq))
        t.append(time.perf_counter() - t0)
    drop_us = float(np.median(t)) * 1e6
    # the drop-in as the reference uses it: weights of a model image that
    # bm_hip_set_mmap registered at load (255M width: K=1024 -> N=4192)
    img = bh.synth_model(1000, K, 1, 32, 1, bh.SYNTH_UNIFORM)
    assert L.bm_hip_set_mmap(bh.ptr(img), img.nbytes)
    wi = bh.image_tensors(img, 0, bh.BM_L_IN_PROJ)
    ni = bh.image_tensors(img, 0, bh.BM_L_IN_NORM)
    out_i = np.empty(wi.rows, np.float32)
    for _ in range(5):
        L.hip_bitlinear_forward(bh.ptr(x), K, C.byref(wi), C.byref(ni), bh.ptr(out_i),
                                bh.ptr(xn), bh.ptr(xq))
    t = []
    for _ in range(50):
        t0 = time.perf_counter()
        L.hip_bitlinear_forward(bh.ptr(x), K, C.byref(wi), C.byref(ni), bh.ptr(out_i),
                                bh.ptr(xn), bh.ptr(xq))
        t.append(time.perf_counter() - t0)
    reg_us = float(np.median(t)) * 1e6
    res = dict(gpu_device_us=round(dev_us, 2), gpu_device_GBps=round(wbytes / dev_us / 1e3, 1),
               gpu_device_us_cold=round(cold_us, 2),
               gpu_device_GBps_cold=round(wbytes / cold_us / 1e3, 1),
               gpu_dropin_us=round(drop_us, 2), gpu_dropin_registered_us=round(reg_us, 2),
               packed_bytes=wbytes,
               note="device call = quantize + GEMV kernels on resident buffers (weights stay "
                    "in cache between calls; _cold: 460 copies of the weights, 516 MB, used in "
                    "turn, so each call streams them from HBM); drop-in = hip_bitlinear_forward on host buffers, "
                    "weights uploaded per call (not in a registered image); drop-in registered "
                    "= the same entry on a model image registered by bm_hip_set_mmap "
                    "(K=1024 -> N=4192), per call: one kernel reading x from and writing its "
                    "results to mapped host memory, completion polled by the host")
    res["roofline_cold"] = roofline_obj(
        "k_rows_fused, K=1024 form (RMSNorm + int8 + GEMV, one launch)",
        "bitlinear_k1024_n4384", "gemv1", wbytes, cold_us,
        "config 1 (K=1024 -> N=4384, one token) through bm_hip_bitlinear_dev, weights cold "
        "(460 copies used in turn); avg_us: HIP events over 460 back-to-back calls, launch "
        "gaps included; bytes: packed weights")
    res["roofline_warm"] = roofline_obj(
        "k_rows_fused, K=1024 form", "bitlinear_k1024_n4384_warm", "gemv1", wbytes,
        dev_us, "the same call with the weights cache-resident")
    if cpu:
        res.update(cpu_gemv1())
    return res


def cpu_gemv_child(threads, kind, reps=200):
    """Times the reference's own bitlinear_forward (kind 1: what dispatch_init
    picks here, AVX2; kind 0: scalar) on the K=1024 -> N=4384 inputs; median
    of `reps` calls after warm-up.  Runs in a process without the GPU."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import native
    R = native.ref()
    name = R.bmref_init(threads, kind).decode()
    R.bmref_set_poll(100)
    packed, x, g, K, N, scale = gemv1_inputs()
    out = np.empty(N, np.float32)
    xn = np.empty(K, np.float32)
    xq = np.zeros(K + 32, np.int8)
    args = (native.ptr(x), K, native.ptr(packed), N, K, C.c_float(scale), native.ptr(g),
            native.ptr(out), native.ptr(xn), native.ptr(xq))
    for _ in range(20):
        R.bmref_bitlinear_forward(*args)
    t = []
    for _ in range(reps):
        t0 = time.perf_counter()
        R.bmref_bitlinear_forward(*args)
        t.append(time.perf_counter() - t0)
    R.bmref_shutdown()
    print(json.dumps(dict(us=round(float(np.median(t)) * 1e6, 2), kernels=name,
                          threads=threads)), flush=True)


def cpu_gemv1():
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import native
    import subprocess
    if not native.ref_available():
        return {}
    out = {}
    for key, threads, kind in (("cpu_avx2", cpu_threads(), 1), ("cpu_scalar", 1, 0)):
        cmd = [sys.executable, os.path.abspath(__file__), "--cpu-gemv", str(threads), str(kind)]
        try:
            r = subprocess.run(cmd, stdout=subprocess.PIPE, timeout=120, text=True)
        except subprocess.TimeoutExpired:
            continue
        lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
        if r.returncode == 0 and lines:
            d = json.loads(lines[-1])
            out[key + "_us"] = d["us"]
            out[key + "_threads"] = d["threads"]
            out[key + "_kernels"] = d["kernels"]
    return out


def leg_stress(L, reps=10):
    K = N = 8192
    w = bh.synth_ternary(5, 1, N, K, bh.SYNTH_P0_60)
    dW = bh.DeviceBuffer.from_array(w)
    del w
    out = {}
    ev = Events(L)
    for M in (1, 16, 4096):
        xq = bh.synth_int8(5, 2, (M, K))
        dx = bh.DeviceBuffer.from_array(xq)
        da = bh.DeviceBuffer(L.bm_hip_i8_act_bytes(M, K))
        do = bh.DeviceBuffer(4 * M * N)
        call = lambda: bh.check(L.bm_hip_ternary_gemm_i32_dev(dx.ptr, M, K, dW.ptr, N, K, 0,
                                                              do.ptr, da.ptr, None), "stress")
        for _ in range(2):
            call()
        ev.start()
        for _ in range(reps):
            call()
        us = ev.stop_ms() * 1e3 / reps
        r = dict(us=round(us, 2), tops=round(2.0 * M * N * K / (us * 1e-6) / 1e12, 1))
        if M < 4096:
            r["weight_GBps_warm"] = round(N * K / 4 / (us * 1e-6) / 1e9, 1)
        out["M%d" % M] = r
        for b in (dx, da, do):
            b.free()
    dW.free()
    # cold: 32 distinct copies of the tensor (537 MB, more than the 256 MB
    # last-level cache), one per call in turn, so every call streams its
    # weights from HBM
    n_copies = 32
    cold = [bh.DeviceBuffer(N * K // 4) for _ in range(n_copies)]
    w = bh.synth_ternary(5, 1, N, K, bh.SYNTH_P0_60)
    src = bh.DeviceBuffer.from_array(w)
    del w
    for c in cold:
        bh.check(L.bm_hip_copy_dev(c.ptr, src.ptr, N * K // 4, None), "copy")
    src.free()
    for M in (1, 16):
        xq = bh.synth_int8(5, 2, (M, K))
        dx = bh.DeviceBuffer.from_array(xq)
        da = bh.DeviceBuffer(L.bm_hip_i8_act_bytes(M, K))
        do = bh.DeviceBuffer(4 * M * N)
        for canon in (0, 1):
            call = lambda c: bh.check(L.bm_hip_ternary_gemm_i32_dev(
                dx.ptr, M, K, c.ptr, N, K, canon, do.ptr, da.ptr, None), "stress")
            for c in cold:
                call(c)
            ev.start()
            for rep in range(2):
                for c in cold:
                    call(c)
            us = ev.stop_ms() * 1e3 / (2 * n_copies)
            if canon:
                # the same weights declared free of code 11 (as a loaded
                # model's are, rewritten once at load): no in-kernel rewrite
                out["M%d" % M]["cold_us_canonical"] = round(us, 2)
                continue
            out["M%d" % M]["cold_us"] = round(us, 2)
            out["M%d" % M]["weight_GBps_cold"] = round(N * K / 4 / (us * 1e-6) / 1e9, 1)
            out["M%d" % M]["weight_frac_of_hbm_cold"] = round(N * K / 4 / (us * 1e-6) / 1e9 /
                                                              HBM_PEAK_GBPS, 4)
        for b in (dx, da, do):
            b.free()
    for c in cold:
        c.free()
    out["note"] = ("M=1: one launch (k_rows_i8); M=16: one launch (k_gemm_few reading the "
                   "int8 rows itself); M=4096: k_prep_i8 + k_gemm; canonical=0 (code 11 "
                   "handled in-kernel; cold_us_canonical: the same calls with canonical=1, "
                   "the weights holding no code 11); warm: the one 16.8 MB weight tensor "
                   "stays cache-resident across calls; cold: 32 copies (537 MB) used in "
                   "turn, so each call streams its weights from HBM")
    wb = N * K // 4
    out["roofline_m1_cold"] = roofline_obj(
        "k_rows_i8, K=8192 form (int8 GEMV, one launch)", "stress_m1", "stress",
        wb + K + 4 * N, out["M1"]["cold_us"],
        "bytes: packed weights + int8 input + int32 output; avg_us: HIP events over 64 "
        "back-to-back calls on cold weights")
    out["roofline_m16_cold"] = roofline_obj(
        "k_gemm_few, int8-row form (M=16 on int8 MFMA, one launch)", "stress_m16", "stress",
        wb + 16 * K + 4 * 16 * N, out["M16"]["cold_us"],
        "bytes: packed weights + int8 inputs + int32 outputs; avg_us: HIP events over 64 "
        "back-to-back calls on cold weights")
    return out


def leg_roofline(L, reps=5):
    """The GEMV's streaming ceiling (gemv_stream_ceiling): the 1B in_proj's
    K=2048 row GEMV over 126 stacked copies of its rows (540 MB in one
    launch), no BASELINE config -- the rate the row kernel reaches once
    launch and latency costs vanish."""
    K, N_layer = 2048, 2 * 4096 + 3 * 64              # in_proj 2048 -> 8384
    row_bytes = K // 4
    target = 512 << 20
    n_layers_eq = (target + N_layer * row_bytes - 1) // (N_layer * row_bytes)
    N = n_layers_eq * N_layer                         # stacked distinct rows, one launch
    wbytes = N * row_bytes
    w_host = bh.synth_ternary(7, 1, N, K, bh.SYNTH_P0_40)
    dW = bh.DeviceBuffer.from_array(w_host)
    del w_host
    x = bh.synth_normal(7, 2, (1, K), 1.0)
    g = np.ones(K, np.float32)
    dx, dg = bh.DeviceBuffer.from_array(x), bh.DeviceBuffer.from_array(g)
    dq, ds = bh.DeviceBuffer(K), bh.DeviceBuffer(4)
    da = bh.DeviceBuffer(L.bm_hip_act_bytes(1, K))
    dout = bh.DeviceBuffer(4 * N)
    bh.check(L.bm_hip_quantize_dev(dx.ptr, 1, K, K, dg.ptr, None, dq.ptr, K, ds.ptr, da.ptr,
                                   None), "quantize")
    ev = Events(L)
    for _ in range(2):                                # warm the code path
        bh.check(L.bm_hip_bitlinear_act_dev(da.ptr, ds.ptr, 1, dW.ptr, N, K, 0.02, 1, dout.ptr,
                                            None), "gemv")
    ev.start()
    for _ in range(reps):
        bh.check(L.bm_hip_bitlinear_act_dev(da.ptr, ds.ptr, 1, dW.ptr, N, K, 0.02, 1, dout.ptr,
                                            None), "gemv")
    ms = ev.stop_ms() / reps
    achieved = wbytes / (ms * 1e-3) / 1e9
    for b in (dW, dx, dg, dq, ds, da, dout):
        b.free()
    return dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBPS, unit="GB/s",
                frac=round(achieved / HBM_PEAK_GBPS, 4), traffic=measured_traffic(N),
                kernel="k_gemv<T=32,P=1,GW=8,canonical,store> (K=2048 decode GEMV, 8 row groups per wave)",
                bytes_per_launch=wbytes, launch_us=round(ms * 1e3, 2),
                rows_per_launch=N)


TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "traffic_per_launch.txt")
PROFILE_FILES = {
    "decode": os.path.join(ROOT, "profiles", "decode_1b_kernels.txt"),
    "gemv1": os.path.join(ROOT, "profiles", "bitlinear_k1024_kernels.txt"),
    "stress": os.path.join(ROOT, "profiles", "stress_k8192_kernels.txt"),
}


def traffic_of(key):
    """HBM bytes per launch of a kernel/workload from the committed counter
    summary (lines 'traffic <key> <read B> <written B>': FETCH_SIZE and
    WRITE_SIZE per dispatch, calibrated with a copy of known size)."""
    try:
        for line in open(TRAFFIC_SUMMARY):
            f = line.split()
            if len(f) == 4 and f[0] == "traffic" and f[1] == key:
                return int(f[2]) + int(f[3])
    except (OSError, ValueError):
        pass
    return None


def profile_avg_us(which, name):
    """Average duration (us) of a kernel in a committed rocprofv3 summary:
    its line 'avg_us <name> <value>'."""
    try:
        for line in open(PROFILE_FILES[which]):
            f = line.split()
            if len(f) == 3 and f[0] == "avg_us" and f[1] == name:
                return float(f[2])
    except (OSError, ValueError, KeyError):
        pass
    return None


def roofline_obj(kernel, key, which, bytes_per_launch, us, note):
    """A roofline object for one kernel: algorithmic bytes per launch over
    its live average duration, against the HBM peak."""
    ach = bytes_per_launch / (us * 1e-6) / 1e9
    return dict(bound="hbm", achieved=round(ach, 1), peak=HBM_PEAK_GBPS, unit="GB/s",
                frac=round(ach / HBM_PEAK_GBPS, 4), traffic=traffic_of(key), kernel=kernel,
                bytes_per_launch=bytes_per_launch, avg_us=round(us, 3),
                profile_avg_us=profile_avg_us(which, key), note=note)


def roofline_decode(c, dev_ms_per_step):
    """The headline decode against HBM: the packed weight bytes of one token
    over the device time of a step, and its dominant kernel (the in_proj +
    SSM kernel: a layer's in_proj rows per launch) at its average duration
    in the decode phase of the committed profile."""
    dm, di, nh = c["d_model"], 2 * c["d_model"], c["n_heads"]
    bpt = packed_bytes_per_token(c)
    ach = bpt / (dev_ms_per_step * 1e-3) / 1e9
    r = dict(bound="hbm", achieved=round(ach, 1), peak=HBM_PEAK_GBPS, unit="GB/s",
             frac=round(ach / HBM_PEAK_GBPS, 4), bytes_per_token=bpt,
             device_ms_per_step=dev_ms_per_step)
    avg = profile_avg_us("decode", "k_inproj_ssm")
    if avg:
        inproj_bytes = (2 * di + 3 * nh) * dm // 4
        k_ach = inproj_bytes / (avg * 1e-6) / 1e9
        r["dominant_kernel"] = dict(name="k_inproj_ssm (in_proj quantize + GEMV + SSM step)",
                                    bytes_per_launch=inproj_bytes, avg_us=avg,
                                    achieved=round(k_ach, 1), frac=round(k_ach / HBM_PEAK_GBPS, 4),
                                    source="profiles/decode_1b_kernels.txt")
    return r


def measured_traffic(rows):
    """HBM bytes per GEMV launch from the committed counter summary (a line
    'bytes_per_launch: <int> rows: <int>'), if it covers this shape."""
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("bytes_per_launch:"):
                f = line.split()
                if int(f[3]) == rows:
                    return int(f[1])
    except (OSError, ValueError, IndexError):
        pass
    return None


def leg_copy(L, reps=5):
    n = 512 << 20
    a, b = bh.DeviceBuffer(n), bh.DeviceBuffer(n)
    bh.check(L.bm_hip_memset(a.ptr, 1, n), "memset")
    ev = Events(L)
    for _ in range(2):
        bh.check(L.bm_hip_copy_dev(b.ptr, a.ptr, n, None), "copy")
    ev.start()
    for _ in range(reps):
        bh.check(L.bm_hip_copy_dev(b.ptr, a.ptr, n, None), "copy")
    ms = ev.stop_ms() / reps
    a.free()
    b.free()
    return dict(bytes_read=n, bytes_written=n, us=round(ms * 1e3, 1),
                GBps_read_plus_write=round(2 * n / (ms * 1e-3) / 1e9, 1))


def leg_mfma(L, iters=2000):
    sink = bh.DeviceBuffer(4)
    ev = Events(L)
    blocks = 512  # 256-thread blocks: two waves on every SIMD of the 256 CUs
    out = {}
    for name, tern in (("fixed_operands_tops", 0), ("ternary_operands_tops", 1)):
        bh.check(L.bm_hip_mfma_peak_dev(blocks, 50, tern, sink.ptr, None), "mfma")
        ev.start()
        bh.check(L.bm_hip_mfma_peak_dev(blocks, iters, tern, sink.ptr, None), "mfma")
        ms = ev.stop_ms()
        out[name] = round(blocks * 4 * iters * 16 * 65536.0 / (ms * 1e-3) / 1e12, 1)
    sink.free()
    return out


def leg_prefill(L, reps=10):
    out = {}
    ev = Events(L)
    for K, N in ((2048, 8512), (4096, 2048)):
        M = 2048
        w = bh.synth_ternary(11, 1, N, K, bh.SYNTH_UNIFORM)
        x = bh.synth_normal(11, 2, (M, K), 1.0)
        dW, dx = bh.DeviceBuffer.from_array(w), bh.DeviceBuffer.from_array(x)
        dg = bh.DeviceBuffer.from_array(np.ones(K, np.float32))
        dq, ds = bh.DeviceBuffer(M * K), bh.DeviceBuffer(4 * M)
        da = bh.DeviceBuffer(L.bm_hip_act_bytes(M, K))
        dout = bh.DeviceBuffer(4 * M * N)
        bh.check(L.bm_hip_quantize_dev(dx.ptr, M, K, K, dg.ptr, None, dq.ptr, K, ds.ptr, da.ptr,
                                       None), "quantize")
        bh.check(L.bm_hip_bitlinear_act_dev(da.ptr, ds.ptr, M, dW.ptr, N, K, 0.02, 1, dout.ptr,
                                            None), "gemm")
        ev.start()
        for _ in range(reps):
            bh.check(L.bm_hip_bitlinear_act_dev(da.ptr, ds.ptr, M, dW.ptr, N, K, 0.02, 1,
                                                dout.ptr, None), "gemm")
        ms = ev.stop_ms() / reps
        ev.start()
        for _ in range(reps):
            bh.check(L.bm_hip_quantize_dev(dx.ptr, M, K, K, dg.ptr, None, dq.ptr, K, ds.ptr,
                                           da.ptr, None), "quantize")
        qms = ev.stop_ms() / reps
        tops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        out["%dx%dx%d" % (M, K, N)] = dict(gemm_us=round(ms * 1e3, 1), tops=round(tops, 1),
                                           frac=round(tops / I8_PEAK_TOPS, 4),
                                           quantize_us=round(qms * 1e3, 1))
        for b in (dW, dx, dg, dq, ds, da, dout):
            b.free()
    return out


def leg_vendor(timeout_s=180):
    """The vendor library's dense int8 GEMM (torch._int_mm, which runs on
    hipBLASLt) on the prefill and stress shapes: int8 x int8 -> int32 with
    neither the ternary decode nor the fp32 slice epilogue -- a reference
    point for what an int8 MFMA GEMM reaches at these sizes on this GPU.
    Run in a child process of its own (torch does not see the device in a
    process whose HIP runtime this library already started)."""
    import subprocess
    try:
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor-child"],
                           stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                           timeout=timeout_s)
    except subprocess.TimeoutExpired:
        log("vendor int8 GEMM child timed out")
        return None
    lines = [l for l in r.stdout.splitlines() if l.startswith("{")]
    if r.returncode != 0 or not lines:
        log("vendor int8 GEMM child failed (rc %d): %s" % (r.returncode, r.stderr[-300:]))
        return None
    return json.loads(lines[-1])


def vendor_child(reps=20):
    try:
        import torch
    except ImportError:
        print("{}")
        return
    if not torch.cuda.is_available():
        print("{}")
        return
    out = {}
    g = torch.Generator(device="cuda").manual_seed(5)
    for M, K, N in ((2048, 2048, 8512), (2048, 4096, 2048), (4096, 8192, 8192)):
        a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device="cuda", generator=g)
        b = torch.randint(-1, 2, (N, K), dtype=torch.int8, device="cuda", generator=g)
        bt = b.t()  # K x N, column-major: the layout hipBLASLt takes without a copy
        for _ in range(3):
            torch._int_mm(a, bt)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            torch._int_mm(a, bt)
        e1.record()
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        tops = 2.0 * M * N * K / (us * 1e-6) / 1e12
        out["%dx%dx%d" % (M, K, N)] = dict(us=round(us, 1), tops=round(tops, 1),
                                           frac=round(tops / I8_PEAK_TOPS, 4))
        del a, b, bt
    out["note"] = ("torch._int_mm (hipBLASLt), dense int8 operands, int32 out; no ternary decode, "
                   "no fp32 epilogue")
    print(json.dumps(out), flush=True)


def cpu_host():
    """What the host grants this process and what it is: CPUs in the
    affinity mask, CPUs of the machine, the cgroup CPU quota (cpu.max, in
    CPUs; None when unlimited) and the CPU model."""
    try:
        granted = len(os.sched_getaffinity(0))
    except AttributeError:
        granted = os.cpu_count() or 1
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
        if q != "max":
            quota = round(int(q) / int(period), 2)
    except (OSError, ValueError):
        pass
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for l in f:
                if l.startswith("model name"):
                    model = l.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return dict(cores_granted=granted, cores_host=os.cpu_count(), cpu_quota=quota,
                cpu_model=model)


def cpu_threads():
    """Pool threads of the CPU baseline: one fewer than the CPUs granted
    (affinity mask and cgroup quota), at most 15.  The reference's pool
    spins without yielding in its completion waits and barriers
    (src/threadpool.c:503-507, 611-614), so a pool thread that loses its
    CPU to another runnable thread (this process's, the runtime's) holds up
    the whole pool, and a cgroup whose quota equals its CPU count is
    throttled as soon as anything beside a full pool runs."""
    h = cpu_host()
    n = h["cores_granted"]
    if h["cpu_quota"]:
        n = min(n, int(h["cpu_quota"]))
    return max(1, min(n, 16) - 1)


def _ref_model_file(c, d):
    """The synthetic image of config c written to a file in d (the reference
    loads models from files, src/model.c:499-540)."""
    blob = bh.synth_model(c["vocab"], c["d_model"], c["n_layers"], c["n_heads"], c["seed"],
                          c["dist"])
    path = os.path.join(d, "model_%d.bin" % c["d_model"])
    with open(path, "wb") as f:
        blob.tofile(f)
        f.flush()
        os.fsync(f.fileno())  # written back before a spinning pool starts
    return path


def _cpu_decode(R, native, path, c, max_steps, budget_s, what):
    """Greedy decode tok/s of the reference (src/main.c:443-500 pattern):
    prefill of the prompt but its last token, then steps until max_steps
    or the time budget."""
    h = R.bmref_model_load(path.encode())
    if not h:
        raise RuntimeError("reference model_load failed")
    beat("cpu: %s model loaded" % what)
    prompt = bh.synth_prompt(c["seed"], c["vocab"], c["prompt"])
    p = np.ascontiguousarray(prompt[:-1], np.int32)
    R.bmref_model_prefill(h, native.ptr(p), p.size)
    beat("cpu: %s prompt prefilled" % what)
    hist, cur = [int(t) for t in prompt], int(prompt[-1])
    times = []
    start = time.perf_counter()
    for i in range(max_steps):
        harr = np.array(hist[-256:], np.int32)
        t0 = time.perf_counter()
        cur = R.bmref_model_step(h, cur, native.ptr(harr), harr.size, 1.0)
        times.append(time.perf_counter() - t0)
        hist.append(cur)
        if i % 16 == 0:
            beat("cpu: %s step %d %.2f ms" % (what, i, times[-1] * 1e3))
        if time.perf_counter() - start > budget_s:
            break
    R.bmref_model_free(h)
    return dict(value=round(len(times) / sum(times), 2), unit="tok/s", steps=len(times))


def _cpu_prefill(R, native, path, c, n_tokens, budget_s):
    """model_prefill (src/model.c:1045-1153) of n_tokens: tokens/s."""
    h = R.bmref_model_load(path.encode())
    toks = np.ascontiguousarray(bh.synth_prompt(c["seed"] + 1, c["vocab"], n_tokens), np.int32)
    t0 = time.perf_counter()
    R.bmref_model_prefill(h, native.ptr(toks), toks.size)
    dt = time.perf_counter() - t0
    R.bmref_model_free(h)
    return dict(tokens=n_tokens, ms=round(dt * 1e3, 1), tok_s=round(n_tokens / dt, 1))


def _cpu_batch_gemm(R, native, K, N, M):
    """bitlinear_forward_batch (AVX2: src/arch/avx2.c:384-452, with the
    per-token RMSNorm + int8 quantization of each token) on the prefill
    GEMM's inputs, M tokens: TOP/s of the 2*M*N*K products."""
    w = bh.synth_ternary(11, 1, N, K, bh.SYNTH_UNIFORM)
    x = bh.synth_normal(11, 2, (M, K), 1.0)
    g = np.ones(K, np.float32)
    out = np.empty((M, N), np.float32)
    xn = np.empty(K, np.float32)
    xq = np.zeros((M, K + 32), np.int8)
    args = (native.ptr(x), M, K, native.ptr(w), N, K, C.c_float(0.02), native.ptr(g),
            native.ptr(out), native.ptr(xn), native.ptr(xq), K + 32)
    R.bmref_bitlinear_forward_batch(*args)  # warm-up
    t0 = time.perf_counter()
    R.bmref_bitlinear_forward_batch(*args)
    dt = time.perf_counter() - t0
    return dict(tokens=M, ms=round(dt * 1e3, 2), tops=round(2.0 * M * N * K / dt / 1e12, 4))


def _cpu_rows_int8(R, native, w, K, N, xq):
    """The reference's row kernel (the AVX2 row worker, src/arch/avx2.c:
    99-268) on int8 activations, one call per token: seconds per token."""
    out = np.empty(N, np.float32)
    t = []
    for m in range(xq.shape[0]):
        row = np.ascontiguousarray(xq[m])
        t0 = time.perf_counter()
        R.bmref_rows_int8(native.ptr(row), native.ptr(w), N, K, C.c_float(1.0), native.ptr(out))
        t.append(time.perf_counter() - t0)
    return t


def beat(msg):
    """A progress line of a CPU child (read by its parent's watchdog)."""
    print("P " + msg, flush=True)
    log(msg)


def cpu_child(threads, budget_s):
    """Runs in a separate process that never touches the GPU: the
    reference's own C (oracle/_ref: dispatch_init -> AVX2+FMA kernels, its
    thread pool with the default spin wait) on bounded samples of every
    workload of the bench.  Prints one JSON line per leg ("CPU <leg> ...")
    so that a leg that runs out of time loses only itself."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import native
    R = native.ref()
    name = R.bmref_init(threads, 1).decode()
    R.bmref_set_poll(100)
    one = threads == 1

    def emit(leg, d):
        d.update(threads=threads, kernels=name)
        print("CPU %s %s" % (leg, json.dumps(d)), flush=True)

    with tempfile.TemporaryDirectory(dir=tempfile.gettempdir()) as d:
        p1b = _ref_model_file(CFG_1B, d)
        beat("cpu[%d]: 1B model file written" % threads)
        emit("decode_1b", _cpu_decode(R, native, p1b, CFG_1B, 64, budget_s, "1B"))
        # time to first token: 1024 tokens (a 256-token sample on one thread)
        n_pf = 256 if one else 1024
        r = _cpu_prefill(R, native, p1b, CFG_1B, n_pf, budget_s)
        r["sample"] = "%d-token prefill" % n_pf
        emit("prefill_1b", r)
        beat("cpu[%d]: prefill %s" % (threads, json.dumps(r)))
        os.unlink(p1b)
        p255 = _ref_model_file(CFG_255M, d)
        emit("decode_255m", _cpu_decode(R, native, p255, CFG_255M, 64 if one else 128, budget_s,
                                        "255M"))
        os.unlink(p255)
    # prefill GEMM shapes at M=2048 (512 tokens on one thread)
    for K, N in ((2048, 8512), (4096, 2048)):
        M = 512 if one else 2048
        r = _cpu_batch_gemm(R, native, K, N, M)
        r["sample"] = "%d of the 2048 tokens" % M if one else "all 2048 tokens"
        emit("gemm_%dx%dx%d" % (2048, K, N), r)
        beat("cpu[%d]: gemm K=%d N=%d %s" % (threads, K, N, json.dumps(r)))
    # stress shape K = N = 8192, int8 activations: M = 1, 16 and a sample of
    # the 4096-token product (the reference has no int8 batch entry: one row
    # kernel call per token)
    K = N = 8192
    w = bh.synth_ternary(5, 1, N, K, bh.SYNTH_P0_60)
    xq = bh.synth_int8(5, 2, (16, K))
    beat("cpu[%d]: stress shape" % threads)
    _cpu_rows_int8(R, native, w, K, N, xq[:2])  # warm-up
    t1 = _cpu_rows_int8(R, native, w, K, N, xq[:1] if one else xq[:1].repeat(9, 0))
    t16 = _cpu_rows_int8(R, native, w, K, N, xq)
    us1 = float(np.median(t1)) * 1e6
    us16 = float(sum(t16)) * 1e6
    samp = 16 if one else 64
    xs = bh.synth_int8(5, 3, (samp, K))
    ts = _cpu_rows_int8(R, native, w, K, N, xs)
    per_tok = float(sum(ts)) / samp
    emit("stress", dict(M1_us=round(us1, 1), M1_weight_GBps=round(N * K / 4 / us1 / 1e3, 2),
                        M16_us=round(us16, 1), M16_tops=round(2.0 * 16 * N * K / us16 / 1e6, 4),
                        M4096_est_ms=round(per_tok * 4096 * 1e3, 1),
                        M4096_tops=round(2.0 * N * K / per_tok / 1e12, 4),
                        sample="M=4096 from %d of its tokens, one row-kernel call each" % samp))
    R.bmref_shutdown()


def thread_states(pid):
    """State, kernel wait channel and CPU time of each thread of a process
    (from /proc, no tracing): how a stalled child was stalled."""
    out = {}
    try:
        for tid in sorted(os.listdir("/proc/%d/task" % pid), key=int):
            base = "/proc/%d/task/%s/" % (pid, tid)
            try:
                comm = open(base + "comm").read().strip()
                st = open(base + "stat").read()
                f = st[st.rindex(")") + 2:].split()
                wchan = open(base + "wchan").read().strip() if os.path.exists(base + "wchan") \
                    else "?"
                key = "%s%s %s %s" % ("main:" if int(tid) == pid else "", comm, f[0], wchan)
                d = out.setdefault(key, dict(n=0, cpu_ticks=0))
                d["n"] += 1
                d["cpu_ticks"] += int(f[11]) + int(f[12])
                if f[0] != "R":
                    # where a waiting thread waits: its system call (or -1 for
                    # a fault) and the mapping its user-space PC lies in
                    sc = _read(base + "syscall").split()
                    where = _mapping(pid, int(sc[-1], 16)) if len(sc) >= 3 else ""
                    d.setdefault("tids", []).append(
                        "%s start=%s cpu=%d sc=%s %s" % (tid, f[19], int(f[11]) + int(f[12]),
                                                         " ".join(sc[:2]), where))
            except (OSError, ValueError, IndexError):
                continue
    except OSError:
        pass
    return out


def _read(path):
    try:
        return open(path).read().strip()
    except OSError:
        return ""


def _mapping(pid, pc):
    """File (and offset in it) of the mapping that holds address pc."""
    for line in _read("/proc/%d/maps" % pid).splitlines():
        f = line.split()
        lo, hi = (int(v, 16) for v in f[0].split("-"))
        if lo <= pc < hi:
            return "%s+0x%x" % (os.path.basename(f[5]) if len(f) > 5 else "anon",
                                pc - lo + int(f[2], 16))
    return "pc=0x%x" % pc


def dropin_child(threads):
    """The drop-in decode leg in a process of its own (its spin-wait pool
    never shares a process with the other legs); prints "DROPIN {json}"."""
    import faulthandler
    import signal
    # the watchdog asks a silent child for its Python stacks before it stops it
    faulthandler.register(signal.SIGUSR1, all_threads=True)
    L = bh.lib()
    if not L.bm_hip_init():
        sys.exit("bm_hip_init: " + bh.last_error())
    r = {"255m": leg_dropin_255m(L, threads)}
    r["1b"] = leg_dropin_1b(L, threads)
    print("DROPIN " + json.dumps(r), flush=True)


def run_dropin(threads, stall_s=60.0, total_s=300.0):
    """dropin_child, watched like the CPU suite: a child that prints nothing
    for stall_s is killed and run again once with half the threads; the
    result records the stalls."""
    import signal
    import subprocess
    import threading
    stalls = []
    start = time.time()
    for t in (threads, max(1, threads // 2)):
        cmd = [sys.executable, os.path.abspath(__file__), "--dropin-child", str(t)]
        # one OpenMP thread: the child's only OpenMP work is writing the
        # synthetic model file
        env = dict(os.environ, OMP_NUM_THREADS="1")
        proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, text=True, bufsize=1, env=env)
        lines, last = [], [time.time()]

        def read(f=proc.stdout, lines=lines, last=last):
            for l in f:
                lines.append(l)
                last[0] = time.time()

        rd = threading.Thread(target=read, daemon=True)
        rd.start()
        killed = False
        threads_seen = None
        while proc.poll() is None:
            time.sleep(0.2)
            if time.time() - last[0] > stall_s or time.time() - start > total_s:
                threads_seen = thread_states(proc.pid)
                try:
                    os.kill(proc.pid, signal.SIGUSR1)  # Python stacks to stderr
                    time.sleep(1.0)
                except OSError:
                    pass
                proc.kill()
                killed = True
                proc.wait()
        rd.join(5)
        if threads_seen:
            log("drop-in: stalled child's threads: %s" % json.dumps(threads_seen))
        for l in lines:
            if l.startswith("DROPIN "):
                d = json.loads(l[7:])
                if stalls:
                    for v in d.values():
                        v["stalls"] = stalls
                return d
        where = [l[2:].strip() for l in lines if l.startswith("P ")]
        stalls.append(dict(threads=t, after=where[-1] if where else "start",
                           stopped="no output for %ds" % stall_s if killed
                           else "rc %s" % proc.returncode))
        log("drop-in: child with %d threads stopped: %s" % (t, json.dumps(stalls[-1])))
        if time.time() - start > total_s:
            break
    return dict(tok_s=None, stalls=stalls)


def run_cpu_suite(threads, stall_s=20.0, total_s=240.0):
    """The CPU baseline legs in a child process, watched: a child that
    prints nothing for stall_s is killed and run again (same thread count
    once, then half), so that the bench line always comes out; the result
    records the retries (`retried`) and where a killed child had got to.
    The reference's pool spins without yielding in its completion waits and
    barriers (src/threadpool.c:515-521, 594-609), so one descheduled thread
    holds up all the others."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import native
    import subprocess
    import threading
    if not native.ref_available():
        return {}
    out, stalls = {}, []
    start = time.time()
    for t in (threads, threads, max(1, threads // 2))[:3 if threads > 1 else 2]:
        cmd = [sys.executable, os.path.abspath(__file__), "--cpu-child", str(t), "25"]
        proc = subprocess.Popen(cmd, stdout=subprocess.PIPE, text=True, bufsize=1)
        lines, last = [], [time.time()]

        def read(f=proc.stdout, lines=lines, last=last):
            for l in f:
                lines.append(l)
                last[0] = time.time()

        rd = threading.Thread(target=read, daemon=True)
        rd.start()
        killed = False
        while proc.poll() is None:
            time.sleep(0.2)
            if time.time() - last[0] > stall_s or time.time() - start > total_s:
                proc.kill()
                killed = True
                proc.wait()
        rd.join(5)
        got = 0
        for l in lines:
            if l.startswith("CPU "):
                _, leg, js = l.split(" ", 2)
                d = json.loads(js)
                d["retried"] = bool(stalls)
                out[leg] = d
                got += 1
        if not killed and proc.returncode == 0 and "stress" in out:
            break
        where = [l[2:].strip() for l in lines if l.startswith("P ")]
        stalls.append(dict(threads=t, after=where[-1] if where else "start"))
        log("cpu: child with %d threads stopped (%s) after: %s"
            % (t, "no output for %ds" % stall_s if killed else "rc %s" % proc.returncode,
               stalls[-1]["after"]))
        if time.time() - start > total_s:
            break
    if stalls:
        out["stalls"] = stalls
    return out


def main():
    if len(sys.argv) == 4 and sys.argv[1] == "--cpu-child":
        cpu_child(int(sys.argv[2]), float(sys.argv[3]))
        return
    if len(sys.argv) == 3 and sys.argv[1] == "--dropin-child":
        dropin_child(int(sys.argv[2]))
        return
    if len(sys.argv) == 2 and sys.argv[1] == "--vendor-child":
        vendor_child()
        return
    if len(sys.argv) == 4 and sys.argv[1] == "--cpu-gemv":
        cpu_gemv_child(int(sys.argv[2]), int(sys.argv[3]))
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--legs",
                    default="decode,sampled,fast,ceiling,mfma,prefill,d255m,gemv1,stress,vendor,"
                            "dropin,cpu")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: the BitLinear hot path runs on exactly one GPU (there is no "
              "multi-GPU path at bs=1); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    legs = set(a.legs.split(","))
    # the CPU baselines first, while this process has not started the GPU
    # runtime (the children never touch the GPU): one thread fewer than the
    # CPUs the box grants (at most 15), then one thread
    cpu_n = run_cpu_suite(cpu_threads()) if "cpu" in legs else {}
    cpu_1 = run_cpu_suite(1) if "cpu" in legs else {}
    cpu_stalls = cpu_n.pop("stalls", []) + cpu_1.pop("stalls", [])
    cpu = None
    if "decode_1b" in cpu_n:
        d = cpu_n["decode_1b"]
        cpu = dict(value=d["value"], unit="tok/s", cores=d["threads"], threads=d["threads"],
                   retried=d["retried"], kind="reference",
                   sample="%d greedy steps of the same 1B-shape decode after a 7-token prefill "
                          "(reference kernels: %s, %d threads, spin-wait pool)"
                          % (d["steps"], d["kernels"], d["threads"]),
                   thread_rule="one pool thread fewer than the CPUs granted (affinity and "
                               "cgroup quota), so that the spin-wait pool never competes with "
                               "the bench process or the host for its last CPU")
        cpu.update(cpu_host())
        if "decode_1b" in cpu_1:
            cpu["value_1_thread"] = cpu_1["decode_1b"]["value"]
        if cpu_stalls:
            cpu["stalled_children"] = cpu_stalls
        log("cpu baseline: %s" % json.dumps(cpu))
    L = bh.lib()
    if not L.bm_hip_init():
        sys.exit("bm_hip_init: " + bh.last_error())
    res = {}
    if "decode" in legs:
        wall, dev_ms, match, samp, pf, fres, ktimes = leg_decode(L, a.steps, a.warmup,
                                                                 "sampled" in legs,
                                                                 "fast" in legs)
        res["kernel_us"] = ktimes
        log("decode kernels, live: %s" % json.dumps(ktimes))
        res["fast"] = fres
        if fres:
            log("fast-mode decode: %s" % json.dumps(fres))
        res["decode"] = (wall, dev_ms, match)
        res["sampled"] = samp
        res["prefill_model"] = pf
        log("prefill: %s" % json.dumps(pf))
        log("decode: %d steps in %.2f ms wall (%.2f ms device)" % (a.steps, wall * 1e3, dev_ms))
        if samp:
            log("sampled decode: %s" % json.dumps(samp))
    roof = leg_roofline(L) if "ceiling" in legs else None
    if roof:
        log("GEMV stream ceiling: %.1f GB/s (%.1f%% of HBM peak), %.1f us per launch"
            % (roof["achieved"], 100 * roof["frac"], roof["launch_us"]))
    mf = leg_mfma(L) if "mfma" in legs else None
    if mf:
        log("mfma ceiling: %s" % json.dumps(mf))
    pre = leg_prefill(L) if "prefill" in legs else None
    if pre and mf:
        for v in pre.values():
            v["frac_of_ternary_ceiling"] = round(v["tops"] / mf["ternary_operands_tops"], 4)
    if pre:
        log("prefill: %s" % json.dumps(pre))
    d255 = leg_d255m(L, "fast" in legs) if "d255m" in legs else None
    fq = leg_fast_quant(L) if "fast" in legs else None
    if fq:
        log("fast-mode quantizer: %s" % json.dumps(fq))
    if d255:
        log("255M-shape decode: %s" % json.dumps(d255))
    g1 = leg_gemv1(L, cpu="cpu" in legs) if "gemv1" in legs else None
    if g1:
        log("K=1024 N=4384 BitLinear: %s" % json.dumps(g1))
    strs = leg_stress(L) if "stress" in legs else None
    if strs:
        log("stress K=N=8192: %s" % json.dumps(strs))
    vend = leg_vendor() if "vendor" in legs else None
    if vend:
        log("vendor int8 GEMM: %s" % json.dumps(vend))
    cpy = leg_copy(L) if "copy" in legs else None
    if cpy:
        log("copy: %s" % json.dumps(cpy))
    # in a child process: it starts the reference's spin-wait pool
    dropin = run_dropin(max(1, cpu_threads() - 1)) if "dropin" in legs else None
    if dropin:
        log("drop-in decode: %s" % json.dumps(dropin))

    bpt = packed_bytes_per_token(CFG_1B)
    line = {"metric": METRIC, "unit": "tok/s", "n_gpus": 1, "steps": a.steps,
            "warmup": a.warmup, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "int8", "data": "synthetic",
            "config": {"workload": "1B-shape BitMamba-2 greedy decode, bs=1 (24 layers, "
                                   "d_model 2048, d_inner 4096, 64 heads, in_proj 2048x8384, "
                                   "out_proj 4096x2048, vocab 50257, ternary p0=0.4)",
                       "prompt_tokens": CFG_1B["prompt"], "seed": CFG_1B["seed"],
                       "parallelism": "single GPU"}}
    if "decode" in res:
        wall, dev_ms, match = res["decode"]
        tok_s = a.steps / wall
        line.update(value=round(tok_s, 2), ms_per_step=round(wall * 1e3 / a.steps, 4),
                    packed_weight_GBps=round(tok_s * bpt / 1e9, 1),
                    packed_bytes_per_token=bpt, device_ms_per_step=round(dev_ms / a.steps, 4),
                    tokens_match_reference=match)
    else:
        line.update(value=None, ms_per_step=None)
    # the reference's CPU figures beside each GPU figure
    def cpu_of(leg):
        return {"threads_%d" % r[leg]["threads"]: r[leg] for r in (cpu_n, cpu_1) if leg in r}
    if cpu_n or cpu_1:
        line["cpu_decode_1b"] = cpu_of("decode_1b")
        if res.get("prefill_model") is not None:
            res["prefill_model"]["cpu"] = cpu_of("prefill_1b")
        if d255:
            d255["cpu"] = cpu_of("decode_255m")
        if dropin:
            dropin["cpu"] = cpu_of("decode_255m")
        if pre:
            for k in pre:
                pre[k]["cpu"] = cpu_of("gemm_" + k)
        if strs:
            strs["cpu"] = cpu_of("stress")
    if "decode" in res:
        c = CFG_1B
        dm, di, nh = c["d_model"], 2 * c["d_model"], c["n_heads"]
        kt = res["kernel_us"]
        line["roofline"] = roofline_obj(
            "k_inproj_ssm (1B in_proj 2048->8384: RMSNorm + int8 + GEMV + the SSM step of its "
            "heads, one launch per layer)", "k_inproj_ssm", "decode", (2 * di + 3 * nh) * dm // 4,
            kt["k_inproj_ssm"],
            "dominant kernel of the headline decode; bytes: a layer's packed in_proj weights; "
            "avg_us: 240 launches back to back on the model's stream between HIP events, the "
            "24 layers in turn (bm_hip_model_time_kernel)")
        rd = roofline_decode(c, line["device_ms_per_step"])
        rd["kernels"] = {
            "k_inproj_ssm": line["roofline"],
            "out_proj": roofline_obj(
                "k_rows_fused, out_proj form (1B out_proj 4096->2048: RMSNorm + int8 + GEMV + "
                "residual)",
                "out_proj", "decode", di * dm // 4, kt["out_proj"], "the layers in turn, live"),
            "lm_head": roofline_obj(
                "k_rows_fused, LM head form (final norm + LM head 2048->50257 + greedy "
                "candidates)", "lm_head", "decode", c["vocab"] * dm // 4, kt["lm_head"],
                "live"),
        }
        line["roofline_decode"] = rd
    line["decode_sampled"] = res.get("sampled")
    if res.get("fast") or fq:
        line["decode_fast"] = dict(res.get("fast") or {}, quantizer=fq,
                                   note="opt-in fast mode: sums of squares as a pairwise tree, "
                                        "not the reference's bits; value stays parity mode")
    line["prefill_1b"] = res.get("prefill_model")
    line.setdefault("roofline", None)
    line["gemv_stream_ceiling"] = roof
    line["mfma_ceiling"] = mf
    line["prefill_gemm"] = pre
    line["decode_255m"] = d255
    # a stalled child leaves {"tok_s": None, "stalls": ...} for both shapes
    line["dropin_decode_255m"] = dropin.get("255m", dropin) if dropin else None
    line["dropin_decode_1b"] = dropin.get("1b", dropin) if dropin else None
    line["bitlinear_k1024_n4384"] = g1
    line["stress_k8192_n8192"] = strs
    line["vendor_int8_gemm"] = vend
    line["cpu_baseline"] = cpu
    if cpy:
        line["copy_calibration"] = cpy
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
