"""Loaders for the native libraries the tests drive.

* the product: bitmamba.c_amd/libbitmamba_hip.so via bitmamba_hip (ctypes)
* the oracle:  oracle/liboracle.so (C restatement of the scalar path)
* the reference build: oracle/_ref/libbmref.so (the reference's own C
  sources compiled by oracle/Makefile; optional -- absent where the
  reference sources were not available at build time)
"""
import ctypes as C
import importlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "bitmamba.c_amd")
if PKG not in sys.path:
    sys.path.insert(0, PKG)
bh = importlib.import_module("bitmamba_hip")

ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
REF_PATH = os.path.join(ROOT, "oracle", "_ref", "libbmref.so")

_vp, _i, _f, _sz, _u64 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_uint64


def ptr(a):
    return a.ctypes.data_as(_vp)


_ORACLE_SIGS = {
    "orc_rng_next": (_u64, [C.POINTER(_u64)]),
    "orc_sample": (_i, [_vp, _i, _f, _f, _f, _i, C.POINTER(_u64)]),
    "orc_decode_weight": (_i, [_i]),
    "orc_luts": (None, [_vp, _vp, _vp]),
    "orc_rms_norm": (_f, [_vp, _i, _vp, _vp]),
    "orc_quantize": (_f, [_vp, _i, _f, _vp]),
    "orc_tmac_slice_count": (_i, [_i]),
    "orc_tmac_totals": (None, [_vp, _vp, _i, _i, _vp, _vp]),
    "orc_tmac_rows_f32": (None, [_vp, _vp, _i, _i, _f, _vp]),
    "orc_bitlinear_forward": (None, [_vp, _i, _vp, _i, _i, _f, _vp, _vp, _vp, _vp]),
    "orc_bitlinear_forward_batch": (None, [_vp, _i, _i, _vp, _i, _i, _f, _vp, _vp, _vp, _vp,
                                           _i]),
    "orc_ternary_gemm_i32": (None, [_vp, _i, _i, _vp, _i, _i, _vp]),
    "orc_ssm_inner": (None, [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                             _i, _i]),
    "orc_model_load": (_vp, [_vp, _sz]),
    "orc_model_free": (None, [_vp]),
    "orc_model_prefill": (None, [_vp, _vp, _i]),
    "orc_model_step": (_i, [_vp, _i, _vp, _i, _f]),
    "orc_model_logits": (C.POINTER(C.c_float), [_vp]),
    "orc_model_config": (_i, [_vp, _i]),
    "orc_model_layer_state": (_i, [_vp, _i, _vp, _vp]),
    "orc_expf_array": (None, [_vp, _vp, _sz]),
    "orc_logf_array": (None, [_vp, _vp, _sz]),
}

_REF_SIGS = {
    "bmref_init": (C.c_char_p, [_i, _i]),
    "bmref_shutdown": (None, []),
    "bmref_set_poll": (None, [_i]),
    "bmref_threads": (_i, []),
    "bmref_rms_norm": (_f, [_vp, _i, _vp, _vp]),
    "bmref_bitlinear_forward": (None, [_vp, _i, _vp, _i, _i, _f, _vp, _vp, _vp, _vp]),
    "bmref_bitlinear_forward_batch": (None, [_vp, _i, _i, _vp, _i, _i, _f, _vp, _vp, _vp, _vp,
                                             _i]),
    "bmref_row_worker_available": (_i, []),
    "bmref_rows_int8": (None, [_vp, _vp, _i, _i, _f, _vp]),
    "bmref_rng_seed": (None, [_u64]),
    "bmref_rng_next": (_u64, []),
    "bmref_lut": (None, [_vp, _vp, _vp]),
    "bmref_model_load": (_vp, [C.c_char_p]),
    "bmref_model_free": (None, [_vp]),
    "bmref_model_prefill": (None, [_vp, _vp, _i]),
    "bmref_model_step": (_i, [_vp, _i, _vp, _i, _f]),
    "bmref_model_step_sample": (_i, [_vp, _i, _vp, _i, _f, _f, _f, _f, _i]),
    "bmref_model_logits": (C.POINTER(C.c_float), [_vp]),
    "bmref_model_vocab": (_i, [_vp]),
    "bmref_model_layer_state": (_i, [_vp, _i, _vp, _vp]),
    "bmref_use_hip": (_i, [_vp]),
    "bmref_model_set_layer_state": (None, [_vp, _i, _vp, _vp, _i]),
    "bmref_kernels_name": (C.c_char_p, []),
    "bmref_model_image": (_i, [_vp, C.POINTER(_vp), C.POINTER(_sz)]),
    "bmref_model_prefill_batch": (_i, [_vp, _vp, _i, _vp]),
}

_oracle = None
_ref = None


def _load(path, sigs):
    L = C.CDLL(path)
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def oracle():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_PATH):
            raise RuntimeError("oracle not built (%s)" % ORACLE_PATH)
        _oracle = _load(ORACLE_PATH, _ORACLE_SIGS)
    return _oracle


def ref_available():
    return os.path.exists(REF_PATH)


def ref():
    global _ref
    if _ref is None:
        _ref = _load(REF_PATH, _REF_SIGS)
    return _ref


# ---------------------------------------------------------------------------
# numpy-level wrappers
# ---------------------------------------------------------------------------
def orc_bitlinear(x, packed, rows, cols, scale, gamma):
    """oracle scalar_bitlinear_forward for each row of x ([M][cols])."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
    M = x.shape[0]
    out = np.empty((M, rows), np.float32)
    xn = np.empty(cols, np.float32)
    xq = np.zeros((M, cols + 32), np.int8)
    oracle().orc_bitlinear_forward_batch(ptr(x), M, cols, ptr(packed), rows, cols, scale,
                                         ptr(gamma), ptr(out), ptr(xn), ptr(xq), cols + 32)
    return out, xn, xq[:, :cols].copy()


def ref_bitlinear(x, packed, rows, cols, scale, gamma):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
    M = x.shape[0]
    out = np.empty((M, rows), np.float32)
    xn = np.empty(cols, np.float32)
    xq = np.zeros((M, cols + 32), np.int8)
    ref().bmref_bitlinear_forward_batch(ptr(x), M, cols, ptr(packed), rows, cols, scale,
                                        ptr(gamma), ptr(out), ptr(xn), ptr(xq), cols + 32)
    return out, xn, xq[:, :cols].copy()


def orc_quantize_rows(x, gamma):
    """(x_norm, int8, scale_x, max_abs) per row, oracle semantics."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, n = x.shape
    xn = np.empty_like(x)
    xq = np.empty((M, n), np.int8)
    sc = np.empty(M, np.float32)
    mx = np.empty(M, np.float32)
    for m in range(M):
        row = np.ascontiguousarray(x[m])
        o = np.empty(n, np.float32)
        mx[m] = oracle().orc_rms_norm(ptr(row), n, ptr(gamma), ptr(o))
        q = np.empty(n, np.int8)
        sc[m] = oracle().orc_quantize(ptr(o), n, mx[m], ptr(q))
        xn[m], xq[m] = o, q
    return xn, xq, sc, mx


def orc_slice_totals(xq, packed, rows, cols):
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    S = max(oracle().orc_tmac_slice_count(cols), 1)
    st = np.empty((rows, S), np.int32)
    rt = np.empty(rows, np.int32)
    oracle().orc_tmac_totals(ptr(xq), ptr(packed), rows, cols, ptr(st), ptr(rt))
    return st, rt


def orc_gemm_i32(xq, packed, N, K):
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    M = xq.shape[0]
    out = np.empty((M, N), np.int32)
    oracle().orc_ternary_gemm_i32(ptr(xq), M, xq.shape[1], ptr(packed), N, K, ptr(out))
    return out


def decode_dense(packed, cols):
    """Closed form: w = min(code - 1, 1) for every column (numpy)."""
    p = np.asarray(packed, dtype=np.uint8)
    codes = np.stack([(p >> (2 * j)) & 3 for j in range(4)], axis=-1).reshape(p.shape[0], -1)
    w = np.minimum(codes.astype(np.int32) - 1, 1)
    return w[:, :cols]


def same_bits(a, b, what="values"):
    """Asserts bitwise equality of two arrays; on failure reports how many
    elements differ and the first few, never a full dump."""
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, "%s: shape %s vs %s" % (what, a.shape, b.shape)
    va = a.view(np.uint8).reshape(a.size, -1) if a.size else a
    vb = b.view(np.uint8).reshape(b.size, -1) if b.size else b
    diff = np.any(va != vb, axis=1) if a.size else np.zeros(0, bool)
    n = int(diff.sum())
    if n:
        idx = np.flatnonzero(diff)[:6]
        fa, fb = a.reshape(-1), b.reshape(-1)
        pairs = ", ".join("[%d] %r vs %r" % (i, fa[i], fb[i]) for i in idx)
        raise AssertionError("%s: %d of %d elements differ: %s" % (what, n, a.size, pairs))
