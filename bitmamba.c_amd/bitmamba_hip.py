"""ctypes binding of libbitmamba_hip.so (the C ABI declared in include/bm_hip.h).

Python callers (tests, bench.py) reach the gfx950 kernels only through this
module.  Loading fails loudly when the library has not been built; there is
no CPU fallback.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbitmamba_hip.so")

_vp, _sz, _i, _f, _u64 = C.c_void_p, C.c_size_t, C.c_int, C.c_float, C.c_uint64
_fp = C.POINTER(C.c_float)
_i8p = C.POINTER(C.c_int8)
_u8p = C.POINTER(C.c_uint8)


class Tensor(C.Structure):
    """struct tensor (src/bitmamba.h:65-74)."""
    _fields_ = [("data", _fp), ("packed_data", _u8p), ("rows", _i), ("cols", _i),
                ("n_elements", _sz), ("is_bitnet", C.c_bool), ("scale", _f)]


class SynthConfig(C.Structure):
    _fields_ = [("vocab", _i), ("d_model", _i), ("n_layers", _i), ("n_heads", _i),
                ("in_proj_rows", _i), ("ternary_dist", _i), ("fp_sigma", _f),
                ("ternary_scale", _f), ("seed", _u64)]


class Bit2Tensor(C.Structure):
    """bm_bit2_tensor_t (bitmamba.c_amd/host/bm_bit2.h)."""
    _fields_ = [("data", _fp), ("packed", _u8p), ("rows", _i), ("cols", _i),
                ("n_elements", _sz), ("is_bitnet", C.c_bool), ("scale", _f)]


class Bit2View(C.Structure):
    _fields_ = [("vocab", _i), ("d_model", _i), ("n_layers", _i), ("n_heads", _i),
                ("n_tensors", _i), ("tensors", C.POINTER(Bit2Tensor))]


class Dispatch(C.Structure):
    """Layout mirror of kernel_dispatch_t (src/dispatch.h:87-95)."""
    _fields_ = [("rms_norm", _vp), ("bitlinear_forward", _vp),
                ("bitlinear_forward_batch", _vp), ("bitlinear_prepare", _vp),
                ("bitlinear_row_worker", _vp), ("ssm_inner", _vp), ("name", C.c_char_p)]


# name -> (restype, argtypes); every symbol of include/bm_hip.h
SIGNATURES = {
    "bm_hip_init": (C.c_bool, []),
    "bm_hip_available": (C.c_bool, []),
    "bm_hip_set_mmap": (C.c_bool, [_vp, _sz]),
    "bm_hip_cleanup": (None, []),
    "bm_hip_last_error": (C.c_char_p, []),
    "hip_rms_norm": (_f, [_vp, _i, _vp, _vp]),
    "hip_bitlinear_forward": (None, [_vp, _i, C.POINTER(Tensor), C.POINTER(Tensor), _vp, _vp, _vp]),
    "hip_bitlinear_forward_batch": (None, [_vp, _i, _i, C.POINTER(Tensor), C.POINTER(Tensor),
                                           _vp, _vp, _vp, _i]),
    "bm_hip_register": (C.c_bool, [C.POINTER(Dispatch)]),
    "bm_hip_bitlinear_forward_batch": (None, [_vp, _i, _i, _vp, _i, _i, _f, _vp, _vp, _vp,
                                              _vp, _i]),
    "bm_hip_batch_begin": (_vp, [_i, _i, _i, _i, _i]),
    "bm_hip_batch_ptr": (_vp, [_vp, _i]),
    "bm_hip_encode_bitlinear": (C.c_bool, [_vp, _i, _i, _vp, _i, _i, _f, _vp, _i]),
    "bm_hip_encode_residual": (None, [_vp, _i]),
    "bm_hip_submit_and_wait": (None, [_vp]),
    "bm_hip_batch_end": (None, [_vp]),
    "bm_hip_malloc": (_vp, [_sz]),
    "bm_hip_free": (None, [_vp]),
    "bm_hip_memcpy_h2d": (_i, [_vp, _vp, _sz]),
    "bm_hip_memcpy_d2h": (_i, [_vp, _vp, _sz]),
    "bm_hip_memset": (_i, [_vp, _i, _sz]),
    "bm_hip_synchronize": (_i, []),
    "bm_hip_canonicalize_dev": (_i, [_vp, _sz, _vp]),
    "bm_hip_stream": (_vp, []),
    "bm_hip_event_create": (_vp, []),
    "bm_hip_event_destroy": (None, [_vp]),
    "bm_hip_event_record": (_i, [_vp, _vp]),
    "bm_hip_event_elapsed_ms": (_f, [_vp, _vp]),
    "bm_hip_copy_dev": (_i, [_vp, _vp, _sz, _vp]),
    "bm_hip_mfma_peak_dev": (_i, [_i, _i, _i, _vp, _vp]),
    "bm_hip_act_bytes": (_sz, [_i, _i]),
    "bm_hip_quantize_dev": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp]),
    "bm_hip_quantize_fast_dev": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp]),
    "bm_hip_bitlinear_act_dev": (_i, [_vp, _vp, _i, _vp, _i, _i, _f, _i, _vp, _vp]),
    "bm_hip_bitlinear_dev": (_i, [_vp, _i, _i, _vp, _vp, _i, _f, _i, _vp, _vp, _i, _vp, _vp,
                                  _vp]),
    "bm_hip_bitlinear_noalloc_dev": (_i, [_vp, _i, _i, _vp, _vp, _i, _f, _i, _vp, _vp]),
    "bm_hip_noalloc_scratch_bytes": (_sz, []),
    "bm_hip_i8_act_bytes": (_sz, [_i, _i]),
    "bm_hip_ternary_gemm_i32_dev": (_i, [_vp, _i, _i, _vp, _i, _i, _i, _vp, _vp, _vp]),
    "bm_hip_model_load": (_vp, [_vp, _sz]),
    "bm_hip_model_free": (None, [_vp]),
    "bm_hip_model_config": (_i, [_vp, _i]),
    "bm_hip_model_reset": (_i, [_vp]),
    "bm_hip_model_prefill": (_i, [_vp, _vp, _i]),
    "bm_hip_model_step": (_i, [_vp, _i, _vp, _i, _f]),
    "bm_hip_model_set_sampler": (_i, [_vp, _f, _f, _f, _i]),
    "bm_hip_model_set_fast": (_i, [_vp, _i]),
    "bm_hip_model_time_kernel": (_i, [_vp, _i, _i, _i, _vp]),
    "bm_hip_model_seed": (_i, [_vp, _u64]),
    "bm_hip_sample_workspace_bytes": (_sz, [_i]),
    "bm_hip_sample_advanced": (_i, [_vp, _i, _f, _f, _f, _i, _vp, _vp, _vp, _vp]),
    "bm_hip_model_state_bytes": (_sz, [_vp]),
    "bm_hip_model_state_save": (_i, [_vp, _vp, _sz]),
    "bm_hip_model_state_load": (_i, [_vp, _vp, _sz]),
    "bm_hip_model_logits": (_i, [_vp, _vp]),
    "bm_hip_model_layer_state": (_i, [_vp, _i, _vp, _vp]),
    "bm_hip_model_set_layer_state": (_i, [_vp, _i, _vp, _vp, _i]),
    "bm_hip_model_generate": (_i, [_vp, _vp, _i, _i, _f, _i, _vp, C.POINTER(C.c_double)]),
    "bm_hip_model_decode": (_i, [_vp, _i, _f, C.POINTER(C.c_double)]),
    "bm_hip_model_tokens": (_i, [_vp, _vp, _i]),
    "bm_hip_libm_eval_dev": (_i, [_i, _vp, _vp, _sz, _vp]),
    "bm_bit2_parse": (_i, [_vp, _sz, C.POINTER(Bit2View)]),
    "bm_bit2_view_free": (None, [C.POINTER(Bit2View)]),
    "bm_bit2_synth_size": (_sz, [C.POINTER(SynthConfig)]),
    "bm_bit2_synth_write": (_i, [C.POINTER(SynthConfig), _vp, _sz]),
    "bm_synth_ternary": (None, [_u64, _i, _i, _i, _i, _vp]),
    "bm_synth_normal": (None, [_u64, _i, _sz, _f, _vp]),
    "bm_synth_int8": (None, [_u64, _i, _sz, _vp]),
    "bm_synth_prompt": (None, [_u64, _i, _i, _vp]),
}

SYNTH_UNIFORM, SYNTH_P0_40, SYNTH_P0_60, SYNTH_RAW_BYTES = 0, 1, 2, 3

_lib = None


def lib():
    """The loaded library with argtypes set (raises if it was never built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("%s is not built; run __graft_entry__.build()" % LIB_PATH)
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error():
    return (lib().bm_hip_last_error() or b"").decode()


def ptr(a):
    return a.ctypes.data_as(_vp)


def check(rc, what="call"):
    if rc != 0:
        raise RuntimeError("%s failed (%d): %s" % (what, rc, last_error()))


# ---------------------------------------------------------------------------
# synthetic data (host side, no GPU needed)
# ---------------------------------------------------------------------------
def synth_ternary(seed, tensor, rows, cols, dist=SYNTH_UNIFORM):
    out = np.empty((rows, (cols + 3) // 4), dtype=np.uint8)
    lib().bm_synth_ternary(seed, tensor, rows, cols, dist, ptr(out))
    return out


def synth_normal(seed, tensor, shape, sigma=1.0):
    out = np.empty(shape, dtype=np.float32)
    lib().bm_synth_normal(seed, tensor, out.size, sigma, ptr(out))
    return out


def synth_int8(seed, tensor, shape):
    out = np.empty(shape, dtype=np.int8)
    lib().bm_synth_int8(seed, tensor, out.size, ptr(out))
    return out


def synth_prompt(seed, vocab, n):
    out = np.empty(n, dtype=np.int32)
    lib().bm_synth_prompt(seed, vocab, n, ptr(out))
    return out


def synth_model(vocab, d_model, n_layers, n_heads, seed, dist=SYNTH_UNIFORM, fp_sigma=0.02,
                ternary_scale=0.02, in_proj_rows=0):
    cfg = SynthConfig(vocab, d_model, n_layers, n_heads, in_proj_rows, dist, fp_sigma,
                      ternary_scale, seed)
    n = lib().bm_bit2_synth_size(C.byref(cfg))
    if n == 0:
        raise ValueError("invalid synthetic model config")
    buf = np.empty(n, dtype=np.uint8)
    check(lib().bm_bit2_synth_write(C.byref(cfg), ptr(buf), n), "bm_bit2_synth_write")
    return buf


BM_L_IN_NORM, BM_L_IN_PROJ, BM_L_OUT_NORM, BM_L_OUT_PROJ = 0, 1, 7, 8  # bm_bit2.h


def image_tensors(blob, layer, which):
    """struct tensor views (pointing into blob) of one layer entry of a
    BIT2 image: the reference's model_load view of the same bytes."""
    v = Bit2View()
    check(lib().bm_bit2_parse(ptr(blob), blob.nbytes, C.byref(v)), "bm_bit2_parse")
    try:
        t = v.tensors[1 + 9 * layer + which]
        return Tensor(t.data, t.packed, t.rows, t.cols, t.n_elements, t.is_bitnet, t.scale)
    finally:
        lib().bm_bit2_view_free(C.byref(v))


# ---------------------------------------------------------------------------
# device buffers
# ---------------------------------------------------------------------------
class DeviceBuffer:
    """A device allocation owned by the library's allocator."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = lib().bm_hip_malloc(max(self.nbytes, 1))
        if not self.ptr:
            raise MemoryError("bm_hip_malloc(%d): %s" % (self.nbytes, last_error()))

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().bm_hip_memcpy_h2d(self.ptr, ptr(a), a.nbytes), "h2d")

    def download(self, shape, dtype):
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(lib().bm_hip_memcpy_d2h(ptr(out), self.ptr, out.nbytes), "d2h")
        return out

    def free(self):
        if self.ptr:
            lib().bm_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sample_advanced(logits, temp, min_p=0.0, top_p=1.0, top_k=0, rng=0x853c49e6748fea9b):
    """sample_advanced (src/model.c:132-361) on the device for host logits:
    returns (token, the logits as the sampler leaves them, the next
    XorShift64* state)."""
    lg = np.ascontiguousarray(logits, np.float32)
    V = lg.size
    L = lib()
    bl = DeviceBuffer.from_array(lg)
    br = DeviceBuffer.from_array(np.array([rng], np.uint64))
    bw = DeviceBuffer(L.bm_hip_sample_workspace_bytes(V))
    bt = DeviceBuffer(4)
    try:
        check(L.bm_hip_sample_advanced(bl.ptr, V, temp, min_p, top_p, top_k, br.ptr, bw.ptr,
                                       bt.ptr, L.bm_hip_stream()), "sample_advanced")
        check(L.bm_hip_synchronize(), "synchronize")
        return (int(bt.download((1,), np.int32)[0]), bl.download((V,), np.float32),
                int(br.download((1,), np.uint64)[0]))
    finally:
        for b in (bl, br, bw, bt):
            b.free()


def make_tensor(packed=None, rows=0, cols=0, scale=1.0, data=None):
    t = Tensor()
    if packed is not None:
        t.packed_data = packed.ctypes.data_as(_u8p)
        t.is_bitnet = True
        t.rows, t.cols, t.scale = rows, cols, scale
        t.n_elements = rows * cols
    if data is not None:
        t.data = data.ctypes.data_as(_fp)
        t.rows = data.shape[0]
        t.n_elements = data.size
        t.scale = 1.0
    return t


class Model:
    """Device-resident model loaded from a BIT2 image (numpy uint8 array)."""

    def __init__(self, image):
        self.image = image  # the library copies it; kept for the caller's convenience
        self.h = lib().bm_hip_model_load(ptr(image), image.nbytes)
        if not self.h:
            raise RuntimeError("bm_hip_model_load: " + last_error())
        L = lib()
        self.vocab, self.d_model, self.n_layers, self.n_heads, self.d_inner = (
            L.bm_hip_model_config(self.h, i) for i in range(5))

    def generate(self, prompt, n_steps, penalty=1.0, stop_on_eos=False):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.empty(max(n_steps, 1), np.int32)
        ms = C.c_double(0.0)
        n = lib().bm_hip_model_generate(self.h, ptr(prompt), prompt.size, n_steps, penalty,
                                        int(stop_on_eos), ptr(out), C.byref(ms))
        if n < 0:
            raise RuntimeError("generate: " + last_error())
        return out[:n].copy(), ms.value

    def set_fast(self, on):
        check(lib().bm_hip_model_set_fast(self.h, int(bool(on))), "set_fast")

    def time_kernel(self, which, layer=0, reps=50):
        """Average microseconds per launch of one decode kernel (0 in_proj +
        SSM, 1 out_proj, 2 LM head) of `layer`, or of the layers in turn
        (layer -1); changes the state: reset afterwards."""
        us = C.c_float(0.0)
        check(lib().bm_hip_model_time_kernel(self.h, which, layer, reps, C.byref(us)),
              "time_kernel")
        return float(us.value)

    def prefill(self, tokens):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        check(lib().bm_hip_model_prefill(self.h, ptr(tokens), tokens.size), "prefill")

    def step(self, token, history, penalty=1.0):
        h = np.ascontiguousarray(history, dtype=np.int32)
        r = lib().bm_hip_model_step(self.h, int(token), ptr(h), h.size, penalty)
        if r < 0:
            raise RuntimeError("step: " + last_error())
        return r

    def set_sampler(self, temp=0.0, min_p=0.0, top_p=1.0, top_k=0):
        check(lib().bm_hip_model_set_sampler(self.h, temp, min_p, top_p, top_k), "set_sampler")

    def seed(self, seed):
        check(lib().bm_hip_model_seed(self.h, seed), "seed")

    def state_save(self):
        """The recurrent state as a BMST image (bytes)."""
        n = lib().bm_hip_model_state_bytes(self.h)
        buf = np.empty(n, np.uint8)
        if lib().bm_hip_model_state_save(self.h, ptr(buf), n) != n:
            raise RuntimeError("state_save: " + last_error())
        return buf.tobytes()

    def state_load(self, image):
        """Loads a BMST image; False (with bm_hip_last_error) if rejected."""
        buf = np.frombuffer(image, np.uint8).copy()
        return lib().bm_hip_model_state_load(self.h, ptr(buf), buf.size) == 0

    def logits(self):
        out = np.empty(self.vocab, np.float32)
        check(lib().bm_hip_model_logits(self.h, ptr(out)), "logits")
        return out

    def layer_state(self, layer):
        cs = np.empty((3, self.d_inner), np.float32)
        ss = np.empty(self.d_inner, np.float32)
        pos = lib().bm_hip_model_layer_state(self.h, layer, ptr(cs), ptr(ss))
        return cs, ss, pos

    def decode(self, n_steps, penalty=1.0):
        ms = C.c_double(0.0)
        check(lib().bm_hip_model_decode(self.h, n_steps, penalty, C.byref(ms)), "decode")
        return ms.value

    def tokens(self, n):
        out = np.empty(n, np.int32)
        n = lib().bm_hip_model_tokens(self.h, ptr(out), n)
        return out[:n]

    def reset(self):
        check(lib().bm_hip_model_reset(self.h), "reset")

    def free(self):
        if self.h:
            lib().bm_hip_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
