"""ctypes access to the oracle (TEST INFRASTRUCTURE).

Loaded only by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
leg, as the checker or the timed CPU stand-in, never by the product.

  Oracle(...)       the CPU restatement in oracle.c (liboracle.so: the
                    reference's deterministic flags; liboracle_fast.so: its
                    optimized flags, for timing)
  Reference(...)    the reference library itself, compiled from its own
                    sources by ref.mk into oracle/_ref/ (present only where it
                    was built; where it is run, the built file comes along)
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_P = ctypes.c_void_p
_FP = ctypes.POINTER(ctypes.c_float)
_IP = ctypes.POINTER(ctypes.c_int)


class Sampler(ctypes.Structure):
    """EmberSampler / OrcSampler layout (src/ember.h:141-155)."""

    _fields_ = [
        ("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("top_k", ctypes.c_int),
        ("min_p", ctypes.c_float), ("repeat_penalty", ctypes.c_float),
        ("presence_penalty", ctypes.c_float), ("frequency_penalty", ctypes.c_float),
        ("repeat_last_n", ctypes.c_int), ("rng_state", ctypes.c_uint64),
        ("history", ctypes.POINTER(ctypes.c_int)),
        ("hist_cap", ctypes.c_int), ("hist_len", ctypes.c_int), ("hist_pos", ctypes.c_int),
    ]


_ORC = {
    "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "orc_expf_n": (None, [_FP, _FP, ctypes.c_long]),
    "orc_quantize_q8_0": (None, [_FP, _P, ctypes.c_int]),
    "orc_quantize_q4_0": (None, [_FP, _P, ctypes.c_int]),
    "orc_matmul": (None, [_FP, _FP, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "orc_matmul_batch": (None, [_FP, _FP, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "orc_block_dot_q8": (ctypes.c_int32, [_P, _P]),
    "orc_block_dot_q4": (ctypes.c_int32, [_P, _P]),
    "orc_model_open": (_P, [ctypes.c_char_p]),
    "orc_model_close": (None, [_P]),
    "orc_state_new": (_P, [_P, ctypes.c_int, ctypes.c_int]),
    "orc_state_free": (None, [_P]),
    "orc_state_ctx": (ctypes.c_int, [_P]),
    "orc_forward": (_FP, [_P, ctypes.c_int, ctypes.c_int]),
    "orc_prefill": (_FP, [_P, _IP, ctypes.c_int, ctypes.c_int]),
    "orc_kv_cache": (_P, [_P, ctypes.c_int]),
    "orc_capture": (None, [_P, ctypes.c_int, ctypes.POINTER(_FP)]),
    "orc_kv_bytes": (ctypes.c_uint64, [_P]),
    "orc_sampler_init": (None, [ctypes.POINTER(Sampler), ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_uint64]),
    "orc_sampler_set_penalties": (None, [ctypes.POINTER(Sampler), ctypes.c_float, ctypes.c_int,
                                         ctypes.c_float, ctypes.c_float, ctypes.c_float]),
    "orc_sampler_accept": (None, [ctypes.POINTER(Sampler), ctypes.c_int]),
    "orc_sampler_free": (None, [ctypes.POINTER(Sampler)]),
    "orc_sample": (ctypes.c_int, [ctypes.POINTER(Sampler), _FP, ctypes.c_int]),
    "orc_rng_u32": (ctypes.c_uint32, [ctypes.POINTER(Sampler)]),
    "orc_threads_init": (None, [ctypes.c_int]),
    "orc_threads_shutdown": (None, []),
}

_REF = {
    "ember_model_load": (_P, [ctypes.c_char_p]),
    "ember_model_free": (None, [_P]),
    "ember_state_new_ex": (_P, [_P, ctypes.c_int, ctypes.c_int]),
    "ember_state_free": (None, [_P]),
    "ember_forward": (_FP, [_P, _P, ctypes.c_int, ctypes.c_int]),
    "ember_prefill": (_FP, [_P, _P, _IP, ctypes.c_int, ctypes.c_int]),
    "ember_quantize_q8_0": (None, [_FP, _P, ctypes.c_int]),
    "ember_quantize_q4_0": (None, [_FP, _P, ctypes.c_int]),
    "ember_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "ember_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "ember_matmul": (None, [_FP, _FP, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]),
    "ember_quantize_file": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int]),
    "ember_sampler_init": (None, [ctypes.POINTER(Sampler), ctypes.c_float, ctypes.c_float, ctypes.c_int, ctypes.c_uint64]),
    "ember_sampler_set_penalties": (None, [ctypes.POINTER(Sampler), ctypes.c_float, ctypes.c_int,
                                           ctypes.c_float, ctypes.c_float, ctypes.c_float]),
    "ember_sampler_accept": (None, [ctypes.POINTER(Sampler), ctypes.c_int]),
    "ember_sampler_free": (None, [ctypes.POINTER(Sampler)]),
    "ember_sample": (ctypes.c_int, [ctypes.POINTER(Sampler), _FP, ctypes.c_int]),
    "ember_threads_init": (None, [ctypes.c_int]),
    "ember_threads_shutdown": (None, []),
    "ember_tokenizer_new": (_P, [_P]),
    "ember_tokenizer_free": (None, [_P]),
    "ember_encode": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(_IP)]),
    "ember_decode": (ctypes.c_char_p, [_P, ctypes.c_int, ctypes.c_int]),
}


def _load(path, protos):
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built (make -C oracle)")
    h = ctypes.CDLL(path)
    for name, (res, args) in protos.items():
        f = getattr(h, name)
        f.restype, f.argtypes = res, args
    return h


_cache = {}


def oracle_lib(fast=False):
    key = "fast" if fast else "exact"
    if key not in _cache:
        _cache[key] = _load(os.path.join(HERE, "liboracle_fast.so" if fast else "liboracle.so"), _ORC)
    return _cache[key]


def reference_path(debug=True, v4=False):
    """debug: the `make debug` flags; else the optimized flags, built for
    x86-64-v3 (AVX2) or, with v4, x86-64-v4 (AVX-512)."""
    if debug:
        return os.path.join(HERE, "_ref", "libember_ref_debug.so")
    return os.path.join(HERE, "_ref", "libember_ref_v4.so" if v4 else "libember_ref.so")


def reference_lib(debug=True, v4=False):
    key = "ref_debug" if debug else ("ref_v4" if v4 else "ref")
    if key not in _cache:
        _cache[key] = _load(reference_path(debug, v4), _REF)
    return _cache[key]


def f32p(a):
    return a.ctypes.data_as(_FP)


def intp(a):
    return a.ctypes.data_as(_IP)


class Oracle:
    """One model + state of the CPU restatement."""

    def __init__(self, path, ctx=0, kv_fp16=False, fast=False):
        self.L = oracle_lib(fast)
        self.m = self.L.orc_model_open(path.encode())
        if not self.m:
            raise RuntimeError(f"oracle cannot open {path}")
        self.s = self.L.orc_state_new(self.m, int(ctx), 1 if kv_fp16 else 0)
        self.ctx = self.L.orc_state_ctx(self.s)
        with open(path, "rb") as f:
            hdr = f.read(256)
        self._hdr = np.frombuffer(hdr[16:48], dtype=np.int32)
        self.vocab = int(self._hdr[6])

    def forward(self, tok, pos):
        p = self.L.orc_forward(self.s, int(tok), int(pos))
        return np.ctypeslib.as_array(p, shape=(self.vocab,)).copy()

    def prefill(self, ids, start=0):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        p = self.L.orc_prefill(self.s, intp(a), len(a), int(start))
        return np.ctypeslib.as_array(p, shape=(self.vocab,)).copy()

    def capture(self, layer, n_tok=1, prefill=False):
        """Record `layer`'s vectors in the following calls (orc_capture) into
        numpy buffers for n_tok tokens; returns the list of six arrays (slot
        4 holds the w1|w3 products when prefill is True).  layer -1 stops."""
        hdr = self._hdr
        dim, hid, nh, nkv, hd = (int(hdr[i]) for i in (0, 1, 3, 4, 5))
        qd, kvd = nh * hd, nkv * hd
        widths = (dim, qd + 2 * kvd, qd, dim, 2 * hid if prefill else hid, dim)
        self._cap = [np.zeros((n_tok, w), dtype=np.float32) for w in widths]
        if layer < 0:
            self.L.orc_capture(self.s, -1, None)
            return None
        arr = (_FP * 6)(*[f32p(a) for a in self._cap])
        self._cap_ptrs = arr
        self.L.orc_capture(self.s, int(layer), arr)
        return self._cap

    def kv_bytes(self):
        return int(self.L.orc_kv_bytes(self.s))

    def kv(self, which):
        """The KV cache as a writable uint8 view [L*ctx*kv_dim*esize]."""
        p = self.L.orc_kv_cache(self.s, which)
        buf = (ctypes.c_uint8 * self.kv_bytes()).from_address(p)
        return np.frombuffer(buf, dtype=np.uint8)

    def close(self):
        if self.s:
            self.L.orc_state_free(self.s)
            self.s = None
        if self.m:
            self.L.orc_model_close(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Reference:
    """One model + state of the compiled reference library."""

    def __init__(self, path, ctx=0, kv_fp16=False, debug=True, v4=False):
        self.L = reference_lib(debug, v4)
        self.m = self.L.ember_model_load(path.encode())
        if not self.m:
            raise RuntimeError(f"reference cannot open {path}")
        self.s = self.L.ember_state_new_ex(self.m, int(ctx), 1 if kv_fp16 else 0)
        with open(path, "rb") as f:
            hdr = f.read(256)
        self.vocab = int(np.frombuffer(hdr[16:48], dtype=np.int32)[6])

    def forward(self, tok, pos):
        p = self.L.ember_forward(self.m, self.s, int(tok), int(pos))
        return np.ctypeslib.as_array(p, shape=(self.vocab,)).copy()

    def prefill(self, ids, start=0):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        p = self.L.ember_prefill(self.m, self.s, intp(a), len(a), int(start))
        return np.ctypeslib.as_array(p, shape=(self.vocab,)).copy()

    def close(self):
        if self.s:
            self.L.ember_state_free(self.s)
            self.s = None
        if self.m:
            self.L.ember_model_free(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
