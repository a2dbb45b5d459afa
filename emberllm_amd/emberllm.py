"""Python binding over libember.so with the reference binding's API.

``Ember`` keeps the class surface of bindings/python/emberllm.py:112-201
(constructor arguments, ``encode``, ``decode``, ``generate``,
``generate_str``, ``close``, context management); it samples through the
library's ember_sample rather than in Python.
``Engine`` is the numpy-level view used by the tests and the benchmark.
"""
import ctypes
import numpy as np

from . import _native

_libc = ctypes.CDLL(None)
_libc.free.argtypes = [ctypes.c_void_p]


class Engine:
    """A loaded model and one device state, with numpy results."""

    def __init__(self, path, ctx=0, kv_fp16=False):
        self.lib = _native.lib()
        self.m = self.lib.ember_model_load(path.encode())
        if not self.m:
            raise RuntimeError(f"failed to load model: {path}")
        self.header = self.lib.ember_model_header(self.m).contents
        self.st = self.lib.ember_state_new_ex(self.m, int(ctx), 1 if kv_fp16 else 0)
        maxs = self.header.max_seq_len
        self.ctx = maxs if ctx <= 0 or ctx > maxs else ctx
        self.vocab = self.header.vocab_size
        self.kv_fp16 = bool(kv_fp16)
        self.dev = self.lib.ember_state_device(self.st)

    def forward(self, tok, pos):
        p = self.lib.ember_forward(self.m, self.st, int(tok), int(pos))
        return np.ctypeslib.as_array(p, shape=(self.vocab,)).copy()

    def prefill(self, ids, start=0):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        p = self.lib.ember_prefill(self.m, self.st, a.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                                   len(a), int(start))
        return np.ctypeslib.as_array(p, shape=(self.vocab,)).copy()

    def kv_row_bytes(self):
        h = self.header
        return h.n_kv_heads * h.head_dim * (2 if self.kv_fp16 else 4)

    def kv_read(self, which, layer, n_pos):
        out = np.empty(n_pos * self.kv_row_bytes(), dtype=np.uint8)
        if self.lib.ehip_kv_read(self.dev, which, layer, n_pos, out.ctypes.data) != 0:
            raise RuntimeError(_native.last_error())
        return out

    def kv_write(self, which, layer, data):
        data = np.ascontiguousarray(data, dtype=np.uint8)
        n_pos = data.size // self.kv_row_bytes()
        if self.lib.ehip_kv_write(self.dev, which, layer, n_pos, data.ctypes.data) != 0:
            raise RuntimeError(_native.last_error())

    def debug_buffer(self, which, n):
        out = np.empty(n, dtype=np.float32)
        if self.lib.ehip_debug_buffer(self.dev, which, out.ctypes.data, out.nbytes) != 0:
            raise RuntimeError(_native.last_error())
        return out

    def set_graph(self, on):
        self.lib.ehip_set_graph_mode(self.dev, 1 if on else 0)

    def decode_fusion(self):
        """Bit 0: the attention kernel merges its chunks itself
        (ehip_decode_fusion)."""
        return self.lib.ehip_decode_fusion(self.dev)

    def time_decode(self, pos0, steps):
        ms = ctypes.c_float()
        if self.lib.ehip_time_decode(self.dev, int(pos0), int(steps), ctypes.byref(ms)) != 0:
            raise RuntimeError(_native.last_error())
        return ms.value

    def generate_greedy(self, tok, pos, n):
        """Greedy decode of n tokens held on the device; returns (tokens, ms)."""
        out = np.zeros(n, dtype=np.int32)
        ms = ctypes.c_float()
        rc = self.lib.ehip_generate_greedy(self.dev, int(tok), int(pos), int(n),
                                           out.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                                           ctypes.byref(ms))
        if rc != 0:
            raise RuntimeError(_native.last_error())
        return out, ms.value

    def sample(self, logits, sampler):
        """ember_sample on the device (ehip_sample); `sampler` is an
        _native.EmberSampler, updated in place."""
        x = np.ascontiguousarray(logits, dtype=np.float32)
        tok = ctypes.c_int()
        if self.lib.ehip_sample(self.dev, x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), len(x),
                                ctypes.byref(sampler), ctypes.byref(tok)) != 0:
            raise RuntimeError(_native.last_error())
        return tok.value

    def generate_sampled(self, tok, pos, n, sampler):
        """Decode + device sampler loop held on the device; returns (tokens, ms)."""
        out = np.zeros(n, dtype=np.int32)
        ms = ctypes.c_float()
        if self.lib.ehip_generate_sampled(self.dev, int(tok), int(pos), int(n), ctypes.byref(sampler),
                                          out.ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                                          ctypes.byref(ms)) != 0:
            raise RuntimeError(_native.last_error())
        return out, ms.value

    def time_kernel(self, kernel, pos, reps):
        ms = ctypes.c_float()
        if self.lib.ehip_time_kernel(self.dev, int(kernel), int(pos), int(reps), ctypes.byref(ms)) != 0:
            raise RuntimeError(_native.last_error())
        return ms.value

    def measure_read_bw(self, nbytes=1 << 30, reps=10):
        """Measured streaming read bandwidth of the GPU in GB/s."""
        gbs = ctypes.c_float()
        if self.lib.ehip_measure_read_bw(self.dev, int(nbytes), int(reps), ctypes.byref(gbs)) != 0:
            raise RuntimeError(_native.last_error())
        return gbs.value

    def close(self):
        if getattr(self, "st", None):
            self.lib.ember_state_free(self.st)
            self.st = None
        if getattr(self, "m", None):
            self.lib.ember_model_free(self.m)
            self.m = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Ember:
    """A loaded model plus its tokenizer and one reusable run state."""

    def __init__(self, path, ctx=0, kv_fp16=False):
        self._lib = _native.lib()
        self.m = self._lib.ember_model_load(path.encode())
        if not self.m:
            raise RuntimeError(f"failed to load model: {path}")
        self.header = self._lib.ember_model_header(self.m).contents
        self.tok = self._lib.ember_tokenizer_new(self.m)
        self.st = self._lib.ember_state_new_ex(self.m, int(ctx), 1 if kv_fp16 else 0)
        maxs = self.header.max_seq_len
        self.ctx = maxs if ctx <= 0 or ctx > maxs else ctx

    def encode(self, text, add_bos=True):
        out = ctypes.POINTER(ctypes.c_int)()
        n = self._lib.ember_encode(self.tok, text.encode(), 1 if add_bos else 0, ctypes.byref(out))
        ids = [out[i] for i in range(n)]
        _libc.free(ctypes.cast(out, ctypes.c_void_p))
        return ids

    def decode(self, prev, tok):
        s = self._lib.ember_decode(self.tok, prev, tok)
        return s.decode("utf-8", "replace") if s else ""

    def generate(self, prompt, max_tokens=128, temperature=0.0, top_k=0, seed=None):
        """Yield decoded text pieces one token at a time.

        Sampling runs in the library (ember_sample) on the returned logits,
        with top-p off; `seed` seeds its xorshift64* stream.
        """
        ids = self.encode(prompt)
        if len(ids) >= self.ctx:
            ids = ids[: self.ctx - 1]
        arr = (ctypes.c_int * len(ids))(*ids)
        smp = _native.EmberSampler()
        self._lib.ember_sampler_init(ctypes.byref(smp), float(temperature), 1.0, int(top_k),
                                     int(seed or 0) & 0xFFFFFFFFFFFFFFFF)
        stops = {self.header.eos_token_id, self.header.eos_token_id2, self.header.bos_token_id}
        logits = self._lib.ember_prefill(self.m, self.st, arr, len(ids), 0)
        prev, pos = ids[-1], len(ids)
        try:
            for _ in range(max_tokens):
                nxt = self._lib.ember_sample(ctypes.byref(smp), logits, self.header.vocab_size)
                if nxt in stops:
                    return
                yield self.decode(prev, nxt)
                prev = nxt
                if pos >= self.ctx - 1:
                    return
                logits = self._lib.ember_forward(self.m, self.st, nxt, pos)
                pos += 1
        finally:
            self._lib.ember_sampler_free(ctypes.byref(smp))

    def generate_str(self, prompt, **kw):
        return "".join(self.generate(prompt, **kw))

    def close(self):
        if getattr(self, "st", None):
            self._lib.ember_state_free(self.st)
            self.st = None
        if getattr(self, "tok", None):
            self._lib.ember_tokenizer_free(self.tok)
            self.tok = None
        if getattr(self, "m", None):
            self._lib.ember_model_free(self.m)
            self.m = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
