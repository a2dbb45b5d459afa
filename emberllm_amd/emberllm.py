"""numpy-level view of libember.so for the tests and the benchmark.

``Engine`` holds one loaded model and one device state and returns numpy
arrays; besides the ember.h calls it reaches the device layer's loops and
measurement hooks (ehip.h).  Applications keep using the reference's own
ctypes binding (bindings/python/emberllm.py), which loads this library
unchanged through EMBER_LIB.
"""
import ctypes
import numpy as np

from . import _native


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

    def debug_capture(self, layer):
        """Record `layer`'s intermediate vectors in the following decode steps
        (-1 stops); see ehip_debug_capture."""
        if self.lib.ehip_debug_capture(self.dev, int(layer)) != 0:
            raise RuntimeError(_native.last_error())

    def debug_read(self, slot):
        """One recorded vector (ehip_debug_capture slot 0..5) as float32."""
        h = self.header
        qd, kvd = h.n_heads * h.head_dim, h.n_kv_heads * h.head_dim
        n = (h.dim, qd + 2 * kvd, qd, h.dim, h.hidden_dim, h.dim)[slot]
        out = np.empty(n, dtype=np.float32)
        if self.lib.ehip_debug_read(self.dev, int(slot), out.ctypes.data, out.nbytes) != 0:
            raise RuntimeError(_native.last_error())
        return out

    def debug_capture_prefill(self, layer, pass_index=0):
        """Record `layer` of prefill pass `pass_index` in the following
        prefills (-1 stops); see ehip_debug_capture_prefill."""
        if self.lib.ehip_debug_capture_prefill(self.dev, int(layer), int(pass_index)) != 0:
            raise RuntimeError(_native.last_error())

    def debug_read_prefill(self, slot):
        """(rows [n_tok][width] float32, first position) of a recorded slot."""
        h = self.header
        qd, kvd = h.n_heads * h.head_dim, h.n_kv_heads * h.head_dim
        width = (h.dim, qd + 2 * kvd, qd, h.dim, 2 * h.hidden_dim, h.dim)[slot]
        n, p0 = ctypes.c_int(), ctypes.c_int()
        if self.lib.ehip_debug_read_prefill(self.dev, int(slot), None, 0, ctypes.byref(n), ctypes.byref(p0)) != 0:
            raise RuntimeError(_native.last_error())
        out = np.empty((n.value, width), dtype=np.float32)
        if self.lib.ehip_debug_read_prefill(self.dev, int(slot), out.ctypes.data, out.nbytes, None, None) != 0:
            raise RuntimeError(_native.last_error())
        return out, p0.value

    def prefill_pass_tokens(self):
        return self.lib.ehip_prefill_pass_tokens(self.dev)

    def set_graph(self, on):
        self.lib.ehip_set_graph_mode(self.dev, 1 if on else 0)

    def decode_fusion(self):
        """Bit 0: the attention kernel merges its chunks itself; bit 1: it
        also computes the wo product (ehip_decode_fusion)."""
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
