"""ehip_sample_noalloc against ehip_sample, through libember.so's C ABI.

The allocation-free entry point runs ehip_sample's kernels with every
intermediate in one static device array.  Two calls in a row (the second on
a smaller vocabulary, with other sampler settings, so it reuses the array
the first left behind) must reproduce ehip_sample exactly: the same token,
the same advanced xorshift64* state, the same history ring, and the same
penalized logits.  Device buffers for the test come from the HIP runtime
that libember.so itself loaded (the entry point allocates none).
"""
import ctypes
import sys

import numpy as np
import pytest

from emberllm_amd import _native, configs, emberllm

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


def say(msg):
    print(f"[no-alloc] {msg}", flush=True)
    sys.stdout.flush()


def hip_runtime():
    """The libamdhip64 that libember.so is linked against (already loaded)."""
    _native.lib()
    with open("/proc/self/maps") as f:
        paths = {ln.split()[-1] for ln in f if "libamdhip64.so" in ln}
    assert paths, "libamdhip64 is not loaded"
    hip = ctypes.CDLL(sorted(paths)[0])
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipFree.argtypes = [ctypes.c_void_p]
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return hip


class DevBuf:
    def __init__(self, hip, host):
        self.hip, self.host = hip, np.ascontiguousarray(host)
        self.ptr = ctypes.c_void_p()
        assert hip.hipMalloc(ctypes.byref(self.ptr), max(1, self.host.nbytes)) == 0
        assert hip.hipMemcpy(self.ptr, self.host.ctypes.data, self.host.nbytes, H2D) == 0

    def read(self):
        out = np.empty_like(self.host)
        assert self.hip.hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, D2H) == 0
        return out

    def free(self):
        self.hip.hipFree(self.ptr)


def make_sampler(lib, temp, top_p, top_k, seed, hist):
    s = _native.EmberSampler()
    lib.ember_sampler_init(ctypes.byref(s), temp, top_p, top_k, seed)
    lib.ember_sampler_set_penalties(ctypes.byref(s), 1.3, 8, 0.2, 0.1, 0.05)
    for t in hist:
        lib.ember_sampler_accept(ctypes.byref(s), int(t))
    return s


def one_call(lib, hip, eng, logits, temp, top_p, top_k, seed, hist):
    n = len(logits)
    # the existing entry point
    sa = make_sampler(lib, temp, top_p, top_k, seed, hist)
    tok_a = eng.sample(logits, sa)
    pen_a = eng.debug_buffer(4, n)
    want = dict(tok=tok_a, rng=int(sa.rng_state), hist=[sa.history[i] for i in range(sa.hist_cap)],
                meta=(sa.hist_len, sa.hist_pos), logits=pen_a)
    # the allocation-free one, on device copies of the same inputs
    sb = make_sampler(lib, temp, top_p, top_k, seed, hist)
    d_log = DevBuf(hip, logits.astype(np.float32))
    d_rng = DevBuf(hip, np.array([sb.rng_state], dtype=np.uint64))
    d_hist = DevBuf(hip, np.array([sb.history[i] for i in range(sb.hist_cap)], dtype=np.int32))
    d_meta = DevBuf(hip, np.array([sb.hist_len, sb.hist_pos], dtype=np.int32))
    d_tok = DevBuf(hip, np.array([-1], dtype=np.int32))
    rc = lib.ehip_sample_noalloc(d_log.ptr, n, ctypes.byref(sb), d_rng.ptr, d_hist.ptr, d_meta.ptr, d_tok.ptr, None)
    assert rc == 0, _native.last_error()
    assert hip.hipDeviceSynchronize() == 0
    got = dict(tok=int(d_tok.read()[0]), rng=int(d_rng.read()[0]), hist=list(d_hist.read()),
               meta=tuple(int(v) for v in d_meta.read()), logits=d_log.read())
    for b in (d_log, d_rng, d_hist, d_meta, d_tok):
        b.free()
    lib.ember_sampler_free(ctypes.byref(sa))
    lib.ember_sampler_free(ctypes.byref(sb))
    return want, got


def test_noalloc_sampler_matches_ehip_sample():
    lib = _native.lib()
    hip = hip_runtime()
    path = configs.model_path("qwen3_06b", threads=16)
    eng = emberllm.Engine(path, ctx=64)
    V = eng.vocab
    rng = np.random.default_rng(99)
    cases = [  # (n, temperature, top_p, top_k, seed): the second call on fewer logits
        (V, 0.8, 0.9, 40, 1234),
        (100_000, 1.1, 0.95, 64, 77),
        (50_000, 0.0, 1.0, 0, 5),
    ]
    for n, temp, top_p, top_k, seed in cases:
        say(f"n={n} T={temp} top_p={top_p} top_k={top_k}")
        logits = (rng.standard_normal(n) * 3.0).astype(np.float32)
        logits[rng.integers(0, n, 50)] = logits.max()   # ties at the top
        hist = rng.integers(0, n, 6)
        want, got = one_call(lib, hip, eng, logits, temp, top_p, top_k, seed, hist)
        assert got["tok"] == want["tok"], (got["tok"], want["tok"])
        assert got["rng"] == want["rng"]
        assert got["meta"] == want["meta"]
        valid = want["meta"][0]   # ring slots past hist_len were never written on either side
        assert [int(v) for v in got["hist"][:valid]] == [int(v) for v in want["hist"][:valid]]
        np.testing.assert_array_equal(got["logits"], want["logits"])
    # sizes beyond the scratch array are refused before any launch
    big = np.zeros(262_145, dtype=np.float32)
    s = make_sampler(lib, 0.8, 0.9, 40, 1, [])
    rc = lib.ehip_sample_noalloc(ctypes.c_void_p(16), len(big), ctypes.byref(s), ctypes.c_void_p(16),
                                 None, None, ctypes.c_void_p(16), None)
    assert rc != 0 and "262144" in _native.last_error()
    lib.ember_sampler_free(ctypes.byref(s))
    eng.close()
