"""Pins the oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against something independent of its own
formula: the compiled reference's golden vectors (tests/golden, written by
make_golden.py from the reference's own sources), numpy's IEEE fp16, exact
integer brute force, float64 bounds, hand-computed cases and invariants.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle
from emberllm_amd import configs

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")
O = oracle.oracle_lib()


def gold(name):
    return np.load(os.path.join(GOLD, name))


# ------------------------------------------------------------------ fp16 ---
def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([O.orc_f16_to_f32(int(v)) for v in h], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32)[~np.isnan(want)], want.view(np.uint32)[~np.isnan(want)])
    assert np.all(np.isnan(got[np.isnan(want)]))


def test_f32_to_f16_matches_ieee_rne():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    edge = np.array([65504, 65519.996, 65520, 2**-14, 2**-24, 2**-25, 1.5 * 2**-25, 2**-25 + 2**-40,
                     1 + 2**-11, 1 + 3 * 2**-11, -0.0, np.inf, -np.inf], dtype=np.float32)
    x = np.concatenate([x, edge])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    got = np.array([O.orc_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, want)


def test_f32_to_f16_reference_golden():
    g = gold("f16.npz")
    got = np.array([O.orc_f32_to_f16(float(v)) for v in g["x"]], dtype=np.uint16)
    assert np.array_equal(got, g["h"])


# ----------------------------------------------------------- quantizers ---
def quant(fn, x, blk):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(len(x) // 32 * blk, np.uint8)
    fn(oracle.f32p(x), out.ctypes.data, len(x))
    return out


def test_quantizers_reference_golden():
    g = gold("quant.npz")
    for i, row in enumerate(g["x"]):
        assert np.array_equal(quant(O.orc_quantize_q8_0, row, 34), g["q8"][i]), i
        assert np.array_equal(quant(O.orc_quantize_q4_0, row, 18), g["q4"][i]), i


def test_q8_closed_form():
    rng = np.random.default_rng(1)
    for scale in (1e-3, 1.0, 1e3):
        x = rng.normal(0, scale, 32).astype(np.float32)
        b = quant(O.orc_quantize_q8_0, x, 34)
        d = b[:2].view(np.float16)[0]
        q = b[2:].view(np.int8).astype(np.int64)
        i = int(np.argmax(np.abs(x)))
        assert q[i] == (127 if x[i] > 0 else -127)                 # largest element -> +-127
        assert d == np.float16(np.float32(np.abs(x).max()) / np.float32(127))
        inv = np.float32(1) / (np.float32(np.abs(x).max()) / np.float32(127))
        y = (x * inv).astype(np.float64)
        assert np.array_equal(q, np.clip(np.sign(y) * np.floor(np.abs(y) + 0.5), -127, 127))
    z = quant(O.orc_quantize_q8_0, np.zeros(32), 34)
    assert not z.any()                                              # zero block -> all zero


def test_q4_closed_form():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 1, 32).astype(np.float32)
    b = quant(O.orc_quantize_q4_0, x, 18)
    q = b[2:]
    codes = np.concatenate([q & 15, q >> 4]).astype(np.int64)     # element i low, i+16 high
    i = int(np.argmax(np.abs(x)))
    assert codes[i] == 0                                            # x*id = -8 -> nibble 0
    d = np.float32(x[i]) / np.float32(-8)
    inv = np.float32(1) / d
    want = np.clip(np.trunc((x * inv + np.float32(8.5)).astype(np.float64)), 0, 15)
    assert np.array_equal(codes, want)


# ------------------------------------------------------------ block dots ---
def test_block_dots_brute_force():
    rng = np.random.default_rng(3)
    for _ in range(200):
        w8 = rng.integers(-127, 128, 32).astype(np.int8)
        x8 = rng.integers(-127, 128, 32).astype(np.int8)
        wq = np.concatenate([np.zeros(2, np.uint8), w8.view(np.uint8)])
        xq = np.concatenate([np.zeros(2, np.uint8), x8.view(np.uint8)])
        assert O.orc_block_dot_q8(wq.ctypes.data, xq.ctypes.data) == int(np.dot(w8.astype(np.int64), x8))
        nib = rng.integers(0, 16, 32)
        w4 = np.concatenate([np.zeros(2, np.uint8), (nib[:16] | (nib[16:] << 4)).astype(np.uint8)])
        assert O.orc_block_dot_q4(w4.ctypes.data, xq.ctypes.data) == int(np.dot(nib - 8, x8.astype(np.int64)))


# ---------------------------------------------------------------- matmul ---
@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_matmul_float64_bound(dtype):
    rng = np.random.default_rng(4 + dtype)
    rows, cols = 48, 256
    W = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    x = rng.normal(0, 1, cols).astype(np.float32)
    if dtype == 0:
        wbytes, Wd, xd = W.copy(), W.astype(np.float64), x.astype(np.float64)
    else:
        blk = 34 if dtype == 1 else 18
        fn = O.orc_quantize_q8_0 if dtype == 1 else O.orc_quantize_q4_0
        wbytes = np.concatenate([quant(fn, r, blk) for r in W])
        Wd = np.zeros((rows, cols))
        for r in range(rows):
            for b in range(cols // 32):
                e = wbytes[(r * cols // 32 + b) * blk:(r * cols // 32 + b + 1) * blk]
                d = float(e[:2].view(np.float16)[0])
                if dtype == 1:
                    v = e[2:].view(np.int8).astype(np.float64)
                else:
                    v = np.concatenate([e[2:] & 15, e[2:] >> 4]).astype(np.float64) - 8
                Wd[r, b * 32:(b + 1) * 32] = v * d
        xq = quant(O.orc_quantize_q8_0, x, 34).reshape(-1, 34)
        xd = np.concatenate([e[2:].view(np.int8) * float(e[:2].view(np.float16)[0]) for e in xq])
    out = np.zeros(rows, np.float32)
    O.orc_matmul(oracle.f32p(out), oracle.f32p(x), wbytes.ctypes.data, dtype, cols, rows)
    want = Wd @ xd
    assert np.abs(out - want).max() <= 1e-5 * (np.abs(Wd) @ np.abs(xd)).max()


# ----------------------------------------------- forward / prefill goldens ---
@pytest.mark.parametrize("name", list(configs.TINY))
def test_forward_prefill_bit_exact_vs_reference(name):
    g = gold(f"tiny_{name}.npz")
    path = configs.model_path(name)
    assert configs.file_sha1(path) == str(g["sha1"])
    for kv16, key in ((False, "fp32"), (True, "fp16")):
        o = oracle.Oracle(path, kv_fp16=kv16)
        got = [o.prefill(g["ids"])] + [o.forward(int(t), len(g["ids"]) + i) for i, t in enumerate(g["toks"])]
        o.close()
        assert np.array_equal(np.array(got, np.float32), g[key]), (name, key)


@pytest.mark.parametrize("name", list(configs.TINY))
def test_prefill_equals_reference_sequential_forwards(name):
    """The reference's own invariant (model.c:283-360 vs 362-414): prefill's
    last logits equal the logits of feeding the prompt one forward at a time."""
    g = gold(f"tiny_{name}.npz")
    o = oracle.Oracle(configs.model_path(name))
    assert np.array_equal(o.prefill(g["ids"]), g["seq_forward"])
    o.close()


REAL_CPU = ["stories110m"] + (list(configs.REAL)[1:] if os.environ.get("EMBER_SLOW") else [])


@pytest.mark.parametrize("name", REAL_CPU)
def test_real_shape_reference_golden(name, oracle_threads):
    g = gold(f"real_{name}.npz")
    path = configs.model_path(name)
    assert configs.file_sha1(path) == str(g["sha1"])
    o = oracle.Oracle(path, ctx=len(g["ids"]) + len(g["toks"]) + 2)
    lg = [o.prefill(g["ids"])] + [o.forward(int(t), len(g["ids"]) + i) for i, t in enumerate(g["toks"])]
    o.close()
    lg = np.array(lg)
    top = np.argsort(-lg, axis=1, kind="stable")[:, :16]
    assert np.array_equal(top, g["top16"]) and np.array_equal(np.argmax(lg, 1), g["argmax"])
    assert np.array_equal(np.take_along_axis(lg, top, 1), g["top16_val"])
    assert np.array_equal(lg[:, ::509], g["sample"])


# --------------------------------------------------------------- sampler ---
def xorshift_star(state):
    x = state
    x ^= x >> 12
    x ^= (x << 25) & 0xFFFFFFFFFFFFFFFF
    x ^= x >> 27
    return x, ((x * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF) >> 32


def test_rng_closed_form():
    s = oracle.Sampler()
    O.orc_sampler_init(ctypes.byref(s), 1.0, 1.0, 0, 0)
    assert s.rng_state == 0x9E3779B97F4A7C15                      # seed 0 replaced
    st = s.rng_state
    for _ in range(100):
        st, out = xorshift_star(st)
        assert O.orc_rng_u32(ctypes.byref(s)) == out and s.rng_state == st


def test_sampler_hand_computed():
    s = oracle.Sampler()
    lg = np.array([1.0, 3.0, 3.0, 0.5, 2.0, -1.0, 0.0, 2.5, 1.5, 0.2], np.float32)
    O.orc_sampler_init(ctypes.byref(s), 0.0, 0.9, 0, 5)
    assert O.orc_sample(ctypes.byref(s), oracle.f32p(lg.copy()), 10) == 1   # first maximum
    # temperature 1, top-k 3: candidates {1, 2, 7} (ties keep index order)
    p = np.exp(lg - lg.max()) / np.exp(lg - lg.max()).sum()
    for seed in range(1, 40):
        O.orc_sampler_init(ctypes.byref(s), 1.0, 1.0, 3, seed)
        st, u = xorshift_star(seed)
        r = (u >> 8) / 16777216.0 * (p[1] + p[2] + p[7])
        want = 1 if r < p[1] else (2 if r < p[1] + p[2] else 7)
        assert O.orc_sample(ctypes.byref(s), oracle.f32p(lg.copy()), 10) == want
    # top-p 0.5 keeps the smallest prefix with mass >= 0.5: {1, 2}
    for seed in range(1, 40):
        O.orc_sampler_init(ctypes.byref(s), 1.0, 0.5, 0, seed)
        assert O.orc_sample(ctypes.byref(s), oracle.f32p(lg.copy()), 10) in (1, 2)


def test_sampler_reference_golden():
    g = gold("sampler.npz")
    V = g["logits"].shape[1]
    for k, (t, p, topk, seed, rp, ln, pr, fr, mp) in enumerate(g["settings"]):
        s = oracle.Sampler()
        O.orc_sampler_init(ctypes.byref(s), t, p, int(topk), int(seed))
        O.orc_sampler_set_penalties(ctypes.byref(s), rp, int(ln), pr, fr, mp)
        for i in range(g["logits"].shape[0]):
            row = np.ascontiguousarray(g["logits"][i].copy())
            assert O.orc_sample(ctypes.byref(s), oracle.f32p(row), V) == g["chosen"][k, i], (k, i)
            assert s.rng_state == g["states"][k, i]
        O.orc_sampler_free(ctypes.byref(s))
