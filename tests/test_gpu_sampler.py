"""GPU parity of the device sampler (ehip_sample, ehip_generate_sampled)
against ember_sample: the reference's own chosen tokens and RNG states
(tests/golden/sampler.npz, from the compiled reference: seven settings,
top_k 0, 5, 40 and 100 among them), and the host sampler (itself pinned to
the reference) on vocabulary-sized logits with ties.  top_k 1..64 takes the
bounded candidate path, top_k 0 or above 64 the whole-vocabulary sort and
sequential walk.  Chosen tokens and RNG states are integers and must match
exactly.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

from emberllm_amd import _native, configs, emberllm

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
L = None


def lib():
    global L
    if L is None:
        L = _native.lib()
    return L


def say(msg):
    print(f"[gpu-sampler] {msg}", flush=True)
    sys.stdout.flush()


def small_model(vocab):
    cfg = dict(configs.TINY["t_llama"], vocab_size=vocab, n_layers=1)
    return configs.model_path(f"samp_v{vocab}", cfg)


def sampler(temp, top_p, top_k, seed, rp=1.0, last_n=0, pres=0.0, freq=0.0, min_p=0.0):
    s = _native.EmberSampler()
    lib().ember_sampler_init(ctypes.byref(s), temp, top_p, int(top_k), int(seed))
    lib().ember_sampler_set_penalties(ctypes.byref(s), rp, int(last_n), pres, freq, min_p)
    return s


def test_device_sampler_reference_golden():
    g = np.load(os.path.join(GOLD, "sampler.npz"))
    V = g["logits"].shape[1]
    say(f"reference golden, vocab {V}")
    eng = emberllm.Engine(small_model(V))
    ran = 0
    for k, (t, p, topk, seed, rp, ln, pr, fr, mp) in enumerate(g["settings"]):
        s = sampler(t, p, topk, seed, rp, ln, pr, fr, mp)
        for i in range(g["logits"].shape[0]):
            c = eng.sample(g["logits"][i], s)
            assert c == g["chosen"][k, i] and s.rng_state == g["states"][k, i], (k, i, c, g["chosen"][k, i])
        lib().ember_sampler_free(ctypes.byref(s))
        ran += 1
    assert ran == len(g["settings"])
    eng.close()


@pytest.mark.parametrize("params", [
    dict(temp=0.8, top_p=0.9, top_k=40),
    dict(temp=1.0, top_p=1.0, top_k=1),
    dict(temp=0.7, top_p=0.95, top_k=64, min_p=0.05),
    dict(temp=1.3, top_p=0.8, top_k=20, rp=1.2, last_n=32, pres=0.3, freq=0.2),
    dict(temp=0.0, top_p=0.9, top_k=0, rp=1.5, last_n=8),
    dict(temp=0.8, top_p=0.9, top_k=0),
    dict(temp=1.0, top_p=1.0, top_k=0),
    dict(temp=0.6, top_p=0.8, top_k=100, min_p=0.02),
    dict(temp=1.1, top_p=0.97, top_k=1000, rp=1.2, last_n=32, pres=0.3, freq=0.2),
], ids=["t08p09k40", "k1", "minp", "penalties", "greedy-penalties", "k0", "k0-p1-whole-vocab",
        "k100-minp", "k1000-penalties"])
def test_device_sampler_matches_host_on_vocab_logits(params):
    V = 151936
    say(f"vocab {V}: {params}")
    eng = emberllm.Engine(small_model(V))
    rng = np.random.default_rng(11)
    p = dict(params)
    a = sampler(p.pop("temp"), p.pop("top_p"), p.pop("top_k"), 77, **p)
    b = sampler(params["temp"], params["top_p"], params["top_k"], 77,
                **{k: v for k, v in params.items() if k not in ("temp", "top_p", "top_k")})
    for step in range(24):
        lg = rng.normal(0, 3, V).astype(np.float32)
        lg[rng.integers(0, V, 64)] = lg[int(np.argmax(lg))]      # ties at the top
        x = lg.copy()
        host = lib().ember_sample(ctypes.byref(b), x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), V)
        dev = eng.sample(lg, a)
        assert dev == host and a.rng_state == b.rng_state, (step, dev, host)
        assert a.hist_len == b.hist_len and a.hist_pos == b.hist_pos
        assert [a.history[i] for i in range(a.hist_len)] == [b.history[i] for i in range(b.hist_len)]
    eng.close()


@pytest.mark.parametrize("top_k", [40, 64, 5])
def test_reference_order_sampler_takes_the_sequential_path(top_k, monkeypatch):
    """In the reference-order mode every top_k goes through the
    whole-vocabulary path, whose softmax sum and running sums are the
    reference's sequential ones (sample.c:131-133, 149-175): the device draws
    equal the host sampler's by construction, not only on these rows."""
    V = 151936
    monkeypatch.setenv("EHIP_ORDER", "reference")
    say(f"vocab {V}: reference order, top_k {top_k}")
    eng = emberllm.Engine(small_model(V))
    rng = np.random.default_rng(13)
    a = sampler(0.8, 0.9, top_k, 91)
    b = sampler(0.8, 0.9, top_k, 91)
    for step in range(24):
        lg = rng.normal(0, 3, V).astype(np.float32)
        lg[rng.integers(0, V, 16)] = lg[int(np.argmax(lg))]      # ties at the top
        x = lg.copy()
        host = lib().ember_sample(ctypes.byref(b), x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), V)
        dev = eng.sample(lg, a)
        assert dev == host and a.rng_state == b.rng_state, (step, dev, host)
    eng.close()


@pytest.mark.parametrize("top_k", [50, 0], ids=["k50", "k0"])
@pytest.mark.parametrize("kind", ["flat", "two-level", "quantized", "one-hot", "spread-ties"])
def test_device_sampler_degenerate_logits(kind, top_k):
    """Flat and heavily tied logits.  With top_k 50 many tokens share the
    bound, which sends the bounded path through its whole-vocabulary stream;
    "spread-ties" (514 tokens tied at the top, about 8 per slice) takes its
    bitonic sort of up to 1024.  With top_k 0 the ties are ordered by index
    in the full sort."""
    V = 151936
    say(f"vocab {V}: {kind} logits, top_k {top_k}")
    eng = emberllm.Engine(small_model(V))
    rng = np.random.default_rng(5)
    a = sampler(0.9, 0.95, top_k, 31)
    b = sampler(0.9, 0.95, top_k, 31)
    for step in range(4):
        if kind == "flat":
            lg = np.full(V, 0.25, np.float32)
        elif kind == "two-level":
            lg = np.where(rng.random(V) < 0.01, 1.0, 0.0).astype(np.float32)
        elif kind == "quantized":
            lg = (np.round(rng.normal(0, 2, V) * 2) / 2).astype(np.float32)
        elif kind == "spread-ties":
            lg = rng.normal(0, 1, V).astype(np.float32)
            lg[::296] = 10.0
        else:
            lg = np.full(V, -50.0, np.float32)
            lg[rng.integers(0, V)] = 50.0
        x = lg.copy()
        host = lib().ember_sample(ctypes.byref(b), x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), V)
        dev = eng.sample(lg, a)
        assert dev == host and a.rng_state == b.rng_state, (kind, step, dev, host)
    eng.close()


@pytest.mark.parametrize("top_k", [40, 0], ids=["k40", "k0"])
@pytest.mark.parametrize("penalties", [True, False], ids=["penalties", "plain"])
def test_generate_sampled_equals_host_loop(penalties, top_k):
    """ehip_generate_sampled = the generate loop of forward + ember_sample.
    Without penalties the lm_head's per-workgroup winners feed the sampler."""
    path = configs.model_path("t_qwen3")
    say(f"device sampling loop vs host loop, penalties {penalties}")
    a, b = emberllm.Engine(path), emberllm.Engine(path)
    ids = np.array([3, 77, 12, 500, 9], dtype=np.int32)
    a.prefill(ids)
    lg = b.prefill(ids)
    pen = dict(rp=1.1, last_n=16) if penalties else {}
    sa = sampler(0.8, 0.9, top_k, 4242, **pen)
    sb = sampler(0.8, 0.9, top_k, 4242, **pen)
    for t in ids:
        lib().ember_sampler_accept(ctypes.byref(sa), int(t))
        lib().ember_sampler_accept(ctypes.byref(sb), int(t))
    first = lib().ember_sample(ctypes.byref(sb), lg.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), len(lg))
    lib().ember_sampler_accept(ctypes.byref(sa), first)   # both loops have now taken `first`
    sa.rng_state = sb.rng_state
    n = 24
    dev, _ = a.generate_sampled(first, len(ids), n, sa)
    host, tok = [], first
    for i in range(n):
        lg = b.forward(tok, len(ids) + i)
        tok = lib().ember_sample(ctypes.byref(sb), lg.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), len(lg))
        host.append(tok)
    assert list(dev) == host, (list(dev), host)
    assert sa.rng_state == sb.rng_state
    a.close()
    b.close()
