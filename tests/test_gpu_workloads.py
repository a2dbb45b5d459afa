"""The benchmark workloads, end to end on the GPU against the oracle
(the reference's bench protocol, src/main.c:230-294: a batched prefill of
random ids, then decode at that depth; teacher forced on the GPU's tokens).

  stories110M Q8_0   pp128, greedy tg128 @128
  SmolLM2-135M Q8_0  pp1024, greedy tg128 @1024
  Qwen2.5-0.5B Q8_0  pp256, sampled tg128 @256 (temperature 0.8, top-k 40,
                     top-p 0.9, fixed seed)
  Qwen3-0.6B Q8_0    pp128, greedy tg128 @128 (depth 4096: test_gpu_parity's
                     KV hand-over case and test_gpu_kernels)
  Qwen3-0.6B Q4_0    pp512, greedy tg256 @512

Each step's logits are compared with the oracle's.  The reference re-quantizes
every matmul input to Q8_0, so any reordered fp32 sum can move an activation
code and the logits of deep models then differ by ~1e-2 relative L2: the
reference's own optimized build differs from its deterministic one by as much
(tests/golden/noise_floor.json).  These end-to-end runs are therefore held to
the noise floor of the reference's two builds measured over the very same
workload protocol (the optimized build teacher forced on the deterministic
build's tokens; tests/parity.py), whose top-1 agreement there is 0.992,
1.000, 0.961, 0.946 and 0.984; the kernel-level bound (1e-6) is
test_gpu_kernels'.  The target figures (1e-3 relative L2, 1e-2 max-abs,
99% top-1) are printed beside the bars for every run.

The device-held loops must also reproduce the C-API loop exactly: the greedy
loop's tokens equal the argmax of ember_forward's logits, and the device
sampler's tokens equal ember_sample's (the host sampler, the reference's
algorithm) on the same logits.

Each workload also runs in the reference-order mode (EHIP_ORDER=reference:
the decode kernels of reforder.hip, every fp32 operation the reference's in
its order, prefill as one step per token), held to the target bar itself at
every step (tests/parity.py check_strict).
"""
import ctypes
import sys

import numpy as np
import pytest

import oracle
from emberllm_amd import _native, configs, emberllm
from parity import check_run, check_strict, compare

pytestmark = [pytest.mark.gpu, pytest.mark.slow]


def say(msg):
    print(f"[gpu-workload] {msg}", flush=True)
    sys.stdout.flush()


def target_view(res):
    rel = np.array([r["rel_l2"] for r in res])
    mab = np.array([r["max_abs"] for r in res])
    top = np.mean([r["agree"] for r in res])
    return (f"target-bar view: rel-L2 median {np.median(rel):.2e} (bar 1e-3), max-abs median "
            f"{np.median(mab):.2e} (bar 1e-2), top-1 {top:.3f} (bar 0.99)")


def _run(name, prompt, steps, sampled=False, reference_order=False):
    path = configs.model_path(name, threads=16)
    V = configs.ALL[name]["vocab_size"]
    rng = np.random.default_rng(prompt * 7 + steps)
    ids = rng.integers(0, V, prompt)
    ctx = prompt + steps + 2
    lib = _native.lib()
    say(f"{name} pp{prompt} tg{steps} {'sampled' if sampled else 'greedy'}{' reference order' if reference_order else ''}")
    eng = emberllm.Engine(path, ctx=ctx)
    orc = oracle.Oracle(path, ctx=ctx)
    first = eng.prefill(ids)
    res = [compare(first, orc.prefill(ids))]
    smp = _native.EmberSampler()
    if sampled:
        lib.ember_sampler_init(ctypes.byref(smp), 0.8, 0.9, 40, 1234)
        pick = lambda lg: lib.ember_sample(ctypes.byref(smp), lg.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                           len(lg))
    else:
        pick = lambda lg: int(np.argmax(lg))
    tok0 = pick(first.copy())
    toks, t = [], tok0
    for i in range(steps):
        pos = prompt + i
        lg = eng.forward(t, pos)
        res.append(compare(lg, orc.forward(t, pos)))
        t = pick(lg.copy())
        toks.append(t)
    eng.close()
    orc.close()
    # the device-held loop from the same start reproduces the API loop's tokens
    dev = emberllm.Engine(path, ctx=ctx)
    dev.prefill(ids)
    if sampled:
        lib.ember_sampler_free(ctypes.byref(smp))
        smp2 = _native.EmberSampler()
        lib.ember_sampler_init(ctypes.byref(smp2), 0.8, 0.9, 40, 1234)
        lib.ember_sample(ctypes.byref(smp2), first.copy().ctypes.data_as(ctypes.POINTER(ctypes.c_float)), V)
        got, _ = dev.generate_sampled(tok0, prompt, steps, smp2)
        lib.ember_sampler_free(ctypes.byref(smp2))
    else:
        got, _ = dev.generate_greedy(tok0, prompt, steps)
    dev.close()
    same = np.mean(np.asarray(got) == np.asarray(toks))
    say(f"{name}: device loop reproduces the API loop on {same * 100:.1f}% of {steps} tokens")
    assert same == 1.0, (list(got[:20]), toks[:20])
    if reference_order:
        say(check_strict(res, f"{name}-pp{prompt}-tg{steps}"))
        return
    say(target_view(res))
    # bars: the reference's optimized build against its deterministic build
    # over this same protocol (noise_floor.json, make_golden.py workload)
    say(check_run(res, f"{name}-pp{prompt}-tg{steps}"))


def test_stories110m_pp128_tg128(oracle_threads):
    _run("stories110m", 128, 128)


def test_smollm2_pp1024_tg128(oracle_threads):
    _run("smollm2_135m", 1024, 128)


def test_qwen25_pp256_sampled_tg128(oracle_threads):
    _run("qwen25_05b", 256, 128, sampled=True)


def test_qwen3_pp128_tg128(oracle_threads):
    _run("qwen3_06b", 128, 128)


def test_qwen3_q4_pp512_tg256(oracle_threads):
    _run("qwen3_06b_q4", 512, 256)


WORKLOADS = [("stories110m", 128, 128, False), ("smollm2_135m", 1024, 128, False), ("qwen25_05b", 256, 128, True),
             ("qwen3_06b", 128, 128, False), ("qwen3_06b_q4", 512, 256, False)]


@pytest.mark.parametrize("name,prompt,steps,sampled", WORKLOADS,
                         ids=[f"{n}-pp{p}-tg{t}{'-sampled' if s else ''}" for n, p, t, s in WORKLOADS])
def test_workload_reference_order(name, prompt, steps, sampled, oracle_threads, monkeypatch):
    monkeypatch.setenv("EHIP_ORDER", "reference")
    _run(name, prompt, steps, sampled=sampled, reference_order=True)
