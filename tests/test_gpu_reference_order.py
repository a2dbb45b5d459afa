"""The reference-order mode (EHIP_ORDER=reference) against the oracle at the
target bar itself, on the benchmark shapes too.

With EHIP_ORDER=reference the state runs the decode step with kernels that
perform every fp32 operation of the reference in its order (reforder.hip:
sequential RMSNorm, block and softmax sums, P.V summed over positions in
order) and prefills as one decode step per token, which is what the
reference's prefill computes.  The deep shapes, which the fast kernels can
only match at the reference builds' own noise floor (~1e-2 relative L2, a
code an ulp decides cascading), are then held to 1e-2 max-abs and 1e-3
relative L2 at every step with >= 99% top-1 and no near-tie excuse: the
kernels' arithmetic is the reference's, and the fast path differs from it
only in summation order.  Through libember.so's C ABI; every case prints its
name before it touches the GPU.
"""
import sys

import numpy as np
import pytest

import oracle
from emberllm_amd import configs, emberllm
from parity import check_strict, compare

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-reference-order] {msg}", flush=True)
    sys.stdout.flush()


# (model, prompt, decode, ctx, fp16 cache): every benchmark shape (Q8_0 and
# Q4_0, bias, QK-norm, GQA, tied / untied, both RoPE pairings), a small F32
# model, an fp16 cache, and a 300-token prompt
CASES = [
    ("stories110m", 16, 24, 48, False), ("smollm2_135m", 16, 24, 48, False), ("qwen25_05b", 16, 24, 48, False),
    ("qwen3_06b", 16, 24, 48, False), ("qwen3_06b_q4", 16, 24, 48, False), ("qwen3_06b", 16, 24, 48, True),
    ("t_f32", 8, 16, 32, False), ("t_g7", 8, 16, 32, True), ("qwen3_06b", 300, 8, 316, False),
]


@pytest.mark.parametrize("name,prompt,decode,ctx,kv16", CASES,
                         ids=[f"{n}-p{p}-d{d}{'-f16kv' if k else ''}" for n, p, d, c, k in CASES])
def test_reference_order_meets_the_target_bar(name, prompt, decode, ctx, kv16, oracle_threads, monkeypatch):
    monkeypatch.setenv("EHIP_ORDER", "reference")
    path = configs.model_path(name, threads=16)
    V = configs.ALL[name]["vocab_size"]
    rng = np.random.default_rng(prompt + decode)
    ids, toks = rng.integers(0, V, prompt), rng.integers(0, V, decode)
    cid = f"{name}-p{prompt}-d{decode}{'-f16kv' if kv16 else ''}"
    say(cid)
    eng = emberllm.Engine(path, ctx=ctx, kv_fp16=kv16)
    orc = oracle.Oracle(path, ctx=ctx, kv_fp16=kv16)
    res = [compare(eng.prefill(ids), orc.prefill(ids))]
    for i, t in enumerate(toks):
        res.append(compare(eng.forward(int(t), prompt + i), orc.forward(int(t), prompt + i)))
    eng.close()
    orc.close()
    say(check_strict(res, cid))
