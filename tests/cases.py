"""Parity cases shared by the GPU tests and the noise-floor fixture."""
from emberllm_amd import configs

TINY_GOLDEN_STEPS = (8, 4)    # prompt tokens, decode steps in tiny_<name>.npz
REAL_GOLDEN = (16, 4)         # the same for real_<name>.npz


def _case(name, kv16=False, prompt=8, decode=16, seed=0, ctx=0):
    cid = f"{name}{'-f16kv' if kv16 else ''}-p{prompt}-d{decode}-s{seed}"
    return dict(id=cid, name=name, kv_fp16=kv16, prompt=prompt, decode=decode, seed=seed, ctx=ctx)


GPU_CASES = (
    [_case(n) for n in configs.TINY]
    + [_case(n, kv16=True) for n in ("t_gqa", "t_qwen3", "t_g7", "t_q4")]
    + [_case("t_g7", prompt=300, decode=6, seed=3)]
    + [_case(n, prompt=16, decode=32, seed=11, ctx=50) for n in configs.REAL]
    + [_case("qwen3_06b", kv16=True, prompt=16, decode=32, seed=11, ctx=50)]
)
CASES = {c["id"]: c for c in GPU_CASES}
