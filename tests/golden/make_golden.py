"""Write the golden fixtures of tests/golden/ from the compiled reference.

Run in the authoring container, where oracle/ref.mk builds the reference's
own C sources (/root/reference/src) into oracle/_ref/.  The fixtures are
data only: inputs are regenerated from seeds by the package's synthetic model
writer, and every fixture records the sha1 of the model file it was made from.

  quant.npz        rows quantized by ember_quantize_q8_0 / _q4_0 (incl. edge rows)
  f16.npz          ember_f32_to_f16 on boundary floats
  sampler.npz      ember_sample choices and RNG states for seeded logits
  tiny_<name>.npz  full logits of ember_prefill + ember_forward (deterministic
                   build) on the small variant models, fp32 and fp16 KV
  real_<name>.npz  per step: argmax, top-16 ids/values, sum, sum of squares and
                   a 1-in-509 logit sample on the benchmark shapes
  noise_floor.json deviation of the reference's optimized build from its
                   deterministic build on the GPU parity cases (tolerance
                   calibration, see tests/parity.py)

Usage: python tests/golden/make_golden.py [quant f16 sampler tiny real noise wide workload]
"""
import ctypes
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]

import oracle  # noqa: E402
from emberllm_amd import configs  # noqa: E402
from parity import compare  # noqa: E402
from cases import GPU_CASES, TINY_GOLDEN_STEPS, REAL_GOLDEN  # noqa: E402


def ref():
    return oracle.reference_lib(debug=True)


def quant_fixture():
    L = ref()
    rng = np.random.default_rng(123)
    rows = [rng.normal(0, 0.02, 64), rng.normal(0, 1.0, 64), rng.normal(0, 300.0, 64),
            np.zeros(64), np.full(64, -0.75), np.linspace(-1, 1, 64),
            np.array([0.5, -0.5, 1.5, -2.5] * 16) * (127 / 2.5),        # exact ties at 1.0 scale
            np.concatenate([np.full(32, 1e-30), np.full(32, 6e4)]),     # tiny and near-fp16-max
            rng.standard_cauchy(64), rng.normal(0, 1e-6, 64)]
    rows += [rng.normal(0, s, 64) for s in (1e-3, 0.1, 7.0) for _ in range(10)]
    X = np.array(rows, dtype=np.float32)
    q8 = np.zeros((len(X), 2 * 34), np.uint8)
    q4 = np.zeros((len(X), 2 * 18), np.uint8)
    for i, r in enumerate(X):
        r = np.ascontiguousarray(r)
        L.ember_quantize_q8_0(oracle.f32p(r), q8[i].ctypes.data, 64)
        L.ember_quantize_q4_0(oracle.f32p(r), q4[i].ctypes.data, 64)
    np.savez_compressed(os.path.join(HERE, "quant.npz"), x=X, q8=q8, q4=q4)


def f16_fixture():
    L = ref()
    rng = np.random.default_rng(7)
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1035156e-05,
            6.0975552e-05, 5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1e-10, 0.1, 1.0 / 3]
    vals += list(rng.normal(0, 1, 2000)) + list(np.exp(rng.uniform(-25, 11, 2000)))
    x = np.array(vals, dtype=np.float32)
    h = np.array([L.ember_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    np.savez_compressed(os.path.join(HERE, "f16.npz"), x=x, h=h)


SAMPLER_SETTINGS = [
    # temp, top_p, top_k, seed, repeat_penalty, last_n, presence, frequency, min_p
    (0.0, 0.9, 0, 1, 1.0, 0, 0.0, 0.0, 0.0),
    (0.8, 0.9, 40, 12345, 1.0, 0, 0.0, 0.0, 0.0),
    (1.0, 1.0, 0, 7, 1.0, 0, 0.0, 0.0, 0.0),
    (0.7, 0.5, 0, 99, 1.0, 0, 0.0, 0.0, 0.0),
    (1.2, 0.95, 5, 3, 1.3, 16, 0.2, 0.1, 0.0),
    (0.9, 1.0, 0, 0, 1.0, 0, 0.0, 0.0, 0.05),
    (0.6, 0.8, 100, 2024, 1.1, 8, 0.0, 0.3, 0.02),
]


def sampler_fixture():
    L = ref()
    rng = np.random.default_rng(2)
    V, steps = 1024, 24
    logits = rng.normal(0, 2.0, (steps, V)).astype(np.float32)
    logits[:, 10] = logits[:, 11]          # exact ties exercise the candidate order
    chosen = np.zeros((len(SAMPLER_SETTINGS), steps), np.int32)
    states = np.zeros((len(SAMPLER_SETTINGS), steps), np.uint64)
    for k, (t, p, topk, seed, rp, ln, pr, fr, mp) in enumerate(SAMPLER_SETTINGS):
        s = oracle.Sampler()
        L.ember_sampler_init(ctypes.byref(s), t, p, topk, seed)
        L.ember_sampler_set_penalties(ctypes.byref(s), rp, ln, pr, fr, mp)
        for i in range(steps):
            row = np.ascontiguousarray(logits[i].copy())
            chosen[k, i] = L.ember_sample(ctypes.byref(s), oracle.f32p(row), V)
            states[k, i] = s.rng_state
        L.ember_sampler_free(ctypes.byref(s))
    np.savez_compressed(os.path.join(HERE, "sampler.npz"), logits=logits, chosen=chosen, states=states,
                        settings=np.array(SAMPLER_SETTINGS, dtype=np.float64))


def run_ref(path, ids, toks, kv16, ctx, debug=True):
    r = oracle.Reference(path, ctx=ctx, kv_fp16=kv16, debug=debug)
    out = [r.prefill(ids)]
    for i, t in enumerate(toks):
        out.append(r.forward(int(t), len(ids) + i))
    r.close()
    return np.array(out)


def tiny_fixture():
    n_prompt, n_dec = TINY_GOLDEN_STEPS
    for name in configs.TINY:
        path = configs.model_path(name)
        V = configs.TINY[name]["vocab_size"]
        rng = np.random.default_rng(5)
        ids = rng.integers(0, V, n_prompt).astype(np.int32)
        toks = rng.integers(0, V, n_dec).astype(np.int32)
        seq = np.array([ref_forward_seq(path, ids)], dtype=np.float32)
        np.savez_compressed(
            os.path.join(HERE, f"tiny_{name}.npz"), ids=ids, toks=toks,
            fp32=run_ref(path, ids, toks, False, 0).astype(np.float32),
            fp16=run_ref(path, ids, toks, True, 0).astype(np.float32),
            seq_forward=seq[0], sha1=configs.file_sha1(path))
        print("tiny", name, flush=True)


def ref_forward_seq(path, ids):
    """The reference's logits after feeding `ids` one forward at a time."""
    r = oracle.Reference(path, debug=True)
    for p, t in enumerate(ids):
        last = r.forward(int(t), p)
    r.close()
    return last


def summarize(logits):
    top = np.argsort(-logits, axis=1, kind="stable")[:, :16]
    return dict(argmax=np.argmax(logits, axis=1), top16=top,
                top16_val=np.take_along_axis(logits, top, axis=1),
                sum=logits.astype(np.float64).sum(1), sumsq=(logits.astype(np.float64) ** 2).sum(1),
                sample=logits[:, ::509])


def real_fixture():
    L = ref()
    L.ember_threads_init(min(8, os.cpu_count() or 1))
    n_prompt, n_dec = REAL_GOLDEN
    for name in configs.REAL:
        path = configs.model_path(name)
        V = configs.REAL[name]["vocab_size"]
        rng = np.random.default_rng(17)
        ids = rng.integers(0, V, n_prompt).astype(np.int32)
        toks = rng.integers(0, V, n_dec).astype(np.int32)
        lg = run_ref(path, ids, toks, False, n_prompt + n_dec + 2)
        np.savez_compressed(os.path.join(HERE, f"real_{name}.npz"), ids=ids, toks=toks,
                            sha1=configs.file_sha1(path), **summarize(lg))
        print("real", name, flush=True)
    L.ember_threads_shutdown()


def noise_fixture():
    """Deviation of the optimized reference from the deterministic one on each
    GPU parity case (same seeds and lengths as tests/test_gpu_parity.py)."""
    fast = oracle.reference_lib(debug=False)
    fast.ember_threads_init(min(8, os.cpu_count() or 1))
    ref().ember_threads_init(min(8, os.cpu_count() or 1))
    out = {}
    for case in GPU_CASES:
        name, kv16, n_prompt, n_dec, seed = case["name"], case["kv_fp16"], case["prompt"], case["decode"], case["seed"]
        path = configs.model_path(name)
        V = configs.ALL[name]["vocab_size"]
        rng = np.random.default_rng(seed)
        ids, toks = rng.integers(0, V, n_prompt), rng.integers(0, V, n_dec)
        ctx = case.get("ctx", 0)
        a = run_ref(path, ids, toks, kv16, ctx, debug=True)
        b = run_ref(path, ids, toks, kv16, ctx, debug=False)
        res = [compare(y, x) for x, y in zip(a, b)]
        out[case["id"]] = dict(
            rel_l2_median=float(np.median([r["rel_l2"] for r in res])),
            rel_l2_max=float(max(r["rel_l2"] for r in res)),
            max_abs_median=float(np.median([r["max_abs"] for r in res])),
            max_abs_max=float(max(r["max_abs"] for r in res)),
            top1=float(np.mean([r["agree"] for r in res])), steps=len(res))
        print("noise", case["id"], out[case["id"]], flush=True)
    with open(os.path.join(HERE, "noise_floor.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)


def wide_fixture():
    """Deviation of the optimized reference from the deterministic one on the
    4,200-token prefill of the 2-layer Qwen3-width models (three passes of
    the GPU's prefill: the end-to-end part of
    tests/test_gpu_kernels.py::test_prefill_three_passes), added to
    noise_floor.json under "<name>-p4200"."""
    n = 4200
    fast = oracle.reference_lib(debug=False)
    fast.ember_threads_init(min(8, os.cpu_count() or 1))
    ref().ember_threads_init(min(8, os.cpu_count() or 1))
    path_json = os.path.join(HERE, "noise_floor.json")
    with open(path_json) as f:
        out = json.load(f)
    for name in configs.WIDE:
        path = configs.model_path(name)
        ids = np.random.default_rng(n).integers(0, configs.WIDE[name]["vocab_size"], n)
        lg = []
        for debug in (True, False):
            r = oracle.Reference(path, ctx=n + 8, debug=debug)
            lg.append(r.prefill(ids))
            r.close()
        c = compare(lg[1], lg[0])
        out.pop(f"{name}-p2300", None)
        out[f"{name}-p{n}"] = dict(rel_l2_median=c["rel_l2"], rel_l2_max=c["rel_l2"], max_abs_median=c["max_abs"],
                                   max_abs_max=c["max_abs"], top1=float(c["agree"]), steps=1)
        print("noise", name, out[f"{name}-p{n}"], flush=True)
    with open(path_json, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)


# the benchmark workloads of tests/test_gpu_workloads.py: (name, prompt, steps, sampled)
WORKLOADS = [("stories110m", 128, 128, False), ("smollm2_135m", 1024, 128, False),
             ("qwen25_05b", 256, 128, True), ("qwen3_06b", 128, 128, False), ("qwen3_06b_q4", 512, 256, False)]


def workload_fixture():
    """Deviation of the optimized reference from the deterministic one over
    the benchmark workloads' full protocol (same seeds and lengths as
    tests/test_gpu_workloads.py): the deterministic build generates its own
    tokens (greedy, or its sampler at T 0.8 / top-k 40 / top-p 0.9, seed
    1234) and the optimized build is teacher forced on them; added to
    noise_floor.json under "<name>-pp<prompt>-tg<steps>"."""
    fast = oracle.reference_lib(debug=False)
    fast.ember_threads_init(min(8, os.cpu_count() or 1))
    ref().ember_threads_init(min(8, os.cpu_count() or 1))
    path_json = os.path.join(HERE, "noise_floor.json")
    with open(path_json) as f:
        out = json.load(f)
    for name, prompt, steps, sampled in WORKLOADS:
        path = configs.model_path(name)
        V = configs.ALL[name]["vocab_size"]
        rng = np.random.default_rng(prompt * 7 + steps)
        ids = rng.integers(0, V, prompt)
        ctx = prompt + steps + 2
        a = oracle.Reference(path, ctx=ctx, debug=True)
        b = oracle.Reference(path, ctx=ctx, debug=False)
        smp = oracle.Sampler()
        ref().ember_sampler_init(ctypes.byref(smp), 0.8, 0.9, 40, 1234)

        def pick(lg):
            if not sampled:
                return int(np.argmax(lg))
            x = np.ascontiguousarray(lg, dtype=np.float32).copy()
            return int(ref().ember_sample(ctypes.byref(smp), oracle.f32p(x), len(x)))

        la = a.prefill(ids)
        res = [compare(b.prefill(ids), la)]
        t = pick(la)
        for i in range(steps):
            la = a.forward(t, prompt + i)
            res.append(compare(b.forward(t, prompt + i), la))
            t = pick(la)
        a.close()
        b.close()
        ref().ember_sampler_free(ctypes.byref(smp))
        key = f"{name}-pp{prompt}-tg{steps}"
        out[key] = dict(
            rel_l2_median=float(np.median([r["rel_l2"] for r in res])),
            rel_l2_max=float(max(r["rel_l2"] for r in res)),
            max_abs_median=float(np.median([r["max_abs"] for r in res])),
            max_abs_max=float(max(r["max_abs"] for r in res)),
            top1=float(np.mean([r["agree"] for r in res])), steps=len(res),
            misses=[[i, r["margin"], r["rms"]] for i, r in enumerate(res) if not r["agree"]])
        print("noise", key, {k: v for k, v in out[key].items()}, flush=True)
        with open(path_json, "w") as f:
            json.dump(out, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    what = sys.argv[1:] or ["quant", "f16", "sampler", "tiny", "real", "noise", "wide", "workload"]
    for w in what:
        globals()[f"{w}_fixture"]()
