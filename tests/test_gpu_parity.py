"""GPU parity: the HIP path, called through libember.so's C ABI (ember.h),
against the oracle (the CPU restatement, bit-exact with the reference's
deterministic build) on identical seeded weights and token streams.

Tolerances: tests/parity.py (the target bar 1e-2 max-abs / 1e-3 rel-L2 /
99% top-1, which the small variant models meet; on the deep benchmark shapes
raised to 1.5x the reference's own optimized-vs-deterministic deviation,
which is ~1e-2 relative L2 there: see parity.py, and test_gpu_kernels.py for
the kernel-level bound at those shapes).  Every case prints its name before
it touches the GPU.
"""
import sys

import numpy as np
import pytest

import oracle
from cases import CASES, GPU_CASES
from emberllm_amd import configs, emberllm
from parity import FLIP_MAX_ABS, FLIP_REL_L2, bars, check_run, compare, near_tie

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu-parity] {msg}", flush=True)
    sys.stdout.flush()


def teacher_forced(case, graph=True):
    """Run one case on the GPU and the oracle; returns per-step compare()s."""
    name = case["name"]
    path = configs.model_path(name, threads=16)
    V = configs.ALL[name]["vocab_size"]
    rng = np.random.default_rng(case["seed"])
    ids, toks = rng.integers(0, V, case["prompt"]), rng.integers(0, V, case["decode"])
    say(f"{case['id']} graph={graph}")
    eng = emberllm.Engine(path, ctx=case["ctx"], kv_fp16=case["kv_fp16"])
    eng.set_graph(graph)
    orc = oracle.Oracle(path, ctx=case["ctx"], kv_fp16=case["kv_fp16"])
    out = [compare(eng.prefill(ids), orc.prefill(ids))]
    for i, t in enumerate(toks):
        pos = case["prompt"] + i
        out.append(compare(eng.forward(t, pos), orc.forward(t, pos)))
    eng.close()
    orc.close()
    return out


FAST = [c for c in GPU_CASES if c["name"] in configs.TINY]
SLOW = [c for c in GPU_CASES if c["name"] in configs.REAL]


@pytest.mark.parametrize("case", FAST, ids=[c["id"] for c in FAST])
def test_small_models(case, oracle_threads):
    say(check_run(teacher_forced(case), case["id"]))


@pytest.mark.parametrize("cid", ["t_llama-p8-d16-s0", "t_qwen3-p8-d16-s0"])
def test_eager_launches(cid, oracle_threads):
    """The same cases with plain stream launches instead of the hipGraph."""
    say(check_run(teacher_forced(CASES[cid], graph=False), cid))


@pytest.mark.slow
@pytest.mark.parametrize("case", SLOW, ids=[c["id"] for c in SLOW])
def test_benchmark_shapes(case, oracle_threads):
    say(check_run(teacher_forced(case), case["id"]))


@pytest.mark.parametrize("schedule", ["folded-wo", "in-kernel-merge", "two-kernel"])
def test_decode_schedules(schedule, oracle_threads, monkeypatch):
    """The Qwen3-0.6B shape (8 kv heads: one per XCD of the MI355X) under each
    decode schedule the state can choose: the attention kernel merging its
    chunks through the XCD's L2 and computing its kv group's share of the wo
    product (the default there), the same merge with wo as its own matvec
    (EHIP_FUSE_WO=0), and the chunk kernel + merge kernel (EHIP_XMERGE=0).
    All must match the oracle, including past one chunk per workgroup
    (prompt 300, decode to depth 332)."""
    if schedule == "two-kernel":
        monkeypatch.setenv("EHIP_XMERGE", "0")
    elif schedule == "in-kernel-merge":
        monkeypatch.setenv("EHIP_FUSE_WO", "0")
    name = "qwen3_06b"
    path = configs.model_path(name, threads=16)
    V = configs.ALL[name]["vocab_size"]
    rng = np.random.default_rng(77)
    ids, toks = rng.integers(0, V, 300), rng.integers(0, V, 32)
    say(f"qwen3_06b schedule={schedule} p300 d32")
    eng = emberllm.Engine(path, ctx=400)
    fusion = eng.decode_fusion()
    want = {"folded-wo": 3, "in-kernel-merge": 1, "two-kernel": 0}[schedule]
    assert fusion == want, f"state chose fusion {fusion}, expected {want} on this device"
    orc = oracle.Oracle(path, ctx=400)
    res = [compare(eng.prefill(ids), orc.prefill(ids))]
    for i, t in enumerate(toks):
        res.append(compare(eng.forward(int(t), 300 + i), orc.forward(int(t), 300 + i)))
    # a schedule whose error flag fired would have re-run its steps on the two-kernel one
    assert eng.decode_fusion() == want, f"the state left fusion {want} during the run"
    eng.close()
    orc.close()
    # bars of the same shape's teacher-forced case (the reference builds' noise floor)
    say(f"{schedule}: " + check_run(res, "qwen3_06b-p16-d32-s11"))


@pytest.mark.parametrize("name", ["smollm2_135m", "qwen25_05b", "qwen3_06b_q4"])
@pytest.mark.parametrize("fold", ["folded-wo", "wo-matvec"])
def test_decode_fold(name, fold, oracle_threads, monkeypatch):
    """The other folds of the wo product.  Shapes whose kv heads are not a
    multiple of 8 (SmolLM2-135M: 3 kv heads of 3 query heads, Qwen2.5-0.5B: 2
    of 7) merge in-kernel on the 1-D grid, one kv head per XCD, and fold wo
    in there (merge mode 4: G * head_dim / 16 of the row's chunk lanes in
    use, two rounds of rows for Qwen2.5); the Qwen3-0.6B Q4_0 shape folds its
    Q4_0 wo on the 2-D grid (mode 5: one block per lane).  With and without
    the fold (EHIP_FUSE_WO=0) the run must match the oracle past one chunk
    per workgroup (prompt 300, decode to depth 332), and keep its schedule
    throughout."""
    if fold == "wo-matvec":
        monkeypatch.setenv("EHIP_FUSE_WO", "0")
    want = 3 if fold == "folded-wo" else 1
    path = configs.model_path(name, threads=16)
    V = configs.ALL[name]["vocab_size"]
    rng = np.random.default_rng(78)
    ids, toks = rng.integers(0, V, 300), rng.integers(0, V, 32)
    say(f"{name} {fold} p300 d32")
    eng = emberllm.Engine(path, ctx=400)
    assert eng.decode_fusion() == want, f"state chose fusion {eng.decode_fusion()}, expected {want}"
    orc = oracle.Oracle(path, ctx=400)
    res = [compare(eng.prefill(ids), orc.prefill(ids))]
    for i, t in enumerate(toks):
        res.append(compare(eng.forward(int(t), 300 + i), orc.forward(int(t), 300 + i)))
    assert eng.decode_fusion() == want, f"the state left fusion {want} during the run"
    eng.close()
    orc.close()
    say(f"{name} {fold}: " + check_run(res, f"{name}-p16-d32-s11"))


@pytest.mark.parametrize("name,n", [("qwen3_06b", 600), ("qwen3_06b", 4096), ("qwen3_06b_q4", 512),
                                    ("qwen25_05b", 300), ("stories110m", 520)])
def test_prefill_fused_swiglu_equals_separate(name, n, monkeypatch):
    """Passes long enough for the matrix-core GEMM tiles quantize the SwiGLU
    rows in the w1|w3 product's epilogue (k_gemm_mfma's EPI_SWIGLU form: gate
    and up rows paired in each tile).  Its codes, scales and code sums are
    the ones k_quant_rows makes from the stored products, so the prefill's
    logits and KV rows equal those of the separate kernels
    (EHIP_PF_SWIGLU=0) bit for bit; Q8_0 and Q4_0 weights, 64- and 128-token
    tiles."""
    path = configs.model_path(name, threads=16)
    V, L = configs.ALL[name]["vocab_size"], configs.ALL[name]["n_layers"]
    ids = np.random.default_rng(n).integers(0, V, n)
    say(f"{name} pp{n}: fused SwiGLU quantization vs separate kernels")
    out = []
    for fused in ("0", "1"):
        monkeypatch.setenv("EHIP_PF_SWIGLU", fused)
        eng = emberllm.Engine(path, ctx=n + 8)
        lg = eng.prefill(ids)
        out.append((lg, eng.kv_read(0, L - 1, n), eng.kv_read(1, L - 1, n)))
        eng.close()
    for a, b in zip(out[0], out[1]):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("name,n,kv16", [("qwen3_06b", 600, False), ("qwen3_06b", 2000, True),
                                         ("qwen3_06b_q4", 2000, False), ("qwen3_06b", 3072, False)])
def test_prefill_fused_qkpost_equals_separate(name, n, kv16, monkeypatch):
    """Passes long enough for the matrix-core q|k|v product take k_qkpost's
    work into its epilogue (k_gemm_mfma's EPI_QKPOST form on 64-token tiles
    with one pipeline: bias, the heads' RMSNorm in k_qkpost's summation
    order, neox RoPE, q into its row, k and v into the cache).  Logits, the
    last layer's K and V rows and the captured raw product equal those of the
    separate kernels on the same tiles (EHIP_PF_QKPOST=0 where the product's
    shape keeps one pipeline and 64-token tiles: 2000 tokens) bit for bit,
    and elsewhere (600 tokens: two pipelines, 3072: 128-token tiles) up to
    the order of the products' block sums; Q8_0 and Q4_0 weights (the
    latter's smaller stages take the pair sums in two rounds), fp32 and fp16
    caches, a partial last token tile (2000 = 31 x 64 + 16)."""
    path = configs.model_path(name, threads=16)
    V, L = configs.ALL[name]["vocab_size"], configs.ALL[name]["n_layers"]
    ids = np.random.default_rng(n).integers(0, V, n)
    say(f"{name} pp{n} kv16={kv16}: fused QK post-processing vs k_qkpost")
    out = []
    for fused in ("0", "1"):
        monkeypatch.setenv("EHIP_PF_QKPOST", fused)
        eng = emberllm.Engine(path, ctx=n + 8, kv_fp16=kv16)
        eng.debug_capture_prefill(L - 1)
        lg = eng.prefill(ids)
        raw, p0 = eng.debug_read_prefill(1)
        assert p0 == 0 and raw.shape[0] == n
        out.append((lg, eng.kv_read(0, L - 1, n), eng.kv_read(1, L - 1, n), raw))
        eng.close()
    for a, b in zip(out[0], out[1]):
        if n == 2000:
            np.testing.assert_array_equal(a, b)
            continue
        # two block-sum orders of the products, each within the bar this
        # model's logits meet against the oracle (set by the reference
        # builds' own spread at this shape): so within twice it of each other
        b_ = bars("qwen3_06b-p16-d32-s11")
        if a.dtype == np.uint8:   # cache rows
            a, b = (x.view(np.float16 if kv16 else np.float32).astype(np.float32) for x in (a, b))
        r = compare(np.ravel(a), np.ravel(b))
        assert r["max_abs"] <= 2 * b_["abs_max"] and r["rel_l2"] <= 2 * b_["rel_max"], (r, b_)


@pytest.mark.parametrize("name,n,kv16,start", [("qwen3_06b", 600, False, 0), ("qwen3_06b_q4", 700, False, 0),
                                               ("qwen3_06b", 1100, True, 0), ("qwen3_06b", 600, False, 640),
                                               ("qwen3_06b", 500, False, 600), ("qwen3_06b", 320, False, 0),
                                               ("qwen3_06b_q4", 300, False, 0), ("smollm2_135m", 1000, True, 0),
                                               ("qwen25_05b", 300, False, 0), ("smollm2_135m", 200, False, 128)])
def test_prefill_fused_kv_images_equal_kvsplit(name, n, kv16, start, monkeypatch):
    """The fused q|k|v products (k_gemm_mfma's EPI_QKPOST form for longer
    passes with 128-dim heads, k_gemm_qkv for short prompts and 64-dim heads)
    of a pass that starts on a 64-key tile also write the pass's own K/V tile
    images for the matrix-core attention (k_pf_kvsplit then converts only the
    earlier tiles).  The images are k_pf_kvsplit's bytes, so logits and the
    last layer's K/V rows equal those of EHIP_PF_KVIMG=0 bit for bit: Q8_0
    and Q4_0 weights, fp32 (hi/lo planes and per-key exponents) and fp16
    caches, head dims 128 and 64 (SmolLM2-135M and Qwen2.5-0.5B shapes),
    passes whose last tile is partial (its rest repeats the last key),
    continuation passes at positions 640 and 128 (earlier tiles converted,
    the pass's fused) and one at 600 (not on a tile boundary: every tile
    converted)."""
    path = configs.model_path(name, threads=16)
    V, L = configs.ALL[name]["vocab_size"], configs.ALL[name]["n_layers"]
    rng = np.random.default_rng(n + start)
    pre = rng.integers(0, V, start)
    ids = rng.integers(0, V, n)
    say(f"{name} pp{n} at {start} kv16={kv16}: fused K/V tile images vs k_pf_kvsplit")
    out = []
    for fused in ("0", "1"):
        monkeypatch.setenv("EHIP_PF_KVIMG", fused)
        eng = emberllm.Engine(path, ctx=start + n + 8, kv_fp16=kv16)
        if start:
            eng.prefill(pre)
        lg = eng.prefill(ids, start)
        out.append((lg, eng.kv_read(0, L - 1, start + n), eng.kv_read(1, L - 1, start + n)))
        eng.close()
    for a, b in zip(out[0], out[1]):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("name,n,kv16,start", [("qwen3_06b", 512, False, 0), ("qwen3_06b_q4", 300, True, 0),
                                               ("smollm2_135m", 1000, False, 0), ("qwen25_05b", 256, False, 0),
                                               ("qwen3_06b", 200, False, 320)])
def test_prefill_split_attention_matches_one_group(name, n, kv16, start, oracle_threads, monkeypatch):
    """Passes whose matrix-core attention grid would leave CUs idle run
    k_pf_flash16 on 32-row workgroups of two key-tile groups (alternate
    tiles, running softmax states merged at the end).  Its summation order is
    not the one-group kernel's (EHIP_PF_FLASH_KS=1), so the two agree within
    the bar the model's logits meet against the oracle, as each of them does
    against the oracle itself: Q8_0 and Q4_0 weights,
    fp32 and fp16 caches, 128- and 64-dim heads, 1, 2, 3 and 7 query heads
    per kv head, a continuation pass at position 320."""
    path = configs.model_path(name, threads=16)
    V = configs.ALL[name]["vocab_size"]
    rng = np.random.default_rng(n + start)
    pre, ids = rng.integers(0, V, start), rng.integers(0, V, n)
    say(f"{name} pp{n} at {start} kv16={kv16}: split-group prefill attention")
    out = []
    for ks in ("1", "2"):
        monkeypatch.setenv("EHIP_PF_FLASH_KS", ks)
        eng = emberllm.Engine(path, ctx=start + n + 8, kv_fp16=kv16)
        if start:
            eng.prefill(pre)
        out.append(eng.prefill(ids, start))
        eng.close()
    orc = oracle.Oracle(path, ctx=start + n + 8, kv_fp16=kv16)
    if start:
        orc.prefill(pre)
    ref = orc.prefill(ids, start)
    orc.close()
    b = bars(f"{name}-p16-d32-s11")
    for r, k in ((compare(out[1], ref), 1), (compare(out[0], ref), 1), (compare(out[1], out[0]), 2)):
        # each path within the bar of the oracle; the two within twice it
        assert r["finite"] and r["max_abs"] <= k * b["abs_max"] and r["rel_l2"] <= k * b["rel_max"], (r, b)


@pytest.mark.parametrize("name", ["t_qwen3", "t_llama"])
def test_graph_equals_eager(name):
    """The captured graph replays exactly the eager launch sequence."""
    path = configs.model_path(name)
    say(f"graph vs eager bit equality ({name})")
    V = configs.ALL[name]["vocab_size"]
    a = emberllm.Engine(path)
    b = emberllm.Engine(path)
    a.set_graph(True)
    b.set_graph(False)
    ids = np.arange(5) * 7 % V
    np.testing.assert_array_equal(a.prefill(ids), b.prefill(ids))
    for pos in range(5, 15):
        np.testing.assert_array_equal(a.forward(pos * 3 % V, pos), b.forward(pos * 3 % V, pos))
    a.close()
    b.close()


def test_repeatable():
    """Two runs of the same stream give identical logits (no races)."""
    path = configs.model_path("t_g7")
    say("repeatability")
    outs = []
    for _ in range(2):
        e = emberllm.Engine(path)
        seq = [e.prefill(np.arange(270) % 384)]
        seq += [e.forward(t, 270 + i) for i, t in enumerate([3, 99, 7])]
        outs.append(np.array(seq))
        e.close()
    np.testing.assert_array_equal(outs[0], outs[1])


def test_prefill_continuation(oracle_threads):
    """ember_prefill at start > 0 (chat continuation, main.c:298-306)."""
    path = configs.model_path("t_bias")
    say("prefill continuation")
    eng = emberllm.Engine(path)
    orc = oracle.Oracle(path)
    a = np.array([5, 9, 33, 7, 100, 2], dtype=np.int32)
    b = np.array([17, 3, 250, 41], dtype=np.int32)
    res = [compare(eng.prefill(a), orc.prefill(a)),
           compare(eng.prefill(b, start=len(a)), orc.prefill(b, start=len(a))),
           compare(eng.forward(11, 10), orc.forward(11, 10))]
    for r in res:  # within one activation-code flip of the oracle (tests/parity.py)
        assert r["rel_l2"] <= FLIP_REL_L2 and r["max_abs"] <= FLIP_MAX_ABS and r["agree"], r
    eng.close()
    orc.close()


def test_zero_length_prefill_returns_previous_logits():
    """n <= 0 returns the current logits unchanged (model.c:285)."""
    path = configs.model_path("t_llama")
    say("zero-length prefill")
    e = emberllm.Engine(path)
    first = e.prefill([1, 2, 3])
    again = e.prefill([])
    np.testing.assert_array_equal(first, again)
    e.close()


def test_kv_cache_matches_oracle(oracle_threads):
    """The cache the GPU prefill writes equals the oracle's: k after QK-norm
    and RoPE, v raw, fp32 or fp16 (model.c:39-48, 323-333)."""
    name = "t_qwen3"
    path = configs.model_path(name)
    L = configs.ALL[name]["n_layers"]
    for kv16 in (False, True):
        say(f"kv cache contents kv_fp16={kv16}")
        eng = emberllm.Engine(path, kv_fp16=kv16)
        orc = oracle.Oracle(path, kv_fp16=kv16)
        ids = np.arange(12) * 37 % 640
        eng.prefill(ids)
        orc.prefill(ids)
        dt = np.float16 if kv16 else np.float32
        for which in (0, 1):
            ocache = orc.kv(which).view(dt).reshape(L, orc.ctx, -1)
            for layer in range(L):
                g = eng.kv_read(which, layer, len(ids)).view(dt).reshape(len(ids), -1).astype(np.float64)
                o = ocache[layer, :len(ids)].astype(np.float64)
                rows = np.linalg.norm(g - o, axis=1) / np.linalg.norm(o, axis=1)
                # most rows agree to rounding; an activation-code flip upstream
                # moves a row by at most the one-flip amplitude (tests/parity.py)
                tight = 2e-3 if kv16 else 1e-5
                assert np.median(rows) <= tight and rows.max() <= FLIP_REL_L2, (kv16, which, layer, rows)
        eng.close()
        orc.close()


def test_prefill_equals_sequential_forward():
    """Property of the reference (model.c:283-360 vs 362-414): prefill's last
    logits equal feeding the same tokens one forward at a time."""
    path = configs.model_path("t_gqa")
    say("prefill vs sequential forwards")
    a = emberllm.Engine(path)
    b = emberllm.Engine(path)
    ids = [3, 77, 5, 300, 12, 9, 150]
    la = a.prefill(ids)
    for p, t in enumerate(ids):
        lb = b.forward(t, p)
    c = compare(la, lb)
    assert c["rel_l2"] <= FLIP_REL_L2 and c["max_abs"] <= FLIP_MAX_ABS and c["agree"], c
    a.close()
    b.close()


def test_tiny_goldens_of_the_reference():
    """The GPU against the compiled reference's own logits (tests/golden)."""
    import os
    here = os.path.dirname(os.path.abspath(__file__))
    for name in configs.TINY:
        g = np.load(os.path.join(here, "golden", f"tiny_{name}.npz"))
        path = configs.model_path(name)
        assert configs.file_sha1(path) == str(g["sha1"]), f"{name}: synthetic model drifted"
        for kv16, key in ((False, "fp32"), (True, "fp16")):
            say(f"reference golden {name} {key}")
            e = emberllm.Engine(path, kv_fp16=kv16)
            got = [e.prefill(g["ids"])] + [e.forward(int(t), len(g["ids"]) + i) for i, t in enumerate(g["toks"])]
            e.close()
            for step, (x, y) in enumerate(zip(got, g[key])):
                c = compare(x, y)
                # within one activation-code flip of the reference (tests/parity.py)
                assert c["agree"] and c["max_abs"] <= FLIP_MAX_ABS and c["rel_l2"] <= FLIP_REL_L2, (name, key, step, c)


@pytest.mark.slow
def test_qwen3_decode_at_depth_4096(oracle_threads):
    """Headline depth: the GPU prefills 4096 tokens, the oracle receives the
    same cache, and both decode 6 steps at positions 4096.. (teacher forced)."""
    name = "qwen3_06b"
    path = configs.model_path(name, threads=16)
    depth, steps = 4096, 6
    ctx = depth + steps + 2
    rng = np.random.default_rng(4096)
    ids = rng.integers(0, 151936, depth)
    say("qwen3 depth-4096 KV hand-over")
    eng = emberllm.Engine(path, ctx=ctx)
    eng.prefill(ids)
    orc = oracle.Oracle(path, ctx=ctx)
    L = configs.ALL[name]["n_layers"]
    row = eng.kv_row_bytes()
    for which in (0, 1):
        dst = orc.kv(which).reshape(L, ctx * row)
        for layer in range(L):
            dst[layer, :depth * row] = eng.kv_read(which, layer, depth)
    res = []
    for i in range(steps):
        tok, pos = int(rng.integers(0, 151936)), depth + i
        res.append(compare(eng.forward(tok, pos), orc.forward(tok, pos)))
    eng.close()
    orc.close()
    # same bar as the depth-16 Qwen3 case
    say(check_run(res, "qwen3_06b-p16-d32-s11"))


def _greedy_case(name, n_prompt, n_gen, seed, ctx=0, kv16=False):
    """Device greedy loop vs the C-API loop (ember_forward + first-max argmax
    on the host, src/sample.c:114-127) and vs the oracle, teacher forced on
    the GPU's own token sequence."""
    path = configs.model_path(name, threads=16)
    V = configs.ALL[name]["vocab_size"]
    rng = np.random.default_rng(seed)
    ids = rng.integers(0, V, n_prompt)
    say(f"device greedy {name} prompt={n_prompt} gen={n_gen} kv16={kv16}")
    a = emberllm.Engine(path, ctx=ctx, kv_fp16=kv16)
    first = a.prefill(ids)
    tok0 = int(np.argmax(first))
    toks, ms = a.generate_greedy(tok0, n_prompt, n_gen)
    assert ms > 0
    last = a.debug_buffer(4, V)
    a.close()
    b = emberllm.Engine(path, ctx=ctx, kv_fp16=kv16)
    b.prefill(ids)
    orc = oracle.Oracle(path, ctx=ctx, kv_fp16=kv16)
    orc.prefill(ids)
    t, res = tok0, []
    for i in range(n_gen):
        lg = b.forward(t, n_prompt + i)
        ref = orc.forward(t, n_prompt + i)
        assert int(np.argmax(lg)) == int(toks[i]), f"step {i}: device loop chose {toks[i]}, API loop {np.argmax(lg)}"
        res.append(compare(lg, ref))
        t = int(toks[i])
    np.testing.assert_array_equal(last, lg)   # bit-identical last logits
    b.close()
    orc.close()
    return res


def test_device_greedy_loop(oracle_threads):
    res = _greedy_case("t_qwen3", 9, 40, 5)
    for r in res:
        assert r["agree"] or near_tie(r), r
    res = _greedy_case("t_g7", 300, 12, 6, kv16=True)
    for r in res:
        assert r["agree"] or near_tie(r), r


def test_device_argmax_first_maximum(tmp_path):
    """Ties resolve to the first index, as the reference's strict `>` scan
    (src/sample.c:114-118): with final_norm zeroed every logit is exactly 0,
    so each greedy step must choose token 0."""
    import shutil
    src = configs.model_path("t_llama")
    path = str(tmp_path / "tied_logits.ember")
    shutil.copy(src, path)
    lib = emberllm._native.lib()
    m = lib.ember_model_load(path.encode())
    t = lib.ember_model_tensor(m, b"final_norm").contents
    off, nbytes = int(t.offset), int(t.nbytes)
    lib.ember_model_free(m)
    with open(path, "r+b") as f:
        f.seek(off)
        f.write(bytes(nbytes))
    say("device argmax tie rule")
    e = emberllm.Engine(path)
    lg = e.prefill([1, 2, 3])
    assert np.all(lg == 0.0)
    toks, _ = e.generate_greedy(5, 3, 4)
    np.testing.assert_array_equal(toks, 0)
    e.close()


@pytest.mark.slow
def test_device_greedy_qwen3_shape(oracle_threads):
    res = _greedy_case("qwen3_06b", 16, 24, 12, ctx=48)
    ok = [r["agree"] or near_tie(r) for r in res]
    assert np.mean(ok) >= 0.99, res


def test_measured_read_bandwidth():
    """ehip_measure_read_bw: a plain streaming read over 256 MiB lands between
    a tenth of and the datasheet's 8 TB/s, and a request below 1 MiB is an
    error (the host rejects it before any launch)."""
    say("measured read bandwidth")
    e = emberllm.Engine(configs.model_path("t_llama"))
    gbs = e.measure_read_bw(256 << 20, 4)
    say(f"read bandwidth {gbs:.0f} GB/s")
    assert 800.0 < gbs < 8000.0, gbs
    with pytest.raises(RuntimeError):
        e.measure_read_bw(1024, 1)
    e.close()


@pytest.mark.parametrize("name", ["qwen3_06b", "stories110m"])
def test_xcd_check_falls_back_to_the_merge_kernel(name, monkeypatch):
    """The in-kernel merge relies on every workgroup of a kv head running on
    the XCD the state's probe recorded; each workgroup checks that and raises
    a flag.  EHIP_XMERGE_TEST_SKEW records the wrong XCDs (the kernels
    themselves run as usual), so the check fires on the first decode launch:
    the state must then switch to the two-kernel merge for good and re-run
    the work, returning exactly what a state created with that schedule
    (EHIP_XMERGE=0) returns, through ember_forward and the device loop.
    Qwen3-0.6B has 8 kv heads (one per XCD), stories110M 12 (two on four of
    the XCDs)."""
    path = configs.model_path(name, threads=16)
    V = configs.ALL[name]["vocab_size"]
    ids = np.arange(100) * 97 % V   # several chunks per kv head, so the merge (and its check) runs
    say("XCD placement check: forced mismatch")
    monkeypatch.setenv("EHIP_XMERGE", "0")
    ref = emberllm.Engine(path, ctx=160)
    assert ref.decode_fusion() == 0
    tok0 = int(np.argmax(ref.prefill(ids)))
    want_fwd = ref.forward(tok0, len(ids))
    want_toks, _ = ref.generate_greedy(tok0, len(ids), 9)
    ref.close()
    monkeypatch.delenv("EHIP_XMERGE")
    monkeypatch.setenv("EHIP_XMERGE_TEST_SKEW", "3")
    for path_kind in ("forward", "device loop"):
        eng = emberllm.Engine(path, ctx=160)
        if not eng.decode_fusion() & 1:
            eng.close()
            pytest.skip("this GPU does not place a kv head's workgroups on one XCD; the merge runs as a second kernel")
        eng.prefill(ids)
        if path_kind == "forward":
            np.testing.assert_array_equal(eng.forward(tok0, len(ids)), want_fwd)
            got, _ = eng.generate_greedy(tok0, len(ids), 9)
        else:
            got, _ = eng.generate_greedy(tok0, len(ids), 9)
        np.testing.assert_array_equal(got, want_toks)
        assert eng.decode_fusion() == 0, "the state must keep the two-kernel schedule after the check fired"
        eng.close()


@pytest.mark.parametrize("name", ["qwen3_06b", "stories110m", "smollm2_135m"])
def test_stale_partial_check_falls_back(name, monkeypatch):
    """Every chunk stores a token of its launch (from the position and the
    API step's ticket) with its partial, and the in-kernel merge checks each
    partial it reads carries the current one.  EHIP_XMERGE_TEST_TOK=1 plants a wrong token in
    chunk 0 (the kernels otherwise run as usual), so the first merge finds a
    'stale' partial: the state must then switch to the two-kernel schedule
    for good and re-run the work, returning exactly what a state created with
    that schedule (EHIP_XMERGE=0) returns, through ember_forward and the
    device loop.  Qwen3-0.6B merges on the 2-D grid with the folded wo
    (mode 3), stories110M on the 1-D grid (mode 2), SmolLM2-135M on the 1-D
    grid with the folded wo (mode 4)."""
    path = configs.model_path(name, threads=16)
    V = configs.ALL[name]["vocab_size"]
    ids = np.arange(100) * 83 % V   # several chunks per kv head, so the merge (and its check) runs
    say(f"stale partial check: planted token ({name})")
    monkeypatch.setenv("EHIP_XMERGE", "0")
    ref = emberllm.Engine(path, ctx=160)
    assert ref.decode_fusion() & 3 == 0
    tok0 = int(np.argmax(ref.prefill(ids)))
    want_fwd = ref.forward(tok0, len(ids))
    want_toks, _ = ref.generate_greedy(tok0, len(ids), 9)
    ref.close()
    monkeypatch.delenv("EHIP_XMERGE")
    monkeypatch.setenv("EHIP_XMERGE_TEST_TOK", "1")
    for path_kind in ("forward", "device loop"):
        eng = emberllm.Engine(path, ctx=160)
        if not eng.decode_fusion() & 1:
            eng.close()
            pytest.skip("this GPU does not place a kv head's workgroups on one XCD; the merge runs as a second kernel")
        eng.prefill(ids)
        if path_kind == "forward":
            np.testing.assert_array_equal(eng.forward(tok0, len(ids)), want_fwd)
        got, _ = eng.generate_greedy(tok0, len(ids), 9)
        np.testing.assert_array_equal(got, want_toks)
        assert eng.decode_fusion() & 3 == 0, "the state must keep the two-kernel schedule after the check fired"
        eng.close()


@pytest.mark.parametrize("name", ["qwen3_06b", "smollm2_135m"])
def test_folded_wo_timeout_falls_back(name, monkeypatch):
    """The folded wo product waits for its kv group's merged output with a
    bounded poll of a flag; on time-out the workgroup raises the error flag
    instead of writing its rows.  EHIP_FW_TEST_SPIN=0 makes every workgroup
    that finds the flag still down time out at once (the kernels otherwise
    run as usual), so the state must switch to the two-kernel schedule for
    good and re-run the work, returning exactly what a state created with
    that schedule returns, through ember_forward and the device loop.
    Qwen3-0.6B folds it on the 2-D grid (merge mode 3), SmolLM2-135M on the
    1-D grid (mode 4)."""
    path = configs.model_path(name, threads=16)
    V = configs.ALL[name]["vocab_size"]
    ids = np.arange(100) * 89 % V
    say("folded wo product: forced time-out")
    monkeypatch.setenv("EHIP_XMERGE", "0")
    ref = emberllm.Engine(path, ctx=160)
    assert ref.decode_fusion() == 0
    tok0 = int(np.argmax(ref.prefill(ids)))
    want_fwd = ref.forward(tok0, len(ids))
    want_toks, _ = ref.generate_greedy(tok0, len(ids), 9)
    ref.close()
    monkeypatch.delenv("EHIP_XMERGE")
    monkeypatch.setenv("EHIP_FW_TEST_SPIN", "0")
    for path_kind in ("forward", "device loop"):
        eng = emberllm.Engine(path, ctx=160)
        if eng.decode_fusion() != 3:
            eng.close()
            pytest.skip("the state does not fold the wo product on this device")
        eng.prefill(ids)
        if path_kind == "forward":
            np.testing.assert_array_equal(eng.forward(tok0, len(ids)), want_fwd)
        got, _ = eng.generate_greedy(tok0, len(ids), 9)
        np.testing.assert_array_equal(got, want_toks)
        assert eng.decode_fusion() == 0, "the state must keep the two-kernel schedule after the time-out"
        eng.close()
