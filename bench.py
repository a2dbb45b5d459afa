#!/usr/bin/env python3
"""Single-stream decode benchmark of the token loop on one MI355X.

Workload (the headline configuration): a Qwen3-0.6B-shape model, Q8_0
(dim 1024, 28 layers, 16 query / 8 KV heads of 128, QK-norm, FFN 3072,
vocab 151936, tied embeddings, RoPE theta 1e6), weights drawn N(0, 0.02)
from the package's seeded generator, norms 1.0, quantized by its bit-exact
Q8_0 quantizer.  The KV cache (fp32) is filled by a batched prefill of 4096
ids; then greedy-shaped decode runs at positions 4096.. .

A step is one decode token through the C API.  `value` is the reference's
own benchmark loop (`ember bench`, src/main.c:230-294: the reference's
main.c compiled unmodified against libember.so, emberllm_amd/_cli/ember):
per rep a pp<depth> prefill, then --steps calls of ember_forward, each
returning the step's logits in host memory, tokens (pos*131+7) % V from
pos = depth; one warmup rep, then the mean of the timed reps' decode rates.
Without that program (it is built where the reference's sources are) the
same protocol runs through ctypes.  Also reported, never as `value`:
  decode_tok_s_device_loop  the device-resident greedy loop
                        (ehip_generate_greedy: decode graph + on-device argmax,
                        no host round trip), HIP events on the state's stream
  api_decode_tok_s      the ember bench protocol through ctypes (ember_forward
                        per token from Python)
  decode_tok_s_depth128 ember bench --pp 128 (decode at depth 128)
  decode_tok_s_sampled  the device loop with the full sampler (temperature
                        0.8, top-k 40, top-p 0.9, fixed seed) at the same depth
  prefill_tok_s_pp128 / _pp4096   ember bench's prefill rates (mean of the
                        timed reps, src/main.c:251-266)
  ttft_ms_pp128 / _pp4096         ember_prefill plus the first token's
                        selection on the host (time to first token)
  load_s                ember_model_load + ember_state_new_ex: the file
                        mapped, weights repacked and uploaded, KV cache and
                        scratch allocated
  roofline              the dominant kernel (split-K attention of one layer
                        at depth 4096, in the form the decode step runs:
                        with its in-kernel merge and folded wo product where
                        the state uses them): algorithmic bytes per launch
                        over its average duration (HIP events, isolated
                        launches on the state's stream)
  cpu_baseline          the reference's own C code, compiled from its
                        sources into oracle/_ref/ (or, absent that, the
                        oracle's port), decoding at the same depth on the
                        host cores; best of a thread sweep on a bounded
                        sample
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK = 8.0e12          # MI355X HBM3E, bytes/s
METRIC = "single-stream decode tok/s (Qwen3-0.6B-shape Q8_0) + %HBM roofline; prefill tok/s"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def weight_bytes(c):
    """Bytes of every quantized matrix, norm and bias read by one decode step."""
    blk = {1: 34, 2: 18}[c["dtype"]] if c["dtype"] else None
    hd, L, dim, hid, V = c["head_dim"], c["n_layers"], c["dim"], c["hidden_dim"], c["vocab_size"]
    qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd

    def mat(rows, cols, b=blk):
        return rows * cols * 4 if b is None else rows * (cols // 32) * b

    per_layer = (mat(qd, dim) + 2 * mat(kvd, dim) + mat(dim, qd) + 2 * mat(hid, dim) + mat(dim, hid)
                 + 4 * 2 * dim + (4 * 2 * hd if c["qk_norm"] else 0)
                 + (4 * (qd + 2 * kvd) if c["qkv_bias"] else 0))
    head_blk = 34 if c["dtype"] in (1, 2) else None   # lm_head / embedding stay Q8_0 in Q4 files
    return L * per_layer + mat(V, dim, head_blk) + 4 * dim + mat(1, dim, head_blk)


def step_bytes(c, pos, e_kv):
    """Algorithmic HBM bytes of the decode step at position `pos`."""
    kvd = c["n_kv_heads"] * c["head_dim"]
    L, V = c["n_layers"], c["vocab_size"]
    return weight_bytes(c) + 2 * L * (pos + 1) * kvd * e_kv + 2 * L * kvd * e_kv + 4 * V


def attn_launch_bytes(c, pos, e_kv):
    """Algorithmic bytes of one layer's attention launch at `pos`: K and V rows
    [0, pos] read once, the new row written, q|k|v in, output out."""
    kvd = c["n_kv_heads"] * c["head_dim"]
    qd = c["n_heads"] * c["head_dim"]
    return 2 * (pos + 1) * kvd * e_kv + 2 * kvd * e_kv + 4 * (qd + 2 * kvd) + 4 * qd


def wo_fold_bytes(c):
    """Algorithmic bytes the folded wo product adds to an attention launch:
    the Q8_0 wo weights read (34 bytes per 32) and the kv groups' partial
    vectors written."""
    qd = c["n_heads"] * c["head_dim"]
    return c["dim"] * (qd // 32) * 34 + 4 * c["n_kv_heads"] * c["dim"]


def profiled_traffic(kernel, model, depth, kv):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC
    summary (FETCH_SIZE and WRITE_SIZE runs, scaled against a copy kernel of
    known size), when one exists for this exact workload; else None."""
    path = os.path.join(ROOT, "profiles", f"qwen3_q8_depth{depth}_traffic.md")
    if model != "qwen3_06b" or kv != "f32" or not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            cells = [x.strip() for x in line.strip().strip("|").split("|")]
            if len(cells) == 5 and cells[0].strip("`").startswith(kernel):
                return int(float(cells[4]) * 1e6)
    return None


def cpu_baseline(path, c, depth, budget_s):
    """The reference's CPU decode at `depth` on this host: best of a thread
    sweep, each point 1 warmup + timed steps within the time budget."""
    if os.path.join(ROOT, "oracle") not in sys.path:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    ncpu = min(16, len(os.sched_getaffinity(0)))
    V = c["vocab_size"]
    # the reference's Makefile builds with -march=native (Makefile:23): its
    # AVX2 (x86-64-v3) build and, where this host has AVX-512, its x86-64-v4
    # build are both swept and the faster reported
    flags = set()
    try:
        with open("/proc/cpuinfo") as f:
            flags = set(next((ln.split(":", 1)[1].split() for ln in f if ln.startswith("flags")), []))
    except OSError:
        pass
    has_v4 = {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= flags
    builds = [False] + ([True] if has_v4 and os.path.exists(oracle.reference_path(False, v4=True)) else [])
    kind = "reference"

    def note(v4):
        return (f"oracle/_ref/{os.path.basename(oracle.reference_path(False, v4))} (the reference's sources with "
                f"its optimized flags -O3 -ffast-math -funroll-loops, -march={'x86-64-v4' if v4 else 'x86-64-v3'} "
                f"in place of -march=native)")
    try:
        for v4 in builds:
            oracle.reference_lib(debug=False, v4=v4)

        def make(ctx, v4):
            return oracle.Reference(path, ctx=ctx, debug=False, v4=v4)

        def set_threads(n, v4):
            libr = oracle.reference_lib(debug=False, v4=v4)
            libr.ember_threads_shutdown()
            libr.ember_threads_init(n)
    except (FileNotFoundError, OSError):
        kind, builds = "port", [False]
        libo = oracle.oracle_lib(fast=True)

        def note(v4):
            return "oracle/liboracle_fast.so (restatement, optimized flags)"

        def make(ctx, v4):
            return oracle.Oracle(path, ctx=ctx, fast=True)

        def set_threads(n, v4):
            libo.orc_threads_shutdown()
            libo.orc_threads_init(n)
    sweep = [t for t in (1, 2, 4, 8, 16) if t <= ncpu]
    if ncpu not in sweep:
        sweep.append(ncpu)
    per_point = budget_s / (len(sweep) * len(builds))
    best = (0.0, 1, 0, False)
    t_start = time.time()
    tried = []
    for v4 in builds:
        eng = make(depth + 64, v4)
        pos = depth
        for nt in sweep:
            set_threads(nt, v4)
            eng.forward((pos * 131 + 7) % V, pos)       # warmup (first touch of pages)
            pos += 1
            n, t0 = 0, time.perf_counter()
            while n < 2 or (time.perf_counter() - t0 < per_point * 0.6 and n < 96):
                eng.forward((pos * 131 + 7) % V, pos)
                pos += 1
                n += 1
                if pos >= depth + 60:
                    pos = depth
            rate = n / (time.perf_counter() - t0)
            tried.append(f"{'v4' if v4 else 'v3'}/{nt}t {rate:.1f}")
            log(f"cpu baseline ({kind}, {'x86-64-v4' if v4 else 'x86-64-v3'}) {nt} threads: "
                f"{rate:.2f} tok/s over {n} steps")
            if rate > best[0]:
                best = (rate, nt, n, v4)
        eng.close()
        set_threads(1, v4)
    cpu = ""
    try:
        with open("/proc/cpuinfo") as f:
            cpu = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    return {"value": round(best[0], 3), "unit": "tok/s", "cores": best[1], "kind": kind,
            "sample": (f"{best[2]} greedy-shaped decode steps (token stream (pos*131+7)%V) at positions "
                       f"{depth}.. of the same model via {note(best[3])}; best of threads {sweep} and builds "
                       f"[{', '.join(tried)} tok/s] ({time.time() - t_start:.0f} s total) on '{cpu}', "
                       f"{ncpu} cores available")}


GPU_CLI = os.path.join(ROOT, "emberllm_amd", "_cli", "ember")


def cli_bench(path, pp, tg, reps, kv16):
    """`ember bench` (src/main.c:230-294) over libember.so: returns its
    prefill and decode rates (mean and sd over the timed reps), or None
    when the program is absent."""
    import re
    import subprocess
    if not os.path.exists(GPU_CLI):
        return None
    cmd = [GPU_CLI, "bench", path, "--pp", str(pp), "--tg", str(tg), "--reps", str(reps)]
    if kv16:
        cmd += ["--kv-type", "f16"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    if r.returncode != 0:
        raise RuntimeError(f"{' '.join(cmd)} failed ({r.returncode}): {r.stderr[-2000:]}")
    out = {}
    for what, key in (("prefill", "pp"), ("decode", "tg")):
        m = re.search(rf"{what}\s+\({key}(\d+)\):\s+([0-9.]+) tok/s\s+\(\+/- ([0-9.]+)\)", r.stdout)
        if not m:
            raise RuntimeError(f"unexpected ember bench output: {r.stdout}")
        out[what] = (float(m.group(2)), float(m.group(3)))
    log(f"ember bench --pp {pp} --tg {tg} --reps {reps}{' --kv-type f16' if kv16 else ''}: "
        f"prefill {out['prefill'][0]:.1f} tok/s, decode {out['decode'][0]:.1f} +/- {out['decode'][1]:.1f} tok/s")
    return out


def ctypes_bench(eng, pp, tg, reps):
    """The same protocol through ctypes (ember_prefill, then ember_forward
    per token with host logits): mean decode rate of the timed reps."""
    lib, V = eng.lib, eng.vocab
    ids = np.array([(i * 131 + 7) % V for i in range(pp)], np.int32)
    pids = ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int))
    rates = []
    for r in range(1 + reps):
        lib.ember_prefill(eng.m, eng.st, pids, pp, 0)
        t = time.perf_counter()
        for pos in range(pp, pp + tg):
            lib.ember_forward(eng.m, eng.st, (pos * 131 + 7) % V, pos)
        if r:
            rates.append(tg / (time.perf_counter() - t))
    return float(np.mean(rates)), float(np.std(rates, ddof=1))


def quantize_bench(model):
    """ember_quantize_file (src/quant.c:59-125) on an fp32 file of `model`'s
    shape: this library (blocks encoded on the GPU) against the reference's
    requantizer compiled from its sources with its default flags
    (oracle/_ref/libember_ref.so: -O3 -ffast-math, one CPU thread as in the
    reference), each after one untimed run that warms the page cache; both
    write their file to the same directory.  The output must equal, byte for
    byte, the file written by the reference's deterministic build
    (libember_ref_debug.so); its fast-math build rounds some blocks
    differently."""
    import filecmp
    import tempfile
    from emberllm_amd import _native, configs
    if os.path.join(ROOT, "oracle") not in sys.path:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    lib, ref, ref_det = _native.lib(), oracle.reference_lib(debug=False), oracle.reference_lib(debug=True)
    t0 = time.time()
    f32 = configs.model_path(f"{model}_f32", dict(configs.ALL[model], dtype=_native.DT_F32), threads=16)
    mb = os.path.getsize(f32) / 1e6
    log(f"fp32 model {f32} ({mb:.0f} MB) ready in {time.time() - t0:.1f} s")
    res = {}
    with tempfile.TemporaryDirectory(dir=os.path.dirname(f32)) as tmp:
        for name, target in (("q8_0", _native.DT_Q8_0), ("q4_0", _native.DT_Q4_0)):
            out, ref_out = os.path.join(tmp, f"gpu_{name}.ember"), os.path.join(tmp, f"ref_{name}.ember")
            times = {}
            for who, fn, dst, reps in (("gpu", lib.ember_quantize_file, out, 3),
                                       ("ref_cpu", ref.ember_quantize_file, ref_out, 1)):
                assert fn(f32.encode(), dst.encode(), target) == 0, who
                ts = []
                for _ in range(reps):
                    t = time.perf_counter()
                    assert fn(f32.encode(), dst.encode(), target) == 0, who
                    ts.append(time.perf_counter() - t)
                times[who] = float(np.mean(ts))
            det_out = os.path.join(tmp, f"det_{name}.ember")
            assert ref_det.ember_quantize_file(f32.encode(), det_out.encode(), target) == 0
            same = filecmp.cmp(out, det_out, shallow=False)
            res[name] = {"gpu_s": round(times["gpu"], 4), "ref_cpu_s": round(times["ref_cpu"], 3),
                         "speedup": round(times["ref_cpu"] / times["gpu"], 1),
                         "identical_to_reference_deterministic_build": same,
                         "out_MB": round(os.path.getsize(out) / 1e6, 1)}
            for p in (out, ref_out, det_out):
                os.remove(p)
            log(f"quantize {name}: GPU {times['gpu']:.3f} s, reference CPU {times['ref_cpu']:.2f} s, "
                f"file identical to the reference's deterministic build: {same}")
    print(json.dumps({"quantize": res, "model": f"{model}-shape fp32 file", "input_MB": round(mb, 1)}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--model", default="qwen3_06b")
    ap.add_argument("--depth", type=int, default=4096)
    ap.add_argument("--kv", choices=("f32", "f16"), default="f32")
    ap.add_argument("--reps", type=int, default=5, help="timed reps of the ember bench protocol (src/main.c:232)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-only", action="store_true", help="skip the prefill and kernel timings")
    ap.add_argument("--no-api", action="store_true",
                    help="profiling aid: skip the ember_forward protocol (ember bench and its ctypes form); "
                         "the line's value is then the device loop's")
    ap.add_argument("--no-cli", action="store_true",
                    help="profiling aid: skip the ember bench program (its own process); the protocol runs "
                         "through ctypes only")
    ap.add_argument("--sampled-only", action="store_true",
                    help="profiling aid: fill the cache to --depth, run only the device sampling loop "
                         "(T 0.8, top-k 40, top-p 0.9) and print its rate; no JSON line")
    ap.add_argument("--prefill-only", action="store_true",
                    help="profiling aid: only prefill --depth tokens (1 untimed and --steps timed runs) "
                         "and print the rate; no JSON line")
    ap.add_argument("--read-sweep", action="store_true",
                    help="only measure the streaming read bandwidth over buffers of 16 MiB to 4 GiB "
                         "(repeated passes over one buffer: what fits in the 256 MB Infinity Cache is "
                         "re-read from it) and print one JSON line")
    ap.add_argument("--quantize", action="store_true",
                    help="only time ember_quantize_file (blocks encoded on the GPU) on an fp32 file of "
                         "--model's shape, to Q8_0 and Q4_0, beside the reference's CPU requantizer on the "
                         "same file; check the outputs are identical and print one JSON line")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only copy 64 MiB device-to-device 8 times (a kernel of known traffic, for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    args = ap.parse_args()
    if args.calibrate_copy:
        import torch
        src = torch.ones(16 << 20, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "64 MiB device-to-device copy x 8"}))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (the token loop is "
              "single-stream on one MI355X; multi-GPU sharding is a design note only)", file=sys.stderr)
        sys.exit(2)

    from emberllm_amd import _native, configs, emberllm

    lib = _native.lib()
    if lib.ehip_device_count() <= 0:
        print("bench.py: no GPU visible to the HIP runtime", file=sys.stderr)
        sys.exit(1)
    if args.read_sweep:
        # a 2-layer model is enough to own a state; the kernel reads its own buffers
        eng = emberllm.Engine(configs.model_path("t_llama"), ctx=64)
        sweep = {}
        for mib in (16, 32, 64, 128, 192, 256, 384, 512, 1024, 4096):
            reps = max(4, min(200, (8 << 30) // (mib << 20)))   # about 8 GiB read per size
            sweep[mib] = round(eng.measure_read_bw(mib << 20, reps), 1)
            log(f"read {mib} MiB x {reps}: {sweep[mib]:.0f} GB/s")
        eng.close()
        print(json.dumps({"read_sweep_GB_s_by_MiB": sweep, "passes": "about 8 GiB per size after one untimed pass"}))
        return
    if args.quantize:
        quantize_bench(args.model)
        return
    c = configs.ALL[args.model]
    K, W, depth = args.steps, args.warmup, args.depth
    e_kv = 2 if args.kv == "f16" else 4
    t0 = time.time()
    path = configs.model_path(args.model, threads=16)
    log(f"model {path} ready in {time.time() - t0:.1f} s")
    # ---- the headline: ember bench over libember.so (its own process) -----
    cli = None
    if not (args.prefill_only or args.sampled_only or args.no_cli or args.no_api):
        cli = cli_bench(path, depth, K, args.reps, args.kv == "f16")
    ctx = depth + max(K, W) + 2
    t = time.perf_counter()
    # ember_model_load + ember_state_new_ex: the file mapped, every weight
    # repacked and uploaded, the KV cache and scratch allocated
    eng = emberllm.Engine(path, ctx=ctx, kv_fp16=args.kv == "f16")
    load_s = time.perf_counter() - t
    log(f"load (model file to a ready state, ctx {ctx}): {load_s:.2f} s")
    rng = np.random.default_rng(4096)
    V = c["vocab_size"]
    out = {"load_s": load_s}
    if args.prefill_only:
        ids = rng.integers(0, V, depth).astype(np.int32)
        eng.prefill(ids)
        t = time.perf_counter()
        for _ in range(K):
            eng.prefill(ids)
        dt = (time.perf_counter() - t) / K
        log(f"prefill pp{depth}: {dt * 1e3:.3f} ms, {depth / dt:.1f} tok/s (mean of {K})")
        eng.close()
        return

    # ---- prefill --------------------------------------------------------
    def prefill_ttft(n, reps=5, warm=1):
        """ember_prefill of n ids at position 0 plus the first token's
        selection on the host, mean of `reps` after `warm`; returns the last
        logits."""
        ids = rng.integers(0, V, n).astype(np.int32)
        firsts = []
        for r in range(warm + reps):
            t = time.perf_counter()
            lg = eng.prefill(ids)
            int(np.argmax(lg))   # the first generated token
            if r >= warm:
                firsts.append(time.perf_counter() - t)
        out[f"ttft_ms_pp{n}"] = float(np.mean(firsts)) * 1e3
        return lg

    if not args.decode_only:
        prefill_ttft(128)
        log(f"time to first token pp128 {out['ttft_ms_pp128']:.2f} ms")
    lg = prefill_ttft(depth, reps=1 if args.decode_only else 5, warm=0 if args.decode_only else 1)
    log(f"time to first token pp{depth} {out[f'ttft_ms_pp{depth}']:.2f} ms")
    tok0 = int(np.argmax(lg))
    if cli:
        out[f"prefill_tok_s_pp{depth}"], out[f"prefill_tok_s_pp{depth}_sd"] = cli["prefill"]

    def sampled_rate():
        smp = _native.EmberSampler()
        lib.ember_sampler_init(ctypes.byref(smp), 0.8, 0.9, 40, 1234)
        eng.generate_sampled(tok0, depth, W, smp)
        _, mss = eng.generate_sampled(tok0, depth, K, smp)
        lib.ember_sampler_free(ctypes.byref(smp))
        rate = K / (mss / 1e3)
        log(f"decode @{depth} sampled (T 0.8, top-k 40, top-p 0.9): {rate:.1f} tok/s")
        return rate

    if args.sampled_only:
        sampled_rate()
        eng.close()
        return

    # ---- decode at depth: device-resident greedy loop --------------------
    eng.generate_greedy(tok0, depth, W)             # warmup (graph capture happens before the
                                                    # timed region of every call)
    _, ms = eng.generate_greedy(tok0, depth, K)     # synchronises before and after
    out["decode_tok_s_device_loop"] = K / (ms / 1e3)
    out["decode_us_per_step_device_loop"] = ms / K * 1e3
    log(f"decode @{depth}, device greedy loop: {out['decode_tok_s_device_loop']:.1f} tok/s "
        f"({ms / K * 1e3:.1f} us/step)")

    # ---- the ember bench protocol through ctypes ----------------------------
    if not args.no_api:
        out["api_decode_tok_s"], out["api_decode_tok_s_sd"] = ctypes_bench(eng, depth, K, args.reps)
        log(f"ember bench protocol via ctypes @{depth}: {out['api_decode_tok_s']:.1f} tok/s")
    if cli:
        tok_s, tok_sd, harness = cli["decode"][0], cli["decode"][1], "ember bench (src/main.c) over libember.so"
    elif not args.no_api:
        tok_s, tok_sd, harness = out["api_decode_tok_s"], out["api_decode_tok_s_sd"], "ember bench protocol via ctypes"
    else:
        tok_s, tok_sd, harness = out["decode_tok_s_device_loop"], 0.0, "device greedy loop (--no-api)"
    ms_step = 1e3 / tok_s
    mean_bytes = float(np.mean([step_bytes(c, depth + i, e_kv) for i in range(K)]))
    log(f"decode @{depth} ({harness}): {tok_s:.1f} tok/s ({ms_step * 1e3:.1f} us/step), "
        f"{mean_bytes / 1e6:.1f} MB/step -> {tok_s * mean_bytes / HBM_PEAK:.3f} of HBM roofline")

    roof = None
    if not args.decode_only:
        # ---- dominant kernel: attention of one layer at this depth ---------
        reps_k = 200
        fusion = eng.decode_fusion()
        ms_att = eng.time_kernel(0, depth, reps_k)
        ab = attn_launch_bytes(c, depth, e_kv) + (wo_fold_bytes(c) if fusion & 2 else 0)
        ms_head = eng.time_kernel(1, depth, reps_k)
        hb = c["vocab_size"] * (c["dim"] // 32) * 34 + 4 * c["vocab_size"]
        ms_w13 = eng.time_kernel(2, depth, reps_k)
        wb = 2 * c["hidden_dim"] * (c["dim"] // 32) * 34 + 4 * c["hidden_dim"]
        if fusion & 2:   # its prologue reads the wo partials and writes the residual
            wb += 4 * (c["n_kv_heads"] + 1) * c["dim"]
        out["kernels"] = {
            "attention_layer": {"us": ms_att * 1e3, "GB_s": ab / (ms_att / 1e3) / 1e9, "bytes": ab},
            "lm_head": {"us": ms_head * 1e3, "GB_s": hb / (ms_head / 1e3) / 1e9, "bytes": hb},
            "w1w3_swiglu": {"us": ms_w13 * 1e3, "GB_s": wb / (ms_w13 / 1e3) / 1e9, "bytes": wb},
        }
        log(f"kernels: {json.dumps(out['kernels'])}")
        # the measured streaming-read peak, the second reference point for the step's fraction
        peak_meas = eng.measure_read_bw(1 << 30, 10)
        out["hbm_read_peak_measured_GB_s"] = peak_meas
        out["hbm_roofline_frac_step_vs_measured"] = round(tok_s * mean_bytes / (peak_meas * 1e9), 4)
        log(f"measured read peak {peak_meas:.0f} GB/s (1 GiB x 10): the step reaches "
            f"{out['hbm_roofline_frac_step_vs_measured']:.3f} of it")
        achieved = ab / (ms_att / 1e3) / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(achieved / (HBM_PEAK / 1e9), 4),
                "traffic": profiled_traffic("ehip::k_attn_dec", args.model, depth, args.kv),
                "kernel": f"k_attn_dec (split-K GQA attention over one layer's KV cache"
                          f"{', chunk partials merged in-kernel by the last workgroup of each kv head' if fusion & 1 else ''}"
                          f"{', then the wo partials of the kv groups (Q8_0 wo weights read)' if fusion & 2 else ''}) "
                          f"at position {depth}, {ab} algorithmic bytes per launch, mean of {reps_k} "
                          f"launches walking the {c['n_layers']} layers' caches"}

        # ---- sampled decode at depth (T 0.8, top-k 40, top-p 0.9) ---------
        out["decode_tok_s_sampled"] = sampled_rate()
    eng.close()

    if not args.decode_only and not args.no_cli and depth != 128:
        # ---- depth 128: ember bench --pp 128 --------------------------------
        c128 = cli_bench(path, 128, K, args.reps, args.kv == "f16")
        if c128:
            out["prefill_tok_s_pp128"], out["prefill_tok_s_pp128_sd"] = c128["prefill"]
            out["decode_tok_s_depth128"], out["decode_tok_s_depth128_sd"] = c128["decode"]

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(path, c, depth, args.cpu_seconds)

    reps = args.reps
    line = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": K,
        "warmup": K if cli else W,
        "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8 dot / f32 accumulate (Q8_0 weights and activations), f32 KV" if e_kv == 4 else
                 "int8 dot / f32 accumulate (Q8_0 weights and activations), f16 KV",
        "data": "synthetic: seeded N(0,0.02) weights quantized to Q8_0, seeded uniform random prompt ids",
        "config": {"workload": f"{args.model}-shape decode of {K} tokens at depth {depth} after a "
                               f"{depth}-token batched prefill; {args.kv} KV cache",
                   "depth": depth, "kv": args.kv, "parallelism": "single GPU, single stream",
                   "harness": (f"{harness}: {reps} timed reps (after 1 warmup rep) of a pp{depth} prefill "
                               f"then {K} ember_forward calls with host logits; value = mean of the reps' rates")
                              if not args.no_api else f"{harness}: {K} steps after {W} warmup steps",
                   "value_sd": round(tok_sd, 2)},
        "hbm_roofline_frac_step": round(tok_s * mean_bytes / HBM_PEAK, 4),
        "bytes_per_step": int(mean_bytes),
    }
    line.update({k: (round(v, 2) if isinstance(v, float) else v) for k, v in out.items()})
    line["roofline"] = roof
    line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
