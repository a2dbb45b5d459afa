"""The reference's own command-line program over libember.so.

`emberllm_amd/_cli/ember` is the reference's unmodified src/main.c,
src/server.c and src/json.c linked against this library (emberllm_amd/Makefile,
target `cli`); `oracle/_ref/ember_cli` is the same program built entirely
from the reference's sources on the CPU (oracle/ref.mk).  Both are built in
the development container, where the reference's sources are, and run here.

On the small variant models (whose logits match the reference's
deterministic build to ~4e-8) the two programs must print the same greedy
completion (src/main.c:143-221), and the reference's OpenAI-style server
(src/server.c:232-416) must answer a chat completion with the same text from
both.  A sampled completion can part ways wherever a draw lands within the
last bits of a running-sum boundary, as the reference's own optimized build
(`oracle/_ref/ember_cli_o3`) does from its deterministic one on 1 of 8 seeds
of t_qwen3 at T 0.9, top-k 40, top-p 0.95; over 8 seeds the GPU build must
reproduce the deterministic build's completions at least as often as the
optimized build does, less one.  `ember bench` (src/main.c:230-294) must run
on the GPU build, and `ember quantize` (src/main.c:527-531) must write the
same file as the reference program.
"""
import json
import os
import socket
import subprocess
import sys
import time
import urllib.request

import pytest

from emberllm_amd import configs

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GPU_CLI = os.path.join(ROOT, "emberllm_amd", "_cli", "ember")
REF_CLI = os.path.join(ROOT, "oracle", "_ref", "ember_cli")
REF_O3_CLI = os.path.join(ROOT, "oracle", "_ref", "ember_cli_o3")

needs_clis = pytest.mark.skipif(
    not all(os.path.exists(p) for p in (GPU_CLI, REF_CLI, REF_O3_CLI)),
    reason="the command-line programs are built where the reference's sources are "
           "(make -C emberllm_amd cli; make -C oracle -f ref.mk)")


def say(msg):
    print(f"[gpu-cli] {msg}", flush=True)
    sys.stdout.flush()


def run(cli, args, timeout=120):
    r = subprocess.run([cli] + args, capture_output=True, text=False, timeout=timeout)
    assert r.returncode == 0, (cli, args, r.returncode, r.stderr[-2000:])
    return r.stdout


@needs_clis
@pytest.mark.parametrize("name,extra", [
    ("t_llama", []),
    ("t_qwen3", []),
    ("t_q4", []),
    ("t_g7", ["--kv-type", "f16"]),
], ids=["t_llama", "t_qwen3", "t_q4", "t_g7-f16kv"])
def test_greedy_generate_matches_the_reference_program(name, extra):
    path = configs.model_path(name)
    args = ["generate", path, "-p", "Once upon a time", "-n", "32", "--threads", "1", "-t", "0"] + extra
    say(f"generate {name} greedy {' '.join(extra)}")
    gpu, ref = run(GPU_CLI, args), run(REF_CLI, args)
    say(f"{name}: {gpu[:80]!r}")
    assert gpu == ref, (gpu, ref)


@needs_clis
@pytest.mark.parametrize("name,sampling", [
    ("t_qwen3", ["-t", "0.9", "--top-k", "40", "--top-p", "0.95"]),
    ("t_g7", ["-t", "0.8", "--top-k", "0", "--top-p", "0.9", "--kv-type", "f16"]),
], ids=["t_qwen3-k40", "t_g7-k0-f16kv"])
def test_sampled_generate_agrees_like_the_reference_builds(name, sampling):
    path = configs.model_path(name)
    gpu_same = o3_same = 0
    for seed in range(1, 9):
        args = ["generate", path, "-p", "Once upon a time", "-n", "32", "--threads", "1", "--seed", str(seed)] + sampling
        ref = run(REF_CLI, args)
        gpu_same += run(GPU_CLI, args) == ref
        o3_same += run(REF_O3_CLI, args) == ref
    say(f"{name} {' '.join(sampling)}: 8 seeds, GPU build = deterministic reference on {gpu_same}, "
        f"the reference's optimized build on {o3_same}")
    assert gpu_same >= o3_same - 1, (gpu_same, o3_same)


@needs_clis
def test_bench_runs_on_the_gpu_build():
    path = configs.model_path("t_qwen3")
    out = run(GPU_CLI, ["bench", path, "--pp", "32", "--tg", "16", "--reps", "2", "--threads", "1"])
    text = out.decode(errors="replace")
    say(text.strip().replace("\n", " | "))
    assert "prefill (pp32)" in text and "decode  (tg16)" in text, text


@needs_clis
@pytest.mark.parametrize("target", ["q8_0", "q4_0"])
def test_quantize_command_writes_the_reference_programs_file(tmp_path, target):
    """`ember quantize` (src/main.c:527-531): the GPU build's file equals the
    one the reference program writes, byte for byte."""
    f32 = configs.model_path("hq_f32_t_qwen3", dict(configs.TINY["t_qwen3"], dtype=0))
    outs = []
    for tag, cli in (("gpu", GPU_CLI), ("ref", REF_CLI)):
        out = str(tmp_path / f"{tag}.ember")
        run(cli, ["quantize", f32, out, target])
        outs.append(open(out, "rb").read())
    say(f"quantize {target}: {len(outs[0])} bytes")
    assert outs[0] == outs[1]


def _free_port():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _serve(cli, path):
    port = _free_port()
    proc = subprocess.Popen([cli, "serve", path, "--host", "127.0.0.1", "--port", str(port), "--threads", "1",
                             "-n", "16"], stdout=subprocess.DEVNULL, stderr=subprocess.PIPE)
    deadline = time.time() + 90
    while time.time() < deadline:
        if proc.poll() is not None:
            raise AssertionError(f"server exited with {proc.returncode}: {proc.stderr.read()[-2000:]}")
        try:
            with urllib.request.urlopen(f"http://127.0.0.1:{port}/health", timeout=2) as r:
                if r.status == 200:
                    return proc, port
        except OSError:
            time.sleep(0.5)
    proc.kill()
    raise AssertionError("server did not answer /health within 90 s")


def _chat(port, content):
    body = json.dumps({"messages": [{"role": "user", "content": content}], "max_tokens": 12,
                       "temperature": 0}).encode()
    req = urllib.request.Request(f"http://127.0.0.1:{port}/v1/chat/completions", data=body,
                                 headers={"Content-Type": "application/json"})
    with urllib.request.urlopen(req, timeout=60) as r:
        return json.loads(r.read())


@needs_clis
def test_server_answers_like_the_reference_program():
    path = configs.model_path("t_qwen3")
    answers = []
    for cli in (GPU_CLI, REF_CLI):
        proc, port = _serve(cli, path)
        try:
            answers.append(_chat(port, "Tell me a story"))
        finally:
            proc.terminate()
            try:
                proc.wait(timeout=20)
            except subprocess.TimeoutExpired:
                proc.kill()
                proc.wait(timeout=20)
    gpu, ref = (a["choices"][0]["message"]["content"] for a in answers)
    say(f"server answer {gpu!r}")
    assert gpu == ref, (gpu, ref)
    assert answers[0]["choices"][0]["finish_reason"] == answers[1]["choices"][0]["finish_reason"]
