"""The host C library under AddressSanitizer and UndefinedBehaviorSanitizer,
on the CPU.

tests/host_asan builds the product's host sources (emberllm_amd/csrc/host:
loader, state and forward entry points, sampler, tokenizer, requantizer,
thread-pool symbols) with both sanitizers against ehip_stub.c, a test double
of the device layer that reads every weight byte the real layer uploads and
writes every block the real requantizer writes.  drive.c then runs the call
sequences of the reference's callers: `ember bench` (src/main.c:230-294),
generate and chat (src/main.c:143-221, 296-330: tokenizer, sampled decode
with penalties, continuation prefill, empty prefill) and the ctypes
binding's lookups, on every small variant model and the SmolLM2-135M and
Qwen3-0.6B shapes, and requantizes an F32 model to both encodings and runs
the results.  Any sanitizer report fails the test.
"""
import os
import subprocess

import pytest

from emberllm_amd import configs

HERE = os.path.dirname(os.path.abspath(__file__))
DIR = os.path.join(HERE, "host_asan")


def test_host_library_under_sanitizers(tmp_path):
    r = subprocess.run(["make", "-s", "-C", DIR], capture_output=True, text=True, timeout=300)
    if r.returncode != 0 and "sanitize" in r.stderr:
        pytest.skip(f"the C compiler has no sanitizer runtime: {r.stderr[-500:]}")
    assert r.returncode == 0, r.stderr[-3000:]
    models = [configs.model_path(n) for n in configs.TINY] + \
             [configs.model_path(n, threads=8) for n in ("smollm2_135m", "qwen3_06b")]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([os.path.join(DIR, "_build", "drive"), str(tmp_path)] + models,
                       capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0 and "drive ok" in r.stdout, (r.returncode, r.stderr[-4000:])
    assert "runtime error" not in r.stderr and "AddressSanitizer" not in r.stderr, r.stderr[-4000:]
