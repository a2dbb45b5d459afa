"""GPU parity of the requantizer: ember_quantize_file, whose blocks are
encoded on the device (ehip_quantize_rows), against the reference's own
ember_quantize_file (src/quant.c:59-125, compiled from its sources:
oracle/_ref) and against the model generator's direct encoding; and
ehip_quantize_rows against the host row quantizers (ember_quant_q8_row /
ember_quant_q4_row, which the CPU suite pins to the reference's quantizer
goldens) on rows built to reach every branch of the block arithmetic
(src/kernels.c:73-115): zero blocks, fp16-subnormal and overflowing scales,
exact .5 ties, equal magnitudes of both signs, infinities and NaNs, and
enough rows to cycle the staging slots several times.  Bytes must match
exactly.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

import oracle
from emberllm_amd import _native, configs
from quant_rows import edge_rows

pytestmark = pytest.mark.gpu
L = None
HAVE_REF = os.path.exists(oracle.reference_path(True))


def lib():
    global L
    if L is None:
        L = _native.lib()
    return L


def say(msg):
    print(f"[gpu-quantize] {msg}", flush=True)
    sys.stdout.flush()


BS = {_native.DT_Q8_0: 34, _native.DT_Q4_0: 18}


def host_blocks(x, dtype):
    rows, cols = x.shape
    out = np.zeros((rows, cols // 32 * BS[dtype]), np.uint8)
    fn = lib().ember_quant_q8_row if dtype == _native.DT_Q8_0 else lib().ember_quant_q4_row
    for r in range(rows):
        row = np.ascontiguousarray(x[r])
        fn(row.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), out[r].ctypes.data, cols)
    return out


def device_blocks(mats):
    """mats: list of (fp32 [rows, cols], dtype) -> list of uint8 block arrays."""
    outs = [np.full((x.shape[0], x.shape[1] // 32 * BS[dt]), 0xA5, np.uint8) for x, dt in mats]
    jobs = (_native.EhipQuantJob * len(mats))()
    for j, ((x, dt), o) in enumerate(zip(mats, outs)):
        jobs[j] = _native.EhipQuantJob(x.ctypes.data, x.shape[0], x.shape[1], dt, o.ctypes.data)
    rc = lib().ehip_quantize_rows(jobs, len(mats))
    assert rc == 0, _native.last_error()
    return outs


@pytest.mark.parametrize("dtype", [_native.DT_Q8_0, _native.DT_Q4_0], ids=["q8_0", "q4_0"])
def test_quantize_rows_edge_cases_match_host(dtype):
    x = edge_rows()
    say(f"{x.shape[0]} edge rows, dtype {dtype}")
    with np.errstate(all="ignore"):
        want = host_blocks(x, dtype)
    got, = device_blocks([(x, dtype)])
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, (bad, got[bad[0]] if bad.size else None, want[bad[0]] if bad.size else None)


def test_quantize_rows_many_jobs_and_slot_cycles():
    """Several jobs of both encodings and widths, together more than ten
    staging slots of fp32, so slots are reused and jobs straddle slots."""
    rng = np.random.default_rng(23)
    shapes = [(3, 32, _native.DT_Q8_0), (70001, 64, _native.DT_Q4_0), (1, 4096, _native.DT_Q8_0),
              (60000, 1024, _native.DT_Q8_0), (5000, 3072, _native.DT_Q4_0), (17, 96, _native.DT_Q8_0)]
    mats = [((rng.standard_normal((r, c)) * rng.uniform(0.01, 2.0, (r, 1))).astype(np.float32), dt)
            for r, c, dt in shapes]
    total = sum(x.nbytes for x, _ in mats)
    say(f"{len(mats)} jobs, {total / 2**20:.0f} MiB of fp32")
    got = device_blocks(mats)
    for (x, dt), g in zip(mats, got):
        if x.shape[0] > 2000:          # the host quantizer is slow in Python: check a spread of rows
            idx = np.unique(np.concatenate([[0, 1, x.shape[0] - 1], rng.integers(0, x.shape[0], 600)]))
        else:
            idx = np.arange(x.shape[0])
        want = host_blocks(x[idx], dt)
        assert np.array_equal(g[idx], want), (x.shape, dt)


def test_quantize_rows_rejects_bad_jobs():
    x = np.zeros((2, 48), np.float32)
    o = np.zeros(200, np.uint8)
    for cols, dt in ((48, _native.DT_Q8_0), (64, 0), (64, 7)):
        job = _native.EhipQuantJob(x.ctypes.data, 1, cols, dt, o.ctypes.data)
        assert lib().ehip_quantize_rows(ctypes.byref(job), 1) != 0
        assert "ehip_quantize_rows" in _native.last_error()


@pytest.mark.parametrize("target", [_native.DT_Q8_0, _native.DT_Q4_0], ids=["q8_0", "q4_0"])
@pytest.mark.parametrize("name", ["t_qwen3", "t_g7"])
def test_quantize_file_equals_reference_and_direct_synthesis(tmp_path, name, target):
    """ember_quantize_file on an fp32 model reproduces, byte for byte, the
    reference's requantizer and the model the generator encodes directly
    (same file rules: 1-D tensors stay fp32, Q4_0 keeps the embedding at
    Q8_0)."""
    base = dict(configs.TINY[name], dtype=_native.DT_F32)
    f32 = configs.model_path(f"hq_f32_{name}", base)
    direct = configs.model_path(f"hq_{target}_{name}", dict(base, dtype=target))
    out = str(tmp_path / "q.ember")
    say(f"{name} -> dtype {target}")
    assert lib().ember_quantize_file(f32.encode(), out.encode(), target) == 0
    got = open(out, "rb").read()
    assert got == open(direct, "rb").read()
    if HAVE_REF:
        ref_out = str(tmp_path / "r.ember")
        assert oracle.reference_lib().ember_quantize_file(f32.encode(), ref_out.encode(), target) == 0
        assert got == open(ref_out, "rb").read()
