"""Rows that reach every branch of the Q8_0 / Q4_0 block arithmetic
(src/kernels.c:73-115), shared by the host and device quantizer tests."""
import numpy as np


def edge_rows():
    """Rows of 64 values (two blocks each) that reach every branch."""
    rng = np.random.default_rng(17)
    rows = []
    rows.append(np.zeros(64, np.float32))                                   # amax 0: d 0, inverse 0
    rows.append(np.array([2.5, -2.5, 1.5, -1.5, 0.5, -0.5, 127, 3.5] * 8, np.float32))   # d 1, exact ties
    rows.append(np.array([-8, 8, 0.5, -0.5, 7.5, -7.5, 1, 3] * 8, np.float32))   # Q4: first of equal magnitudes
    rows.append(np.array([8, -8, -0.5, 0.5, -7.5, 7.5, -1, -3] * 8, np.float32))
    rows.append((rng.standard_normal(64) * 1e-7).astype(np.float32))      # fp16-subnormal scale
    rows.append((rng.standard_normal(64) * 1e-40).astype(np.float32))     # fp32-subnormal values
    rows.append((rng.standard_normal(64) * 1e38).astype(np.float32))      # scale past 65504
    rows.append((rng.standard_normal(64) * 1e7).astype(np.float32))
    r = rng.standard_normal(64).astype(np.float32)
    r[5], r[40] = np.inf, -np.inf
    rows.append(r)
    r = rng.standard_normal(64).astype(np.float32)
    r[3], r[33] = np.nan, np.nan
    rows.append(r)
    rows.append(np.full(64, -3.0, np.float32))                              # constant block
    # values at code boundaries: x*inv landing on k + 0.5 after rounding
    a = np.float32(1.3)
    d = a / np.float32(127.0)
    inv = np.float32(1.0) / d
    r = np.concatenate([[a], (np.arange(63, dtype=np.float32) - 31.5) / inv]).astype(np.float32)
    rows.append(r)
    # 1/d infinite (amax below ~3.7e-37): every product infinite, and 0 * inf NaN
    rows.append((rng.standard_normal(64) * 1e-38).astype(np.float32))
    r = np.zeros(64, np.float32)
    r[7], r[40], r[41] = 2e-39, -3e-38, 1e-45
    rows.append(r)
    # d subnormal but 1/d finite
    rows.append((rng.standard_normal(64) * 1e-36).astype(np.float32))
    for s in (1e-3, 0.02, 1.0, 50.0):
        rows.append((rng.standard_normal(64) * s).astype(np.float32))
    return np.stack(rows)
