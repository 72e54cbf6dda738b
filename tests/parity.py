"""Parity helpers shared by the GPU tests."""
from __future__ import annotations

import numpy as np

# Attention tolerance from the hot-path contract: against an fp32/fp64-accumulated
# reference, max |err| <= 2e-3 and mean |err| <= 2e-4 (fp16 outputs).
MAX_ABS_TOL = 2e-3
MEAN_ABS_TOL = 2e-4


def assert_attention_close(actual, expected, max_tol=MAX_ABS_TOL, mean_tol=MEAN_ABS_TOL, what=""):
    """actual: fp16 kernel output; expected: float64 oracle output (same shape)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    assert np.isfinite(a).all(), f"{what}: non-finite output"
    err = np.abs(a - e)
    mx = float(err.max()) if err.size else 0.0
    mean = float(err.mean()) if err.size else 0.0
    assert mx <= max_tol and mean <= mean_tol, (
        f"{what}: max abs {mx:.3e} (tol {max_tol}), mean abs {mean:.3e} (tol {mean_tol})")
    return mx, mean
