"""Shared checks for the parity tests."""
from __future__ import annotations

import numpy as np

# The north-star bound: max-abs 2e-3 and relative 1e-2 on
# the f32 output, against the reference's CPU attention. The same 2e-3 bounds
# the reference's own kernel test (tests/sdk/kernels_attention.cpp:228).
ATOL = 2e-3
RTOL = 1e-2


def assert_close(got: np.ndarray, want: np.ndarray, atol: float = ATOL, rtol: float = RTOL, what: str = "") -> None:
    """max |got - want| <= atol, and ||got - want|| / ||want|| <= rtol."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    diff = np.abs(got - want)
    max_abs = float(diff.max()) if diff.size else 0.0
    rel = float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)) if diff.size else 0.0
    worst = np.unravel_index(int(diff.argmax()), diff.shape) if diff.size else None
    assert max_abs <= atol, f"{what}: max-abs {max_abs:.3e} > {atol} at {worst}"
    assert rel <= rtol, f"{what}: relative {rel:.3e} > {rtol}"
