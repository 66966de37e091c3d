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


def assert_p_rounded_normalised(got, want, n_heads, what=""):
    """A decode output whose probabilities were rounded to binary16 after
    normalisation, as the oracle rounds them. Most heads agree with the
    oracle to f32 noise (the median head's largest error is below 2e-6 of
    the largest output); a head whose probability lands on the other side of
    a binary16 rounding boundary (the two sides' f32 arithmetic differs in
    the last bits) moves by one binary16 step of that weight, below 2e-4.
    Rounding the unnormalised probabilities instead moves every head, by
    1e-5 or more."""
    scale = np.abs(want).max()
    head = (np.abs(got - want) / scale).reshape(n_heads, -1).max(axis=1)
    med = float(np.median(head))
    assert med < 2e-6 and head.max() < 2e-4, (what, med, float(head.max()))
