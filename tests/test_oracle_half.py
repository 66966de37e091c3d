"""Pins the oracle's binary16 conversions (oracle.cpp widen/narrow, restating
S/numeric/half.hpp:18-41 and :46-82).

Checked three ways: against numpy's IEEE-754 binary16 conversion (round to
nearest even, subnormals, overflow to inf) at every binary16 value, its float
neighbours and the halfway points -- the boundary set of the reference's own
test (tests/sdk/kernels_vision.cpp:83-116); against the NaN rule the
reference documents (quiet, sign and top payload bits kept); and, where
oracle/_ref was built from the reference's half.hpp, bit for bit against it.
"""
from __future__ import annotations

import numpy as np
import pytest

import binding as orc


def _boundary_floats() -> np.ndarray:
    """Every finite binary16 value, the midpoints to the next one, and the
    float neighbours of both; plus the float range around the subnormal
    cutoff, 65520 and its neighbour, and the infinities."""
    h = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(f)
    f = f[fin]
    nxt = (h[fin].astype(np.uint32) + 1).astype(np.uint16).view(np.float16).astype(np.float32)
    ok = np.isfinite(nxt) & (np.sign(nxt) == np.sign(f)) & (nxt != 0)
    mid = np.where(ok, (f.astype(np.float64) + nxt.astype(np.float64)) / 2, f).astype(np.float32)
    pts = np.concatenate([f, mid])
    both = np.concatenate([pts, np.nextafter(pts, np.float32(0)), np.nextafter(pts, np.copysign(np.inf, pts))])
    lo = np.float32(2.0**-26).view(np.uint32)
    hi = np.float32(2.0**-23).view(np.uint32)
    sub = np.arange(lo, hi + 1, dtype=np.uint32).view(np.float32)
    extra = np.array([65520.0, np.nextafter(np.float32(65520.0), np.float32(0)), np.inf, -np.inf], np.float32)
    return np.concatenate([both, sub, -sub, extra]).astype(np.float32)


def test_narrow_matches_ieee_round_to_nearest_even():
    x = _boundary_floats()
    got = orc.float_to_fp16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} mismatches, first at {x[bad[0]]!r}: {got[bad[0]]:#06x} vs {want[bad[0]]:#06x}"


def test_widen_is_exact_for_every_half():
    h = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    got = orc.fp16_to_float(h)
    want = h.view(np.float16).astype(np.float32)
    fin = ~np.isnan(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))
    # NaN halves widen to NaN with the payload shifted up and the sign kept.
    nan = ~fin
    bits = got[nan].view(np.uint32)
    hb = h[nan].astype(np.uint32)
    assert np.array_equal(bits, ((hb & 0x8000) << 16) | 0x7F800000 | ((hb & 0x3FF) << 13))


def test_round_trip_of_every_finite_half():
    h = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16)
    keep = np.isfinite(f)
    assert np.array_equal(orc.float_to_fp16(orc.fp16_to_float(h[keep])), h[keep])


def test_nan_is_quiet_and_keeps_sign_and_top_payload():
    bits = np.array([0x7FC00000, 0x7FC02000, 0xFFC02000, 0x7F800001, 0x7FFFFFFF, 0xFF801000], np.uint32)
    got = orc.float_to_fp16(bits.view(np.float32)).astype(np.uint32)
    want = ((bits >> 16) & 0x8000) | 0x7C00 | 0x200 | ((bits >> 13) & 0x3FF)
    assert np.array_equal(got, want)


def test_overflow_edges():
    # 65504 is the largest half; 65520 is the first float that rounds past it.
    x = np.array([65504.0, 65519.996, 65520.0, 1e9, -65520.0], np.float32)
    got = orc.float_to_fp16(x)
    assert list(got) == [0x7BFF, 0x7BFF, 0x7C00, 0x7C00, 0xFC00]


@pytest.mark.skipif(orc.ref_half() is None, reason="oracle/_ref was not built (reference tree absent at build time)")
def test_matches_the_reference_half_hpp_bit_for_bit():
    ref = orc.ref_half()
    x = np.concatenate([_boundary_floats(),
                        np.array([0x7FC00000, 0x7FC02000, 0xFFC02000, 0x7F800001, 0x7FFFFFFF], np.uint32)
                        .view(np.float32)])
    want = np.empty(x.shape, np.uint16)
    ref.ref_float_to_fp16_n(x, want, x.size)
    assert np.array_equal(orc.float_to_fp16(x), want)
    h = np.arange(0x10000, dtype=np.uint32).astype(np.uint16)
    wide = np.empty(h.shape, np.float32)
    ref.ref_fp16_to_float_n(h, wide, h.size)
    assert np.array_equal(orc.fp16_to_float(h).view(np.uint32), wide.view(np.uint32))
