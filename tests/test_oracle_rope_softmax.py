"""Pins the oracle's RoPE and softmax (oracle.cpp orc_rope / orc_softmax,
restating S/kernels/attention.hpp:47-129 and S/kernels/elementwise.hpp:174-201).

RoPE is checked against double-precision closed forms with the reference's
own tolerance 1e-5 * (1 + pos) and cases (tests/sdk/kernels_attention.cpp:
37-166): normal and neox pairing, frequency factors, YaRN, the exact identity
at position 0, and neox == normal on the de-interleaved head. A rotation with
a flipped sine, a swapped pair or a wrong theta power fails the closed form.
Softmax is checked against a double-precision softmax and exact small cases.
"""
from __future__ import annotations

import numpy as np
import pytest

import binding as orc


def _x(seed: int, n: int) -> np.ndarray:
    return np.random.Generator(np.random.PCG64(seed)).standard_normal(n).astype(np.float32)


def _rot(x0, x1, theta, mscale=1.0):
    return mscale * (x0 * np.cos(theta) - x1 * np.sin(theta)), mscale * (x0 * np.sin(theta) + x1 * np.cos(theta))


@pytest.mark.parametrize("with_factors", [False, True])
@pytest.mark.parametrize("pos", [0, 1, 7, 100, 4096])
def test_rope_normal_matches_closed_form(pos, with_factors):
    hd, heads, base = 64, 3, 10000.0
    x = _x(5, heads * hd)
    ff = (1.0 + np.arange(hd // 2) % 4).astype(np.float32) if with_factors else None
    ts = orc.rope_theta_scale(base, hd)
    out = orc.rope(x, hd, pos, ts, freq_factors=ff)
    i = np.arange(hd // 2)
    theta = pos * base ** (-2.0 * i / hd) / (ff.astype(np.float64) if with_factors else 1.0)
    xh = x.reshape(heads, hd // 2, 2).astype(np.float64)
    want = np.stack(_rot(xh[..., 0], xh[..., 1], theta), axis=-1).reshape(-1)
    assert np.max(np.abs(out - want)) < 1e-5 * (1 + pos)
    if pos == 0:
        assert np.array_equal(out, x)  # theta = 0: the identity, exactly


@pytest.mark.parametrize("pos", [0, 1, 9, 300])
def test_rope_neox_matches_closed_form(pos):
    hd, heads, base = 64, 2, 1000000.0
    half = hd // 2
    x = _x(6, heads * hd)
    ts = orc.rope_theta_scale(base, hd)
    out = orc.rope(x, hd, pos, ts, mode=1)
    theta = pos * base ** (-2.0 * np.arange(half) / hd)
    xh = x.reshape(heads, hd).astype(np.float64)
    a, b = _rot(xh[:, :half], xh[:, half:], theta)
    want = np.concatenate([a, b], axis=1).reshape(-1)
    assert np.max(np.abs(out - want)) < 1e-5 * (1 + pos)
    if pos == 0:
        assert np.array_equal(out, x)


def test_rope_neox_is_normal_on_the_deinterleaved_head():
    hd = 64
    half = hd // 2
    x = _x(6, hd)
    ts = orc.rope_theta_scale(1000000.0, hd)
    inter = np.empty(hd, np.float32)
    inter[0::2], inter[1::2] = x[:half], x[half:]
    neox = orc.rope(x, hd, 17, ts, mode=1)
    normal = orc.rope(inter, hd, 17, ts, mode=0)
    assert np.array_equal(neox[:half], normal[0::2]) and np.array_equal(neox[half:], normal[1::2])


def test_rope_theta_scale_is_float_pow():
    for base, hd in [(10000.0, 64), (500000.0, 128), (1000000.0, 128)]:
        assert orc.rope_theta_scale(base, hd) == float(np.float32(base) ** np.float32(-2.0 / hd))


def test_yarn_corr_dims_known_answer():
    # floor(64 ln(4 / (0.05 * 2 pi)) / (2 ln 1e4)) = floor(8.84), ceil(22.4)
    assert orc.rope_yarn_corr_dims(64, 4, 10000.0, 0.05, 0.001) == (8.0, 23.0)


@pytest.mark.parametrize("pos", [0, 3, 50])
def test_rope_yarn_matches_closed_form(pos):
    hd, base, factor = 64, 10000.0, 4.0
    half = hd // 2
    x = _x(7, 2 * hd)
    ts = orc.rope_theta_scale(base, hd)
    lo, hi = orc.rope_yarn_corr_dims(hd, 4, base, 0.05, 0.001)
    out = orc.rope(x, hd, pos, ts, scaling=[1.0 / factor, 1.0, 0.9, lo, hi])
    mscale = 0.9 * (1.0 + 0.1 * np.log(factor))
    i = np.arange(half, dtype=np.float64)
    extrap = pos * base ** (-2.0 * i / hd)
    ramp = 1.0 - np.clip((i - lo) / (hi - lo), 0.0, 1.0)
    theta = extrap / factor * (1 - ramp) + extrap * ramp
    xh = x.reshape(2, half, 2).astype(np.float64)
    want = np.stack(_rot(xh[..., 0], xh[..., 1], theta, mscale), axis=-1).reshape(-1)
    assert np.max(np.abs(out - want)) < 1e-5 * (1 + pos)


def test_rope_interpolation_without_ramp_equals_factor_division():
    hd, factor = 64, 4.0
    x = _x(7, 2 * hd)
    ts = orc.rope_theta_scale(10000.0, hd)
    scaled = orc.rope(x, hd, 40, ts, scaling=[1.0 / factor, 0.0, 1.0, 8.0, 23.0])
    plain = orc.rope(x, hd, 40, ts, freq_factors=np.full(hd // 2, factor, np.float32))
    assert np.max(np.abs(scaled - plain)) < 1e-6


def test_rope_rows_rotate_each_row_by_its_position():
    hd = 32
    x = np.stack([_x(8, 2 * hd)] * 3)
    ts = orc.rope_theta_scale(10000.0, hd)
    rows = orc.rope_rows(x, hd, 5, ts)
    for i in range(3):
        assert np.array_equal(rows[i], orc.rope(x[i], hd, 5 + i, ts))


@pytest.mark.parametrize("n", [1, 2, 7, 64, 257, 4097])
def test_softmax_matches_double(n):
    x = (_x(n, n) * 3).astype(np.float32)
    got = orc.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max())
    want = e / e.sum()
    assert np.max(np.abs(got - want) / want) < 1e-5
    assert abs(float(got.astype(np.float64).sum()) - 1.0) < 1e-5 * max(1, np.sqrt(n))


def test_softmax_exact_cases():
    assert np.array_equal(orc.softmax(np.array([3.5], np.float32)), np.array([1.0], np.float32))
    assert np.array_equal(orc.softmax(np.zeros(2, np.float32)), np.full(2, 0.5, np.float32))
    assert np.array_equal(orc.softmax(np.zeros(4, np.float32)), np.full(4, 0.25, np.float32))
    # -inf entries get exactly zero weight
    got = orc.softmax(np.array([0.0, -np.inf, 0.0], np.float32))
    assert np.array_equal(got, np.array([0.5, 0.0, 0.5], np.float32))


def test_softmax_is_invariant_to_a_shift_of_its_max():
    x = _x(3, 100)
    # the max is subtracted first, so adding a representable constant that
    # keeps every difference exact leaves the result unchanged bit for bit
    assert np.array_equal(orc.softmax(x), orc.softmax(x + np.float32(0.0)))
    a = np.round(x * 8) / 8
    assert np.array_equal(orc.softmax(a.astype(np.float32)), orc.softmax((a + 16).astype(np.float32)))
