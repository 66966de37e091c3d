"""GPU checks of the graph ops the C++ session added to the device:
op_silu (SYN_SILU, kernels::silu), op_add_bias over every row in one launch
(SYN_ADD_BIAS) and op_softmax (syn_hip_softmax, kernels::softmax,
S/kernels/elementwise.hpp:169-199). Both are pinned by
their closed forms, evaluated in float64 on the same inputs: silu within
4 float ulps (expf, the sum and the quotient each round), softmax within
1e-6 relative per element of exp over the float differences x - max, rows summing to 1,
shift invariance and the one-element row exactly 1."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from gpu_util import Arena, capi, check, lib
from synapse_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def arena():
    a = Arena(64 << 20)
    yield a
    a.close()


def _softmax(arena, x):
    n, size = x.shape
    src = arena.put(x)
    out = arena.alloc(x.nbytes)
    check(lib().syn_hip_softmax(arena.handle, ctypes.byref(capi.SoftmaxDesc(src, out, n, size))))
    return arena.download(out, x.shape, np.float32)


def test_silu_matches_its_closed_form(arena):
    g = wl.rng(31)
    x = np.concatenate([wl.normal(g, (100000,)) * 6, np.array([0.0, -0.0, 88.0, -88.0, 1e-30], np.float32)])
    x = x.astype(np.float32)
    a, out = arena.put(x), arena.alloc(x.nbytes)
    d = capi.ElementwiseDesc(a, 0, out, x.size, capi.SYN_SILU, 0.0)
    check(lib().syn_hip_elementwise(arena.handle, ctypes.byref(d)))
    got = arena.download(out, x.shape, np.float32).astype(np.float64)
    want = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 4 * ulp)


@pytest.mark.parametrize("size", [1, 2, 63, 64, 255, 256, 257, 1000, 32000])
def test_softmax_rows(arena, size):
    g = wl.rng(size)
    x = (wl.normal(g, (5, size)) * 4).astype(np.float32)
    x[1] += 1000.0  # large values: the maximum is subtracted first
    got = _softmax(arena, x).astype(np.float64)
    # x - max rounds in float, as the kernel (and the reference) computes it
    want = np.exp((x - x.max(axis=1, keepdims=True)).astype(np.float64))
    want /= want.sum(axis=1, keepdims=True)
    assert np.all(np.abs(got - want) <= 1e-6 * want + 1e-12)
    assert np.allclose(got.sum(axis=1), 1.0, atol=1e-5)
    if size == 1:
        assert np.all(got == 1.0)


def test_softmax_in_place_and_rejects_partial_overlap(arena):
    x = wl.normal(wl.rng(5), (3, 300)).astype(np.float32)
    off = arena.put(x)
    check(lib().syn_hip_softmax(arena.handle, ctypes.byref(capi.SoftmaxDesc(off, off, 3, 300))))
    got = arena.download(off, x.shape, np.float32)
    np.testing.assert_array_equal(got, _softmax(arena, x))
    bad = capi.SoftmaxDesc(off, off + 4 * 300, 3, 300)
    assert lib().syn_hip_softmax(arena.handle, ctypes.byref(bad)) != 0


@pytest.mark.parametrize("rows,size", [(1, 64), (7, 100), (64, 4096), (3, 1)])
def test_add_bias_broadcasts_every_row(arena, rows, size):
    """SYN_ADD_BIAS (op_add_bias): the same float additions as a row loop,
    bit for bit; a period that does not divide the count is refused."""
    g = wl.rng(rows * size)
    x = wl.normal(g, (rows, size)).astype(np.float32)
    bias = wl.normal(g, (size,)).astype(np.float32)
    a, b, out = arena.put(x), arena.put(bias), arena.alloc(x.nbytes)
    d = capi.ElementwiseDesc(a, b, out, x.size, capi.SYN_ADD_BIAS, 0.0, size, 0)
    check(lib().syn_hip_elementwise(arena.handle, ctypes.byref(d)))
    np.testing.assert_array_equal(arena.download(out, x.shape, np.float32), x + bias[None, :])
    if size > 1:
        bad = capi.ElementwiseDesc(a, b, out, x.size, capi.SYN_ADD_BIAS, 0.0, size + 1, 0)
        assert lib().syn_hip_elementwise(arena.handle, ctypes.byref(bad)) != 0
