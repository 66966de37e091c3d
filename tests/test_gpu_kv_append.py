"""GPU: syn_hip_kv_append, the run's append (S/kernels/attention.hpp:165-175).

K rows land in the cache's row-major K block, V rows transposed in V^T, both
rounded to binary16 (numpy's float16 conversion rounds to nearest even, as
the device does). Runs start anywhere on the cache's 64-position tile grid,
rows come as f32 or binary16, aligned (vector loads) or 4 bytes off (the
element path), head sizes whose rows are not a multiple of 8 included; every
cache position outside the run must keep what it held."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from gpu_util import capi, lib
from synapse_amd import workloads as wl
from synapse_amd.capi import SYN_F16, SYN_F32, check

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def arena():
    a = capi.Arena(256 << 20)
    yield a
    a.close()


def _run(arena, max_ctx, n_kv, hd, pos0, n, dtype, misalign):
    g = wl.rng(pos0 * 7 + n + hd + dtype)
    row = n_kv * hd
    cache = capi.kv_state(arena, max_ctx, n_kv, hd)
    # Fill the whole state with a known pattern first.
    old_k = g.integers(0, 0x7bff, size=(max_ctx, row), dtype=np.uint16)
    old_v = g.integers(0, 0x7bff, size=(max_ctx, row), dtype=np.uint16)
    capi.upload_cache(arena, cache, old_k, old_v)
    k = wl.normal(g, (n, row))
    v = wl.normal(g, (n, row))
    np_t = np.float32 if dtype == SYN_F32 else np.float16
    k_in, v_in = k.astype(np_t), v.astype(np_t)
    size = np.dtype(np_t).itemsize
    offs = []
    for x in (k_in, v_in):
        base = arena.alloc(x.nbytes + 16)
        off = base + misalign
        if x.nbytes:
            arena.upload(off, x.view(np.uint8).reshape(-1))
        offs.append(off)
    assert all(o % size == 0 for o in offs)
    check(lib().syn_hip_kv_append(arena.handle, ctypes.byref(cache), offs[0], offs[1], n, pos0, dtype))
    got_k, got_v = capi.download_cache(arena, cache, max_ctx)
    want_k, want_v = old_k.copy(), old_v.copy()
    want_k[pos0:pos0 + n] = k_in.astype(np.float16).view(np.uint16)
    want_v[pos0:pos0 + n] = v_in.astype(np.float16).view(np.uint16)
    return got_k, got_v, want_k, want_v


@pytest.mark.parametrize("max_ctx,n_kv,hd,pos0,n", [
    (2048, 8, 128, 0, 2048),     # config 3's run
    (300, 8, 128, 100, 37),      # both ends ragged on the 64-position grid
    (200, 2, 64, 63, 2),         # a run across one tile edge
    (129, 4, 128, 128, 1),       # the last position alone
    (96, 2, 12, 5, 70),          # rows of 24 elements: part of a 64-feature tile
    (96, 3, 20, 17, 40),         # rows of 60 elements: binary16 rows not 16-byte multiples
    (5000, 1, 256, 4000, 999),
])
@pytest.mark.parametrize("dtype", [SYN_F32, SYN_F16])
@pytest.mark.parametrize("misalign", [0, 4])
def test_kv_append_writes_exactly_the_run(arena, max_ctx, n_kv, hd, pos0, n, dtype, misalign):
    mark = arena.top
    got_k, got_v, want_k, want_v = _run(arena, max_ctx, n_kv, hd, pos0, n, dtype, misalign)
    arena.top = mark
    assert np.array_equal(got_k, want_k)
    assert np.array_equal(got_v, want_v)


def test_kv_append_of_nothing_is_a_no_op(arena):
    mark = arena.top
    got_k, got_v, want_k, want_v = _run(arena, 64, 2, 64, 10, 0, SYN_F32, 0)
    arena.top = mark
    assert np.array_equal(got_k, want_k) and np.array_equal(got_v, want_v)
