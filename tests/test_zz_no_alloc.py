"""GPU: the allocation-free entry point (syn_hip_attention_noalloc) against
syn_hip_attention through the C ABI.

The allocation-free variant keeps the split-KV decode's partials in the
library's static device array instead of caller scratch; the kernels are the
same, so its outputs and its appended cache rows equal syn_hip_attention's bit
for bit. Two calls in a row, the second with a smaller input (the array keeps
the first call's contents), and a step whose partials exceed the array's size
is an error without a launch.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from gpu_util import SYN_F32, Arena, attn_desc, capi, check, lib, put_rows, scratch_for
from synapse_amd import workloads as wl

pytestmark = pytest.mark.gpu


def _step(arena, fn, cache, scratch, q, k, v, pos, n_heads, scale):
    q_off, k_off, v_off = (put_rows(arena, x, SYN_F32) for x in (q, k, v))
    out_off = arena.alloc(q.size * 4)
    d = attn_desc(cache, q_off, k_off, v_off, out_off, scratch, n_heads, pos, q.shape[0], scale)
    check(fn(arena.handle, ctypes.byref(d)))
    return arena.download(out_off, q.shape, np.float32)


@pytest.mark.parametrize("shapes", [[(32, 8, 128, 4096), (32, 8, 128, 700)], [(16, 4, 64, 2000), (8, 2, 32, 129)]])
def test_noalloc_matches_attention(shapes):
    L = lib()
    with Arena(512 << 20) as arena:
        for n_heads, n_kv, hd, ctx in shapes:
            cfg = wl.Decode("noalloc", n_heads, n_kv, hd, ctx, 500000.0)
            kc, vc, q, k, v = wl.decode_inputs(cfg, seed=ctx + n_heads)
            caches = []
            for _ in range(2):
                c = capi.kv_state(arena, ctx + 1, n_kv, hd)
                capi.upload_cache(arena, c, kc, vc)
                caches.append(c)
            scratch = scratch_for(arena, n_heads, n_kv, hd, ctx + 1)
            want = _step(arena, L.syn_hip_attention, caches[0], scratch, q, k, v, ctx, n_heads, cfg.scale)
            got = _step(arena, L.syn_hip_attention_noalloc, caches[1], (0, 0), q, k, v, ctx, n_heads, cfg.scale)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (n_heads, n_kv, hd, ctx)
            ka, va = capi.download_cache(arena, caches[0], ctx + 1)
            kb, vb = capi.download_cache(arena, caches[1], ctx + 1)
            assert np.array_equal(ka, kb) and np.array_equal(va, vb)


def test_noalloc_prefill_runs_the_same_launches():
    """A run of many tokens needs no scratch: the same result as syn_hip_attention."""
    L = lib()
    with Arena(256 << 20) as arena:
        p = wl.Prefill("noalloc", 8, 2, 64, 300, 10000.0)
        q, k, v = wl.prefill_inputs(p, seed=5)
        outs = []
        for fn in (L.syn_hip_attention, L.syn_hip_attention_noalloc):
            c = capi.kv_state(arena, p.n, p.n_kv, p.head_dim)
            outs.append(_step(arena, fn, c, (0, 0), q, k, v, 0, p.n_heads, p.scale))
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_noalloc_rejects_partials_beyond_its_array():
    """256 KV heads of hd 256 with 16 query heads each: two splits of partials
    need 2 x 256 x 16 x 258 floats = 8.5 MB > 4 MiB."""
    L = lib()
    limit = int(L.syn_hip_attention_noalloc_scratch_limit())
    assert limit == 4 << 20
    n_heads, n_kv, hd, ctx = 4096, 256, 256, 200
    with Arena(256 << 20) as arena:
        cache = capi.kv_state(arena, ctx + 1, n_kv, hd)
        rows = np.zeros((1, n_heads * hd), np.float32)
        kv = np.zeros((1, n_kv * hd), np.float32)
        q_off, k_off, v_off = put_rows(arena, rows, SYN_F32), put_rows(arena, kv, SYN_F32), put_rows(arena, kv, SYN_F32)
        out_off = arena.alloc(rows.size * 4)
        d = attn_desc(cache, q_off, k_off, v_off, out_off, (0, 0), n_heads, ctx, 1, 1.0 / 16)
        assert L.syn_hip_attention_noalloc(arena.handle, ctypes.byref(d)) == -1  # SYN_HIP_EINVAL
        assert b"static scratch" in L.syn_hip_last_error()
