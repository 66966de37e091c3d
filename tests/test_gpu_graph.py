"""Decode steps captured in a HIP graph (capi.HipGraph) replay to the eager
result bit for bit. Each replay follows eager work on the same stream (another
layer's step, a fill that clears the captured step's output) and a
synchronisation, and every replay is checked, as graph replays have to be on
this hardware (a captured memset node has given wrong results after the first
replay; the decode step captures kernel launches only)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from gpu_util import SYN_F32, Arena, AttnDesc, capi, check, lib, scratch_for
from synapse_amd import workloads as wl

pytestmark = pytest.mark.gpu


def _decode_layer(arena, g, n_heads, n_kv, hd, ctx, scratch):
    row = n_kv * hd
    cache = capi.kv_state(arena, ctx + 1, n_kv, hd)
    kc = wl.to_f16_bits(wl.normal(g, (ctx, row)))
    vc = wl.to_f16_bits(wl.normal(g, (ctx, row)))
    capi.upload_cache(arena, cache, kc, vc)
    d = AttnDesc(cache=cache, q_offset=arena.put(wl.normal(g, (n_heads * hd,))),
                 k_offset=arena.put(wl.normal(g, (row,))), v_offset=arena.put(wl.normal(g, (row,))),
                 out_offset=arena.alloc(n_heads * hd * 4), scratch_offset=scratch[0], scratch_bytes=scratch[1],
                 n_heads=n_heads, pos=ctx, n=1, scale=float(np.float32(1) / np.sqrt(np.float32(hd))),
                 q_dtype=SYN_F32, kv_dtype=SYN_F32)
    return d


def test_decode_graph_replays_match_eager():
    n_heads, n_kv, hd, ctx = 32, 8, 128, 1500
    arena = Arena(96 << 20)
    try:
        g = wl.rng(4242)
        scratch = scratch_for(arena, n_heads, n_kv, hd, ctx + 1)
        layers = [_decode_layer(arena, g, n_heads, n_kv, hd, ctx, scratch) for _ in range(3)]
        out_bytes = n_heads * hd * 4
        L = lib()

        def step(d):
            check(L.syn_hip_attention(arena.handle, ctypes.byref(d)))

        for d in layers:
            step(d)
        eager = [arena.download(d.out_offset, (n_heads * hd,), np.float32) for d in layers]
        # Layers 0 and 1 in one graph; layer 2 runs eagerly between replays.
        graph = capi.HipGraph(arena, lambda: [step(layers[0]), step(layers[1])])
        try:
            for rep in range(4):
                for d in layers[:2]:
                    arena.fill(d.out_offset, 0, out_bytes)
                step(layers[2])
                arena.sync()
                graph.launch()
                arena.sync()
                for i in range(2):
                    got = arena.download(layers[i].out_offset, (n_heads * hd,), np.float32)
                    assert np.array_equal(got.view(np.uint32), eager[i].view(np.uint32)), (rep, i)
            got2 = arena.download(layers[2].out_offset, (n_heads * hd,), np.float32)
            assert np.array_equal(got2.view(np.uint32), eager[2].view(np.uint32))
        finally:
            graph.close()
    finally:
        arena.close()
