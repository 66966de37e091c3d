"""GPU: a seeded sweep of attention shapes against the CPU oracle.

Each case draws a head layout (query heads, KV heads, head size), a cached
prefix, a run length and the row dtype from a fixed seed, then runs the
reference's sequence for a layer: a run appended and attended
(syn_hip_attention), then a few single-token steps on the same cache. Every
output row is compared with oracle.attention_rows (the restatement of
session::execute(op_attention), S/graph/session.hpp:348-374) at the parity
bound, and the cache rows with the oracle's append bit for bit. The draws
cover the paths the host picks between: the causal prefill kernel and its
4-wave form above hd 128, the generic kernel (head sizes not a multiple of 8,
more than 16 query heads per KV head), the split-KV decode kernel with one or
many splits, whole-softmax short sequences and ragged 64-position tiles."""
from __future__ import annotations

import numpy as np
import pytest

import binding as orc
from gpu_util import SYN_F16, SYN_F32, Arena, attention, capi, scratch_for
from helpers import assert_close
from synapse_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def arena():
    a = Arena(1 << 30)
    yield a
    a.close()


def _draw(i):
    g = np.random.default_rng(1000 + i)
    n_kv = int(g.choice([1, 2, 4, 8]))
    group = int(g.choice([1, 2, 4, 8, 20]))
    hd = int(g.choice([8, 12, 16, 24, 36, 40, 64, 72, 96, 128, 160, 256]))
    pos = int(g.choice([0, 0, 1, 63, 64, 130, 700]))
    n = int(g.integers(1, 300))
    steps = int(g.integers(1, 4))
    dtype = SYN_F16 if g.random() < 0.5 else SYN_F32
    return n_kv * group, n_kv, hd, pos, n, steps, dtype


CASES = [_draw(i) for i in range(40)]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_random_layer_against_the_oracle(arena, case):
    n_heads, n_kv, hd, pos, n, steps, dtype = CASES[case]
    total = pos + n + steps
    cfg = wl.Prefill("case", n_heads, n_kv, hd, total, 10000.0)
    q, k, v = wl.prefill_inputs(cfg, seed=case + 1, f16_exact=dtype == SYN_F16)
    mark = arena.top
    cache = capi.kv_state(arena, total, n_kv, hd)
    scratch = scratch_for(arena, n_heads, n_kv, hd, total)
    ok_k, ok_v = orc.new_cache(total, n_kv, hd)
    what = f"H={n_heads} Hkv={n_kv} hd={hd} pos={pos} n={n} dtype={dtype}"
    # rows 0..pos-1, then the run, then single-token steps
    spans = ([(0, pos)] if pos else []) + [(pos, pos + n)] + [(t, t + 1) for t in range(pos + n, total)]
    for a, b in spans:
        got = attention(arena, cache, scratch, q[a:b], k[a:b], v[a:b], a, n_heads, cfg.scale, dtype, dtype)
        want = orc.attention_rows(q[a:b], k[a:b], v[a:b], a, ok_k, ok_v, n_heads, cfg.scale, 8)
        assert_close(got, want, what=f"{what} rows {a}..{b}")
    dk, dv = capi.download_cache(arena, cache, total)
    arena.top = mark
    assert np.array_equal(dk, ok_k[:total]) and np.array_equal(dv, ok_v[:total]), what
