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


def _draw_image(i):
    g = np.random.default_rng(2000 + i)
    n = int(g.choice([1, 7, 32, 65, 200, 257, 300, 577]))
    batch = int(g.integers(1, 4))
    n_heads = int(g.choice([1, 2, 4, 12, 16]))
    hd = int(g.choice([8, 12, 32, 40, 64, 80, 128]))
    dtype = SYN_F16 if g.random() < 0.6 else SYN_F32
    return n, batch, n_heads, hd, dtype


IMAGE_CASES = [_draw_image(i) for i in range(24)]


@pytest.mark.parametrize("case", range(len(IMAGE_CASES)))
def test_random_images_against_the_oracle(arena, case):
    """Bidirectional attention (syn_hip_self_attention) over seeded image
    shapes: the head-resident and tiled matrix-core forms, the f32 form and
    the generic one, every image against oracle.self_attention."""
    from gpu_util import self_attention
    n, batch, n_heads, hd, dtype = IMAGE_CASES[case]
    g = wl.rng(3000 + case)
    shape = (batch * n, n_heads * hd)
    q, k, v = (wl.normal(g, shape, 0.5) for _ in range(3))
    if dtype == SYN_F16:
        q, k, v = (x.astype(np.float16).astype(np.float32) for x in (q, k, v))
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    got = self_attention(arena, q, k, v, n, batch, n_heads, scale, dtype)
    for b in range(batch):
        sl = slice(b * n, (b + 1) * n)
        want = orc.self_attention(q[sl], k[sl], v[sl], n_heads, scale, threads=8)
        assert_close(got[sl], want, what=f"image {b} n={n} heads={n_heads} hd={hd} dtype={dtype}")


@pytest.mark.parametrize("case", range(8))
def test_random_ragged_batches_against_the_oracle(arena, case):
    """syn_hip_attend_batch over seeded batches: 1 to 40 sequences (more
    than one launch's table holds) of lengths from 1 to 4000, each output
    against oracle.attend_rows."""
    from gpu_util import SeqDesc, check, lib, put_rows
    from gpu_util import seq_array
    g = np.random.default_rng(4000 + case)
    n_kv = int(g.choice([1, 2, 8]))
    n_heads = n_kv * int(g.choice([1, 4, 8]))
    hd = int(g.choice([64, 128]))
    lengths = [int(x) for x in g.integers(1, 4000, size=int(g.integers(1, 41)))]
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    row = n_kv * hd
    mark = arena.top
    seqs, refs = [], []
    for L in lengths:
        kc = wl.to_f16_bits(wl.normal(g, (L, row)))
        vc = wl.to_f16_bits(wl.normal(g, (L, row)))
        q = wl.normal(g, (1, n_heads * hd))
        cache = capi.kv_state(arena, L, n_kv, hd)
        capi.upload_cache(arena, cache, kc, vc)
        seqs.append(SeqDesc(cache=cache, q_offset=put_rows(arena, q, SYN_F32), out_offset=arena.alloc(n_heads * hd * 4),
                            pos=L - 1))
        refs.append(orc.attend_rows(q, L - 1, kc, vc, n_heads, scale, threads=8))
    arr = seq_array(seqs)
    need = int(lib().syn_hip_attend_batch_scratch_bytes(arr, len(seqs), n_heads))
    scratch = arena.alloc(max(need, 256))
    check(lib().syn_hip_attend_batch(arena.handle, arr, len(seqs), n_heads, scale, SYN_F32, scratch, need))
    for i, s in enumerate(seqs):
        got = arena.download(s.out_offset, (1, n_heads * hd), np.float32)
        assert_close(got, refs[i], what=f"sequence {i} of {len(seqs)} (length {lengths[i]})")
    arena.top = mark
