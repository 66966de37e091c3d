"""GPU parity: causal prefill (flash kernel) and the tiny config's
prefill-then-decode sequence, against the CPU oracle."""
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


def _prefill(arena, n_heads, n_kv, hd, n, pos=0, seed=1, dtype=SYN_F32, check_rows=None, threads=8):
    cfg = wl.Prefill("case", n_heads, n_kv, hd, pos + n, 10000.0)
    q, k, v = wl.prefill_inputs(cfg, seed=seed, f16_exact=dtype == SYN_F16)
    max_ctx = pos + n + 3
    mark = arena.top
    cache = capi.kv_state(arena, max_ctx, n_kv, hd)
    scratch = scratch_for(arena, n_heads, n_kv, hd, max_ctx)
    ok_k, ok_v = orc.new_cache(max_ctx, n_kv, hd)
    if pos:
        # rows 0..pos-1 from an earlier run (the same kernels)
        attention(arena, cache, scratch, q[:pos], k[:pos], v[:pos], 0, n_heads, cfg.scale, dtype, dtype)
        orc.attention_rows(q[:pos], k[:pos], v[:pos], 0, ok_k, ok_v, n_heads, cfg.scale, threads)
    got = attention(arena, cache, scratch, q[pos:], k[pos:], v[pos:], pos, n_heads, cfg.scale, dtype, dtype)
    dk, dv = capi.download_cache(arena, cache, pos + n)
    arena.top = mark
    if check_rows is None:
        want = orc.attention_rows(q[pos:], k[pos:], v[pos:], pos, ok_k, ok_v, n_heads, cfg.scale, threads)
        return got, want, (dk, dv), ok_k, ok_v
    # Large runs: append on the oracle, then attend only sampled query rows.
    for i in range(pos, pos + n):
        orc.lib().orc_kv_append(np.ascontiguousarray(k[i]), np.ascontiguousarray(v[i]), ok_k, ok_v, max_ctx, n_kv,
                                hd, i)
    want = {}
    for (a, b) in check_rows:
        want[(a, b)] = orc.attend_rows(q[pos + a:pos + b], pos + a, ok_k, ok_v, n_heads, cfg.scale, threads)
    return got, want, (dk, dv), ok_k, ok_v


def test_prefill_tiny_config1_then_decode(arena):
    """Config 1: H = Hkv = 8, hd = 32, theta 1e4: a 32-token causal prefill,
    then 32 decode steps appending to the same cache."""
    c = wl.C1_PREFILL
    total = c.n + wl.C1_DECODE_STEPS
    g = wl.rng(wl.SEED + 7)
    q = wl.normal(g, (total, c.n_heads * c.head_dim))
    k = wl.normal(g, (total, c.n_kv * c.head_dim))
    v = wl.normal(g, (total, c.n_kv * c.head_dim))
    cache = capi.kv_state(arena, total, c.n_kv, c.head_dim)
    scratch = scratch_for(arena, c.n_heads, c.n_kv, c.head_dim, total)
    ok_k, ok_v = orc.new_cache(total, c.n_kv, c.head_dim)
    got = attention(arena, cache, scratch, q[:c.n], k[:c.n], v[:c.n], 0, c.n_heads, c.scale)
    want = orc.attention_rows(q[:c.n], k[:c.n], v[:c.n], 0, ok_k, ok_v, c.n_heads, c.scale)
    assert_close(got, want, what="C1 prefill")
    for p in range(c.n, total):
        got = attention(arena, cache, scratch, q[p:p + 1], k[p:p + 1], v[p:p + 1], p, c.n_heads, c.scale)
        want = orc.attention_rows(q[p:p + 1], k[p:p + 1], v[p:p + 1], p, ok_k, ok_v, c.n_heads, c.scale)
        assert_close(got, want, what=f"C1 decode pos {p}")
    dk, dv = capi.download_cache(arena, cache, total)
    assert np.array_equal(dk, ok_k) and np.array_equal(dv, ok_v)


@pytest.mark.parametrize("n_heads,n_kv,hd,n,pos", [
    (32, 8, 128, 300, 0), (32, 8, 128, 129, 0), (8, 8, 64, 200, 0), (16, 4, 128, 77, 100), (4, 2, 16, 50, 0),
    (8, 2, 256, 130, 0), (6, 3, 40, 65, 3), (12, 4, 96, 257, 0), (8, 1, 128, 64, 64), (4, 2, 12, 40, 5),
])
def test_prefill_shapes(arena, n_heads, n_kv, hd, n, pos):
    got, want, (dk, dv), ok_k, ok_v = _prefill(arena, n_heads, n_kv, hd, n, pos, seed=n + hd)
    assert np.array_equal(dk, ok_k[:pos + n]) and np.array_equal(dv, ok_v[:pos + n])
    assert_close(got, want, what=f"prefill {n_heads}/{n_kv}/{hd} n={n} pos={pos}")


def test_prefill_llama3_8b_2048(arena):
    """Config 3 at full size (f16 inputs): every one of the 2048 query rows
    against the oracle (34 GFLOP on the host, about a second on 8 threads),
    so every pairing (r, n_qt - 1 - r) of the 8-wave blocks and their LDS
    merge of the late tile's keys is compared."""
    c = wl.C3
    got, want, _, _, _ = _prefill(arena, c.n_heads, c.n_kv, c.head_dim, c.n, 0, seed=wl.SEED, dtype=SYN_F16)
    assert_close(got, want, what="C3 all rows")


@pytest.mark.parametrize("n,pos", [(2048, 0), (300, 0), (1000, 77)])
def test_prefill_is_deterministic(arena, n, pos):
    """Two runs of the same attend over the same cache give the same bits:
    config 3's shape (every 8-wave block merges its later tile's two
    partials through LDS in a fixed order), an odd tile count (the middle
    tile, whose block has one tile) and a run after cached rows. The
    reference pins thread-count invariance bit for bit
    (tests/sdk/llama_threads.cpp:32-58)."""
    n_heads, n_kv, hd = 32, 8, 128
    cfg = wl.Prefill("case", n_heads, n_kv, hd, pos + n, 500000.0)
    q, k, v = wl.prefill_inputs(cfg, seed=n + pos, f16_exact=True)
    mark = arena.top
    cache = capi.kv_state(arena, pos + n, n_kv, hd)
    scratch = scratch_for(arena, n_heads, n_kv, hd, pos + n)
    if pos:
        attention(arena, cache, scratch, q[:pos], k[:pos], v[:pos], 0, n_heads, cfg.scale, SYN_F16, SYN_F16)
    a = attention(arena, cache, scratch, q[pos:], k[pos:], v[pos:], pos, n_heads, cfg.scale, SYN_F16, SYN_F16)
    b = attention(arena, cache, scratch, q[pos:], None, None, pos, n_heads, cfg.scale, SYN_F16, SYN_F16,
                  append=False)
    c = attention(arena, cache, scratch, q[pos:], None, None, pos, n_heads, cfg.scale, SYN_F16, SYN_F16,
                  append=False)
    arena.top = mark
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(b.view(np.uint32), c.view(np.uint32))


def test_prefill_21_tiles_after_cached_rows(arena):
    """A run of 2600 tokens (21 query tiles of 128, the last ragged) after
    300 cached rows: every row against the oracle."""
    got, want, (dk, dv), ok_k, ok_v = _prefill(arena, 32, 8, 128, 2600, 300, seed=77, dtype=SYN_F16)
    assert np.array_equal(dk, ok_k[:2900]) and np.array_equal(dv, ok_v[:2900])
    assert_close(got, want, what="prefill 2600 at pos 300")


def test_prefill_batch_equals_token_by_token(arena):
    """Batched prefill equals decoding the same tokens one at a time (the
    reference's llama_prefill property, tests/sdk/llama_prefill.cpp:20-52),
    here to the parity bound, since the two paths are different kernels."""
    n_heads, n_kv, hd, n = 32, 8, 128, 40
    cfg = wl.Prefill("case", n_heads, n_kv, hd, n, 500000.0)
    q, k, v = wl.prefill_inputs(cfg, seed=21)
    c1 = capi.kv_state(arena, n, n_kv, hd)
    c2 = capi.kv_state(arena, n, n_kv, hd)
    scratch = scratch_for(arena, n_heads, n_kv, hd, n)
    batched = attention(arena, c1, scratch, q, k, v, 0, n_heads, cfg.scale)
    single = np.concatenate([attention(arena, c2, scratch, q[i:i + 1], k[i:i + 1], v[i:i + 1], i, n_heads,
                                       cfg.scale) for i in range(n)])
    assert_close(batched, single, what="batched vs single")


def test_prefill_is_causal(arena):
    """Changing a later token's K, V leaves every earlier token's output as is."""
    n_heads, n_kv, hd, n = 16, 4, 128, 150
    cfg = wl.Prefill("case", n_heads, n_kv, hd, n, 10000.0)
    q, k, v = wl.prefill_inputs(cfg, seed=33)
    outs = []
    for perturb in (False, True):
        kk, vv = k.copy(), v.copy()
        if perturb:
            kk[100:] += 3.0
            vv[100:] -= 5.0
        c = capi.kv_state(arena, n, n_kv, hd)
        outs.append(attention(arena, c, scratch_for(arena, n_heads, n_kv, hd, n), q, kk, vv, 0, n_heads,
                              cfg.scale))
    assert np.array_equal(outs[0][:100], outs[1][:100])
    assert not np.array_equal(outs[0][100:], outs[1][100:])
