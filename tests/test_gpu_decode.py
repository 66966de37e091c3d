"""GPU parity: single-token decode (split-KV kernel) against the CPU oracle.

Every case runs syn_hip_attention / syn_hip_attend through the C ABI and
compares with oracle.attention_rows (the restatement of
session::execute(op_attention), S/graph/session.hpp:348-374) on the same
seeded inputs, to max-abs 2e-3 / relative 1e-2.
"""
from __future__ import annotations

import numpy as np
import pytest

import binding as orc
from gpu_util import SYN_F16, SYN_F32, Arena, attention, capi, scratch_for
from helpers import assert_close, assert_p_rounded_normalised
from synapse_amd import workloads as wl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def arena():
    a = Arena(1 << 30)
    yield a
    a.close()


def _case(arena, n_heads, n_kv, hd, ctx, seed, q_dtype=SYN_F32, theta=10000.0, max_ctx=None):
    """ctx rows already cached, then one appended step at position ctx."""
    cfg = wl.Decode("case", n_heads, n_kv, hd, ctx, theta)
    kc, vc, q, k, v = wl.decode_inputs(cfg, seed=seed)
    max_ctx = max_ctx or ctx + 1
    mark = arena.top
    cache = capi.kv_state(arena, max_ctx, n_kv, hd)
    if ctx:
        capi.upload_cache(arena, cache, kc, vc)
    scratch = scratch_for(arena, n_heads, n_kv, hd, max_ctx)
    got = attention(arena, cache, scratch, q, k, v, ctx, n_heads, cfg.scale, q_dtype=q_dtype)
    ok_k, ok_v = orc.new_cache(max_ctx, n_kv, hd)
    ok_k[:ctx], ok_v[:ctx] = kc, vc
    want = orc.attention_rows(q, k, v, ctx, ok_k, ok_v, n_heads, cfg.scale)
    dk, dv = capi.download_cache(arena, cache, ctx + 1)
    arena.top = mark
    return got, want, (dk, dv), (ok_k[: ctx + 1], ok_v[: ctx + 1])


def test_decode_llama3_8b_kv4096(arena):
    """Config 2 at full size: H=32, Hkv=8, hd=128, 4096 cached rows + 1."""
    got, want, dev_cache, ref_cache = _case(arena, 32, 8, 128, 4096, seed=wl.SEED, theta=500000.0)
    # The appended row is stored as binary16, bit for bit (kv_append).
    assert np.array_equal(dev_cache[0][-1], ref_cache[0][-1])
    assert np.array_equal(dev_cache[1][-1], ref_cache[1][-1])
    assert_close(got, want, what="C2 decode")


def test_decode_f16_query_matches_f32_query(arena):
    """q given as binary16 is the same computation (the kernel rounds q to f16)."""
    a, _, _, _ = _case(arena, 32, 8, 128, 1000, seed=3, q_dtype=SYN_F32)
    b, _, _, _ = _case(arena, 32, 8, 128, 1000, seed=3, q_dtype=SYN_F16)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("ctx", [0, 1, 30, 31, 32, 33, 127, 128, 129, 255, 256, 257, 1000, 2047, 5000, 9001])
def test_decode_lengths_cross_split_edges(arena, ctx):
    got, want, _, _ = _case(arena, 32, 8, 128, ctx, seed=100 + ctx)
    assert_close(got, want, what=f"ctx {ctx}")


@pytest.mark.parametrize("n_heads,n_kv,hd,ctx", [(4, 2, 16, 0), (4, 2, 16, 15), (32, 8, 128, 31), (32, 8, 128, 32),
                                                (32, 8, 128, 100), (32, 8, 128, 127), (8, 4, 64, 64), (6, 3, 40, 90)])
def test_decode_short_sequences_round_normalised_p(arena, n_heads, n_kv, hd, ctx):
    """Up to 128 rows the kernel takes the softmax whole and rounds the
    normalised p to binary16 where attend_group rounds it
    (S/kernels/attention.hpp:222-227), so it follows the oracle to f32
    rounding but for the odd weight that rounds the other way."""
    got, want, _, _ = _case(arena, n_heads, n_kv, hd, ctx, seed=500 + ctx)
    assert_p_rounded_normalised(got, want, n_heads, what=f"ctx {ctx}")


@pytest.mark.parametrize("ctx", [70000, 150000])
def test_decode_long_contexts(arena, ctx):
    """Long caches take longer splits (512 and 1024 positions here, 137 and
    147 splits), so the merge combines many partials."""
    got, want, _, _ = _case(arena, 32, 8, 128, ctx, seed=7 + ctx, theta=500000.0)
    assert_close(got, want, what=f"ctx {ctx}")


@pytest.mark.parametrize("n_heads,n_kv,hd,ctx", [(16, 1, 128, 32000), (8, 1, 40, 20000), (4, 1, 256, 16500)])
def test_decode_merge_of_up_to_256_splits(arena, n_heads, n_kv, hd, ctx):
    """One KV head keeps the chunk at 128 positions up to 256 splits: the
    merge kernel's weights then come from all four of a lane's split slots
    (250, 157 and 129 splits here), for head sizes whose output quads fill
    the waves unevenly (hd 40: 10 quads over 4 waves)."""
    got, want, _, _ = _case(arena, n_heads, n_kv, hd, ctx, seed=ctx + hd, theta=500000.0)
    assert_close(got, want, what=f"ctx {ctx}, hd {hd}")


@pytest.mark.parametrize("n_heads,n_kv,hd", [(8, 8, 32), (4, 2, 16), (16, 8, 64), (28, 4, 128), (32, 2, 128),
                                             (16, 1, 128), (8, 2, 80), (12, 4, 96), (8, 4, 256), (6, 3, 40)])
def test_decode_head_layouts(arena, n_heads, n_kv, hd):
    got, want, _, _ = _case(arena, n_heads, n_kv, hd, 700, seed=hd + n_heads)
    assert_close(got, want, what=f"{n_heads}/{n_kv}/{hd}")


@pytest.mark.parametrize("n_heads,n_kv,hd", [(4, 2, 12), (32, 1, 64), (6, 2, 20)])
def test_decode_generic_shapes(arena, n_heads, n_kv, hd):
    """head_dim not a multiple of 8, or more than 16 heads per KV head: the
    plain f32 kernel."""
    got, want, _, _ = _case(arena, n_heads, n_kv, hd, 300, seed=7)
    assert_close(got, want, what=f"{n_heads}/{n_kv}/{hd}")


@pytest.mark.parametrize("n_heads,n_kv,hd", [(4, 2, 16), (32, 8, 128), (4, 2, 12)])
def test_decode_position_zero_returns_fp16_v(arena, n_heads, n_kv, hd):
    """One position: softmax is exactly 1, so out is V's binary16 value, bit
    for bit (tests/sdk/kernels_attention.cpp:231-238)."""
    got, _, dev_cache, _ = _case(arena, n_heads, n_kv, hd, 0, seed=11)
    group = n_heads // n_kv
    v16 = dev_cache[1][0].view(np.float16).astype(np.float32)
    want = np.concatenate([v16[(h // group) * hd:(h // group + 1) * hd] for h in range(n_heads)])
    assert np.array_equal(got[0], want)


def test_decode_gqa_growing_cache(arena):
    """The reference's GQA test (tests/sdk/kernels_attention.cpp:178-240):
    n_heads 4, n_kv 2, hd 16, max_ctx 12, decoding positions 0..11 on one
    cache; each step also checked against a double reference on the
    f16-rounded q, K, V within 2e-3."""
    n_heads, n_kv, hd, max_ctx = 4, 2, 16, 12
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    g = wl.rng(9)
    cache = capi.kv_state(arena, max_ctx, n_kv, hd)
    scratch = scratch_for(arena, n_heads, n_kv, hd, max_ctx)
    ok_k, ok_v = orc.new_cache(max_ctx, n_kv, hd)
    ks, vs = [], []
    for pos in range(max_ctx):
        q = wl.normal(g, (1, n_heads * hd))
        k = wl.normal(g, (1, n_kv * hd))
        v = wl.normal(g, (1, n_kv * hd))
        ks.append(k[0])
        vs.append(v[0])
        got = attention(arena, cache, scratch, q, k, v, pos, n_heads, scale)
        want = orc.attention_rows(q, k, v, pos, ok_k, ok_v, n_heads, scale)
        assert_close(got, want, what=f"pos {pos}")
        r = lambda x: orc.round16(np.asarray(x)).astype(np.float64)
        for h in range(n_heads):
            gk = h // (n_heads // n_kv)
            s = np.array([r(q[0, h * hd:(h + 1) * hd]) @ r(ks[t][gk * hd:(gk + 1) * hd]) for t in range(pos + 1)])
            p = np.exp(s * scale - (s * scale).max())
            ref = (p / p.sum()) @ np.stack([r(vs[t][gk * hd:(gk + 1) * hd]) for t in range(pos + 1)])
            assert np.max(np.abs(got[0, h * hd:(h + 1) * hd] - ref)) < 2e-3


@pytest.mark.parametrize("ctx", [0, 1, 31, 127, 128, 129, 4000, 4096])
def test_decode_ignores_slots_from_the_new_row_on(arena, ctx):
    """Every cache slot from the step's position on holds NaN before the step,
    K rows and V^T columns up to the row stride alike. The kernel must read
    none of them: the new row's slot is overwritten by the step, the rest lie
    past the sequence."""
    n_heads, n_kv, hd = 32, 8, 128
    cfg = wl.Decode("case", n_heads, n_kv, hd, ctx, 500000.0)
    kc, vc, q, k, v = wl.decode_inputs(cfg, seed=60 + ctx)
    max_ctx = ctx + 40
    mark = arena.top
    cache = capi.kv_state(arena, max_ctx, n_kv, hd)
    nan16 = np.uint16(0x7E00)
    kfull = np.full((max_ctx, n_kv * hd), nan16, dtype=np.uint16)
    kfull[:ctx] = kc
    arena.upload(cache.k_offset, kfull)
    vt = np.full((n_kv * hd, cache.ctx_stride), nan16, dtype=np.uint16)
    vt[:, :ctx] = vc.T
    arena.upload(cache.v_offset, vt)
    scratch = scratch_for(arena, n_heads, n_kv, hd, max_ctx)
    got = attention(arena, cache, scratch, q, k, v, ctx, n_heads, cfg.scale)
    dk, dv = capi.download_cache(arena, cache, ctx + 1)
    arena.top = mark
    ok_k, ok_v = orc.new_cache(ctx + 1, n_kv, hd)
    ok_k[:ctx], ok_v[:ctx] = kc, vc
    want = orc.attention_rows(q, k, v, ctx, ok_k, ok_v, n_heads, cfg.scale)
    assert np.isfinite(got).all()
    assert np.array_equal(dk[ctx], ok_k[ctx]) and np.array_equal(dv[ctx], ok_v[ctx])
    assert_close(got, want, what=f"NaN past ctx {ctx}")


def test_decode_is_deterministic(arena):
    """Fixed split count and merge order: two runs agree bit for bit."""
    a, _, _, _ = _case(arena, 32, 8, 128, 6000, seed=5)
    b, _, _, _ = _case(arena, 32, 8, 128, 6000, seed=5)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("ctx", [0, 127, 128, 4096])
def test_decode_step_with_f16_rows(arena, ctx):
    """A step whose new K, V row arrives as binary16 (kv_dtype f16) stores
    and attends the same halves as the f32 row it rounds from."""
    n_heads, n_kv, hd = 32, 8, 128
    cfg = wl.Decode("case", n_heads, n_kv, hd, ctx, 500000.0)
    kc, vc, q, k, v = wl.decode_inputs(cfg, seed=40 + ctx)
    k, v = (x.astype(np.float16).astype(np.float32) for x in (k, v))
    outs, caches = [], []
    for kv_dtype in (SYN_F32, SYN_F16):
        mark = arena.top
        cache = capi.kv_state(arena, ctx + 1, n_kv, hd)
        if ctx:
            capi.upload_cache(arena, cache, kc, vc)
        scratch = scratch_for(arena, n_heads, n_kv, hd, ctx + 1)
        outs.append(attention(arena, cache, scratch, q, k, v, ctx, n_heads, cfg.scale, kv_dtype=kv_dtype))
        caches.append(capi.download_cache(arena, cache, ctx + 1))
        arena.top = mark
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(caches[0][0], caches[1][0]) and np.array_equal(caches[0][1], caches[1][1])
    ok_k, ok_v = orc.new_cache(ctx + 1, n_kv, hd)
    ok_k[:ctx], ok_v[:ctx] = kc, vc
    want = orc.attention_rows(q, k, v, ctx, ok_k, ok_v, n_heads, cfg.scale)
    assert_close(outs[1], want, what=f"f16 rows ctx {ctx}")

