"""GPU: RoPE and the attention temperature folded into the attention call.

syn_hip_attention_rope runs a layer's op_rope(q), op_rope(k),
op_attn_temperature(q) and op_attention (S/graph/session.hpp:337-374) as
one call; a single-token step is one decode kernel that rotates q and the new
K row in LDS. It is checked bit for bit against the separate calls
(syn_hip_rope, syn_hip_attn_temperature, syn_hip_attention) on identical
caches: outputs and every cache row. The runs it does not fuse (several
tokens, head sizes the split-KV kernel does not take) make the separate calls
themselves and must write the rotated rows where the descriptor says.
syn_hip_attn_temperature is checked against the reference's formula
(S/kernels/elementwise.hpp:66-72) evaluated on the host.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from gpu_util import SYN_F32, Arena, attn_desc, capi, check, lib, put_rows, scratch_for
from synapse_amd import workloads as wl
from synapse_amd.capi import AttnRopeDesc, RopeDesc, TemperatureDesc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def arena():
    a = Arena(1 << 30)
    yield a
    a.close()


def _host_temperature(pos: np.ndarray, scale: float, floor_len: int) -> np.ndarray:
    q = np.floor(pos.astype(np.float32) / np.float32(floor_len)).astype(np.float32)
    return (np.log(q.astype(np.float64) + 1.0) * np.float64(np.float32(scale)) + 1.0).astype(np.float32)


def _rope_params(hd, mode, yarn, ff_off):
    sc = [0.25, 1.0, 0.9, 8.0, 23.0] if yarn else [1.0, 0.0, 1.0, 0.0, 0.0]
    theta_scale = float(np.float32(500000.0) ** np.float32(-2.0 / hd))
    return dict(freq_factors_offset=ff_off, theta_scale=theta_scale, mode=mode, freq_scale=sc[0],
                ext_factor=sc[1], attn_factor=sc[2], corr_low=sc[3], corr_high=sc[4])


def _layer(arena, n_heads, n_kv, hd, ctx, n, mode=0, yarn=False, ff=False, temp=None, seed=1):
    """Runs one layer both ways on two caches holding the same ctx rows;
    returns (fused out, separate out, fused cache, separate cache, rotated
    q and k rows the fused call wrote)."""
    g = wl.rng(seed)
    row, qsz = n_kv * hd, n_heads * hd
    kc = wl.to_f16_bits(wl.normal(g, (ctx, row))) if ctx else None
    vc = wl.to_f16_bits(wl.normal(g, (ctx, row))) if ctx else None
    q, k, v = wl.normal(g, (n, qsz)), wl.normal(g, (n, row)), wl.normal(g, (n, row))
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    mark = arena.top
    caches = [capi.kv_state(arena, ctx + n, n_kv, hd) for _ in range(2)]
    if ctx:
        for c in caches:
            capi.upload_cache(arena, c, kc, vc)
    ff_off = put_rows(arena, (1.0 + np.arange(hd // 2) % 4).astype(np.float32), SYN_F32) if ff else capi.NO_OFFSET
    p = _rope_params(hd, mode, yarn, ff_off)
    q_off, k_off, v_off = (put_rows(arena, x, SYN_F32) for x in (q, k, v))
    qr_off, kr_off = arena.alloc(q.nbytes), arena.alloc(k.nbytes)
    outs = [arena.alloc(n * qsz * 4) for _ in range(2)]
    scratch = scratch_for(arena, n_heads, n_kv, hd, ctx + n)
    # Separate calls: rope q, [temperature], rope k, attention.
    for src, dst, size in ((q_off, qr_off, qsz), (k_off, kr_off, row)):
        d = RopeDesc(in_offset=src, out_offset=dst, n=n, size=size, head_dim=hd, pos=ctx, **p)
        check(lib().syn_hip_rope(arena.handle, ctypes.byref(d)))
        if temp is not None and src == q_off:
            t = TemperatureDesc(in_offset=qr_off, out_offset=qr_off, n=n, size=qsz, pos=ctx, floor_len=temp[1],
                                scale=temp[0])
            check(lib().syn_hip_attn_temperature(arena.handle, ctypes.byref(t)))
    d = attn_desc(caches[1], qr_off, kr_off, v_off, outs[1], scratch, n_heads, ctx, n, scale)
    check(lib().syn_hip_attention(arena.handle, ctypes.byref(d)))
    want_qr = arena.download(qr_off, q.shape, np.float32)
    want_kr = arena.download(kr_off, k.shape, np.float32)
    # Fused: the unrotated rows in, rotated rows (if any) to fresh buffers.
    qr2, kr2 = arena.alloc(q.nbytes), arena.alloc(k.nbytes)
    check(lib().syn_hip_fill(arena.handle, qr2, 0, q.nbytes))
    check(lib().syn_hip_fill(arena.handle, kr2, 0, k.nbytes))
    d = attn_desc(caches[0], q_off, k_off, v_off, outs[0], scratch, n_heads, ctx, n, scale)
    r = AttnRopeDesc(q_out_offset=qr2, k_out_offset=kr2, temp_scale=temp[0] if temp else 0.0,
                     temp_floor_len=temp[1] if temp else 0, **p)
    check(lib().syn_hip_attention_rope(arena.handle, ctypes.byref(d), ctypes.byref(r)))
    got = [arena.download(o, (n, qsz), np.float32) for o in outs]
    cache_rows = [capi.download_cache(arena, c, ctx + n) for c in caches]
    rotated = (arena.download(qr2, q.shape, np.float32), arena.download(kr2, k.shape, np.float32))
    arena.top = mark
    return got[0], got[1], cache_rows[0], cache_rows[1], rotated, (want_qr, want_kr)


@pytest.mark.parametrize("n_heads,n_kv,hd,ctx,mode,yarn,ff,temp", [
    (32, 8, 128, 4096, 0, False, False, None),        # config 2 with Llama RoPE
    (32, 8, 128, 4096, 0, False, True, None),         # with frequency factors (Llama 3.1)
    (28, 4, 128, 1000, 1, False, False, None),        # neox pairs (Qwen2)
    (32, 8, 128, 300, 0, True, False, (0.5, 8192)),   # YaRN and the temperature (Mistral 3)
    (4, 2, 16, 15, 0, False, False, (0.1, 8)),        # the tiny models' shape, whole-softmax length
    (8, 4, 64, 0, 1, True, True, (0.1, 1)),           # first position
    (16, 1, 256, 2047, 0, False, False, None),
])
def test_decode_step_fused_equals_separate_calls(arena, n_heads, n_kv, hd, ctx, mode, yarn, ff, temp):
    got, want, cache_f, cache_s, rotated, _ = _layer(arena, n_heads, n_kv, hd, ctx, 1, mode, yarn, ff, temp,
                                                     seed=ctx + hd)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(cache_f[0], cache_s[0]) and np.array_equal(cache_f[1], cache_s[1])
    # One kernel: the rotated rows never leave the chip.
    assert not rotated[0].any() and not rotated[1].any()


@pytest.mark.parametrize("temp", [(0.37, 3), (0.1, 8192), (1.7, 1)])
def test_fused_temperature_equals_separate_over_positions(arena, temp):
    """The fused step's temperature factor is computed on the device by the
    same function as syn_hip_attn_temperature's rows: bit-equal outputs and
    cache rows at many positions, with a floor length above 1 and a nonzero
    scale (factors change every floor_len positions)."""
    for ctx in (1, 2, 3, 5, 8, 13, 21, 34, 55, 89, 127, 128, 129, 200, 377, 610, 987, 1597, 2584, 4095, 4096):
        got, want, cache_f, cache_s, _, _ = _layer(arena, 8, 2, 64, ctx, 1, 0, False, False, temp, seed=ctx)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), ctx
        assert np.array_equal(cache_f[0], cache_s[0]) and np.array_equal(cache_f[1], cache_s[1]), ctx


@pytest.mark.parametrize("n_heads,n_kv,hd,ctx,n,mode,yarn", [
    (32, 8, 128, 100, 37, 0, False),   # a run after 100 cached rows
    (32, 8, 128, 0, 2048, 0, False),   # config 3's run
    (28, 4, 128, 61, 200, 1, True),    # neox pairs, YaRN
    (4, 2, 12, 20, 1, 0, False),       # head size the split-KV kernel does not take
    (6, 2, 20, 0, 5, 1, False),
])
def test_runs_fuse_into_two_launches(arena, n_heads, n_kv, hd, ctx, n, mode, yarn):
    """Several tokens (prefill) and head sizes the split-KV kernel does not
    take: the rotation, temperature and append in one launch, then the
    attention kernel. Outputs and cache rows equal the separate calls; q_out
    holds the rotated, scaled q rows as binary16 (the separate calls' f32
    rows rounded to nearest even); k_out is not written."""
    got, want, cache_f, cache_s, rotated, want_rot = _layer(arena, n_heads, n_kv, hd, ctx, n, mode, yarn, True,
                                                            (0.25, 4), seed=n + hd)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(cache_f[0], cache_s[0]) and np.array_equal(cache_f[1], cache_s[1])
    q16 = rotated[0].reshape(-1).view(np.uint16)[:want_rot[0].size].reshape(want_rot[0].shape)
    assert np.array_equal(q16, want_rot[0].astype(np.float16).view(np.uint16))
    assert not rotated[1].any()


@pytest.mark.parametrize("n,launches", [(2048, 2), (37, 2), (1, 1)])
def test_fused_call_launch_count(arena, n, launches):
    """Captured into a HIP graph, syn_hip_attention_rope records two kernel
    launches for a run of config 3's shape and one for a decode step (the
    separate calls: rope q, rope k, the append, then attention)."""
    n_heads, n_kv, hd, ctx = 32, 8, 128, 64
    g = wl.rng(n)
    row, qsz = n_kv * hd, n_heads * hd
    mark = arena.top
    cache = capi.kv_state(arena, ctx + n, n_kv, hd)
    q_off, k_off, v_off = (put_rows(arena, wl.normal(g, (n, m)), SYN_F32) for m in (qsz, row, row))
    qr, kr, out = arena.alloc(n * qsz * 4), arena.alloc(n * row * 4), arena.alloc(n * qsz * 4)
    scratch = scratch_for(arena, n_heads, n_kv, hd, ctx + n)
    d = attn_desc(cache, q_off, k_off, v_off, out, scratch, n_heads, ctx, n, float(1 / np.sqrt(hd)))
    r = AttnRopeDesc(q_out_offset=qr, k_out_offset=kr, **_rope_params(hd, 0, False, capi.NO_OFFSET))
    arena.sync()
    with capi.HipGraph(arena, lambda: check(lib().syn_hip_attention_rope(arena.handle, ctypes.byref(d),
                                                                         ctypes.byref(r)))) as hg:
        nodes = hg.nodes
    arena.top = mark
    assert nodes == launches


def test_fused_step_rejects_f16_rows(arena):
    hd, n_heads, n_kv = 64, 4, 2
    mark = arena.top
    cache = capi.kv_state(arena, 8, n_kv, hd)
    buf = arena.alloc(1 << 16)
    d = attn_desc(cache, buf, buf, buf, buf + 4096, (buf, 0), n_heads, 0, 1, 0.125, q_dtype=capi.SYN_F16)
    r = AttnRopeDesc(q_out_offset=buf, k_out_offset=buf, **_rope_params(hd, 0, False, capi.NO_OFFSET))
    assert lib().syn_hip_attention_rope(arena.handle, ctypes.byref(d), ctypes.byref(r)) == -1  # SYN_HIP_EINVAL
    arena.top = mark


@pytest.mark.parametrize("pos,n,floor_len,scale", [(0, 4096, 8192, 0.1), (8190, 300, 8192, 0.1), (0, 2048, 1, 0.5),
                                                   (123456, 100, 4, 0.25), (4294967000, 200, 7, 0.3)])
def test_attn_temperature_matches_the_reference_formula(arena, pos, n, floor_len, scale):
    """One launch for n rows; each row's factor computed on the device equals
    the reference's float quotient, double logarithm, float rounding."""
    size = 64
    x = wl.normal(wl.rng(pos % 1000 + n), (n, size))
    mark = arena.top
    off = put_rows(arena, x, SYN_F32)
    out = arena.alloc(x.nbytes)
    d = TemperatureDesc(in_offset=off, out_offset=out, n=n, size=size, pos=pos, floor_len=floor_len, scale=scale)
    check(lib().syn_hip_attn_temperature(arena.handle, ctypes.byref(d)))
    got = arena.download(out, x.shape, np.float32)
    arena.top = mark
    t = _host_temperature(np.arange(pos, pos + n, dtype=np.uint64).astype(np.uint32), scale, floor_len)
    want = (x * t[:, None]).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
