"""The HIP path against the committed golden fixtures (tests/golden/*.npz),
through the C ABI, to the parity bound (max-abs 2e-3, relative 1e-2); the
RoPE kernel to the closed-form tolerance of the reference's own test."""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np
import pytest

from gpu_util import SYN_F16, SYN_F32, Arena, SeqDesc, attention, capi, check, lib, put_rows, scratch_for, \
    self_attention, seq_array
from helpers import assert_close

pytestmark = pytest.mark.gpu
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def load(name: str):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def scale_of(hd) -> float:
    return float(np.float32(1) / np.sqrt(np.float32(int(hd))))


@pytest.fixture(scope="module")
def arena():
    a = Arena(256 << 20)
    yield a
    a.close()


def test_c1_tiny_prefill_then_decode(arena):
    fx = load("c1_tiny")
    H, KV, hd, n_pre = (int(fx[k]) for k in ("n_heads", "n_kv", "head_dim", "n_prefill"))
    q, k, v = fx["q"], fx["k"], fx["v"]
    total = q.shape[0]
    cache = capi.kv_state(arena, total, KV, hd)
    scratch = scratch_for(arena, H, KV, hd, total)
    out = [attention(arena, cache, scratch, q[:n_pre], k[:n_pre], v[:n_pre], 0, H, scale_of(hd))]
    for p in range(n_pre, total):
        out.append(attention(arena, cache, scratch, q[p:p + 1], k[p:p + 1], v[p:p + 1], p, H, scale_of(hd)))
    assert_close(np.concatenate(out), fx["out"], what="c1")
    dk, dv = capi.download_cache(arena, cache, total)
    assert np.array_equal(dk, fx["k_cache"]) and np.array_equal(dv, fx["v_cache"])


def test_c2_decode(arena):
    fx = load("c2_decode")
    H, KV, hd, ctx = (int(fx[k]) for k in ("n_heads", "n_kv", "head_dim", "ctx"))
    cache = capi.kv_state(arena, ctx + 1, KV, hd)
    capi.upload_cache(arena, cache, fx["k_cached"], fx["v_cached"])
    out = attention(arena, cache, scratch_for(arena, H, KV, hd, ctx + 1), fx["q"], fx["k"], fx["v"], ctx, H,
                    scale_of(hd))
    assert_close(out, fx["out"], what="c2")


def test_c3_prefill(arena):
    fx = load("c3_prefill")
    H, KV, hd = (int(fx[k]) for k in ("n_heads", "n_kv", "head_dim"))
    q, k, v = (fx[x].astype(np.float32) for x in ("q", "k", "v"))
    cache = capi.kv_state(arena, q.shape[0], KV, hd)
    out = attention(arena, cache, scratch_for(arena, H, KV, hd, q.shape[0]), q, k, v, 0, H, scale_of(hd),
                    SYN_F16, SYN_F16)
    assert_close(out, fx["out"], what="c3")


def test_c4_ragged(arena):
    fx = load("c4_ragged")
    H, KV, hd = int(fx["n_heads"]), int(fx["n_kv"]), int(fx["head_dim"])
    seqs = []
    for i, L in enumerate(fx["lengths"]):
        cache = capi.kv_state(arena, int(L), KV, hd)
        capi.upload_cache(arena, cache, fx[f"k_cache{i}"], fx[f"v_cache{i}"])
        seqs.append(SeqDesc(cache=cache, q_offset=put_rows(arena, fx[f"q{i}"], SYN_F32),
                            out_offset=arena.alloc(H * hd * 4), pos=int(L) - 1))
    arr = seq_array(seqs)
    need = int(lib().syn_hip_attend_batch_scratch_bytes(arr, len(seqs), H))
    scratch = arena.alloc(max(need, 256))
    check(lib().syn_hip_attend_batch(arena.handle, arr, len(seqs), H, scale_of(hd), SYN_F32, scratch, need))
    for i, s in enumerate(seqs):
        assert_close(arena.download(s.out_offset, (1, H * hd), np.float32), fx[f"out{i}"], what=f"c4 seq {i}")


def test_c5_vit(arena):
    fx = load("c5_vit")
    H, hd, n, batch = (int(fx[k]) for k in ("n_heads", "head_dim", "n", "batch"))
    q, k, v = (fx[x].astype(np.float32) for x in ("q", "k", "v"))
    out = self_attention(arena, q, k, v, n, batch, H, scale_of(hd), SYN_F16)
    assert_close(out, fx["out"], what="c5")


@pytest.mark.parametrize("mode", ["normal", "neox", "yarn_ff"])
def test_rope(arena, mode):
    fx = load("rope")
    x, hd, pos = fx["x"], int(fx["head_dim"]), int(fx["pos"])
    mark = arena.top
    in_off = put_rows(arena, x, SYN_F32)
    out_off = arena.alloc(x.nbytes)
    ff_off = put_rows(arena, fx["freq_factors"], SYN_F32) if mode == "yarn_ff" else capi.NO_OFFSET
    sc = fx["yarn"] if mode == "yarn_ff" else [1.0, 0.0, 1.0, 0.0, 0.0]
    d = capi.RopeDesc(in_offset=in_off, out_offset=out_off, freq_factors_offset=ff_off, n=x.shape[0],
                      size=x.shape[1], head_dim=hd, pos=pos, theta_scale=float(fx["theta_scale"]),
                      mode=1 if mode == "neox" else 0, freq_scale=float(sc[0]), ext_factor=float(sc[1]),
                      attn_factor=float(sc[2]), corr_low=float(sc[3]), corr_high=float(sc[4]))
    check(lib().syn_hip_rope(arena.handle, ctypes.byref(d)))
    got = arena.download(out_off, x.shape, np.float32)
    arena.top = mark
    # same angles (repeated f32 multiplication); cos/sin from two libraries
    assert np.max(np.abs(got - fx[mode])) <= 2e-6 * (1 + np.abs(x).max())
