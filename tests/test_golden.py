"""The oracle against the committed golden fixtures (tests/golden/*.npz,
written by tests/golden/make_golden.py): it must reproduce every stored
output bit for bit (a change to the oracle that moves a single rounding shows
up here), and every stored output must lie within the reference's 2e-3 of
the fixture's double-precision attention on the same binary16 operands."""
from __future__ import annotations

import pathlib

import numpy as np
import pytest

import binding as orc

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"


def load(name: str):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def scale_of(hd) -> float:
    return float(np.float32(1) / np.sqrt(np.float32(int(hd))))


def test_c1_tiny_prefill_then_decode():
    fx = load("c1_tiny")
    H, KV, hd, n_pre = (int(fx[k]) for k in ("n_heads", "n_kv", "head_dim", "n_prefill"))
    q, k, v = fx["q"], fx["k"], fx["v"]
    kc, vc = orc.new_cache(q.shape[0], KV, hd)
    out = [orc.attention_rows(q[:n_pre], k[:n_pre], v[:n_pre], 0, kc, vc, H, scale_of(hd))]
    for p in range(n_pre, q.shape[0]):
        out.append(orc.attention_rows(q[p:p + 1], k[p:p + 1], v[p:p + 1], p, kc, vc, H, scale_of(hd)))
    out = np.concatenate(out)
    assert np.array_equal(out, fx["out"])
    assert np.array_equal(kc, fx["k_cache"]) and np.array_equal(vc, fx["v_cache"])
    assert np.max(np.abs(fx["out"] - fx["out_f64"])) < 2e-3


def test_c2_decode():
    fx = load("c2_decode")
    H, KV, hd, ctx = (int(fx[k]) for k in ("n_heads", "n_kv", "head_dim", "ctx"))
    kc, vc = orc.new_cache(ctx + 1, KV, hd)
    kc[:ctx], vc[:ctx] = fx["k_cached"], fx["v_cached"]
    out = orc.attention_rows(fx["q"], fx["k"], fx["v"], ctx, kc, vc, H, scale_of(hd))
    assert np.array_equal(out, fx["out"])
    assert np.max(np.abs(fx["out"] - fx["out_f64"])) < 2e-3


def test_c3_prefill():
    fx = load("c3_prefill")
    H, KV, hd = (int(fx[k]) for k in ("n_heads", "n_kv", "head_dim"))
    q, k, v = (fx[x].astype(np.float32) for x in ("q", "k", "v"))
    kc, vc = orc.new_cache(q.shape[0], KV, hd)
    out = orc.attention_rows(q, k, v, 0, kc, vc, H, scale_of(hd), threads=8)
    assert np.array_equal(out, fx["out"])
    assert np.max(np.abs(fx["out"] - fx["out_f64"])) < 2e-3


def test_c4_ragged():
    fx = load("c4_ragged")
    H, hd = int(fx["n_heads"]), int(fx["head_dim"])
    for i, L in enumerate(fx["lengths"]):
        out = orc.attend_rows(fx[f"q{i}"], int(L) - 1, fx[f"k_cache{i}"], fx[f"v_cache{i}"], H, scale_of(hd))
        assert np.array_equal(out, fx[f"out{i}"])
        assert np.max(np.abs(out - fx[f"out_f64_{i}"])) < 2e-3


def test_c5_vit():
    fx = load("c5_vit")
    H, hd, n = int(fx["n_heads"]), int(fx["head_dim"]), int(fx["n"])
    for b in range(int(fx["batch"])):
        sl = slice(b * n, (b + 1) * n)
        out = orc.self_attention(*(fx[x][sl].astype(np.float32) for x in ("q", "k", "v")), H, scale_of(hd),
                                 threads=3)
        assert np.array_equal(out, fx["out"][sl])
    assert np.max(np.abs(fx["out"] - fx["out_f64"])) <= 1e-5


@pytest.mark.parametrize("mode", ["normal", "neox", "yarn_ff"])
def test_rope(mode):
    fx = load("rope")
    hd, pos, ts = int(fx["head_dim"]), int(fx["pos"]), float(fx["theta_scale"])
    kw = {"normal": {}, "neox": {"mode": 1},
          "yarn_ff": {"freq_factors": fx["freq_factors"], "scaling": fx["yarn"]}}[mode]
    assert np.array_equal(orc.rope_rows(fx["x"], hd, pos, ts, **kw), fx[mode])
