"""Writes the committed golden fixtures tests/golden/*.npz.

Each fixture holds seeded inputs, the CPU oracle's outputs for them (the
restatement of the reference's semantics, oracle/oracle.cpp) and a
double-precision reference on the same binary16-rounded operands (stored
rounded to f32, the *_f64 arrays). The
reference repository holds no attention vectors of its own (its goldens are
whole-model logits), so these are the vectors the HIP path and the oracle
are held to: tests/test_golden.py checks that the oracle still reproduces
them bit for bit and stays within 2e-3 of the double reference, and
tests/test_gpu_golden.py checks the HIP path against them.

    python tests/golden/make_golden.py      # needs oracle/liboracle.so

Shapes are BASELINE.json's configs, truncated where the full size would make
the fixture large: config 1 in full, config 2's heads at 64 cached rows,
config 3's heads at 16 tokens, 3 ragged sequences, 2 ViT images.
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "oracle"))
import binding as orc  # noqa: E402

SEED = 20261201


def rng(tag: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(SEED + tag))


def r16(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float64)


def brute_causal(q, k_rows, v_rows, pos0, n_heads, n_kv, hd, scale):
    """Double precision on binary16-rounded q, K, V; token i sees rows 0..pos0+i."""
    group = n_heads // n_kv
    K = r16(k_rows).reshape(-1, n_kv, hd)
    V = r16(v_rows).reshape(-1, n_kv, hd)
    out = np.zeros(q.shape, np.float64)
    for i in range(q.shape[0]):
        n_pos = pos0 + i + 1
        for h in range(n_heads):
            s = K[:n_pos, h // group] @ r16(q[i, h * hd:(h + 1) * hd]) * scale
            p = np.exp(s - s.max())
            out[i, h * hd:(h + 1) * hd] = (p / p.sum()) @ V[:n_pos, h // group]
    return out


def brute_self(q, k, v, n_heads, scale):
    n, row = q.shape
    hd = row // n_heads
    out = np.zeros((n, row), np.float64)
    for h in range(n_heads):
        sl = slice(h * hd, (h + 1) * hd)
        s = q[:, sl].astype(np.float64) @ k[:, sl].astype(np.float64).T * scale
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, sl] = (p / p.sum(axis=1, keepdims=True)) @ v[:, sl].astype(np.float64)
    return out


def scale_of(hd: int) -> float:
    return float(np.float32(1) / np.sqrt(np.float32(hd)))


def roped(x, hd, pos0, base):
    return orc.rope_rows(x, hd, pos0, orc.rope_theta_scale(base, hd))


def c1_tiny():
    """Config 1: H = Hkv = 8, hd 32, theta 1e4; a 32-token causal prefill at
    position 0, then 32 single-token decode steps on the same cache."""
    H, KV, hd, n_pre, n_dec, base = 8, 8, 32, 32, 32, 10000.0
    total = n_pre + n_dec
    g = rng(1)
    q = roped(g.standard_normal((total, H * hd)).astype(np.float32), hd, 0, base)
    k = roped(g.standard_normal((total, KV * hd)).astype(np.float32), hd, 0, base)
    v = g.standard_normal((total, KV * hd)).astype(np.float32)
    kc, vc = orc.new_cache(total, KV, hd)
    out = [orc.attention_rows(q[:n_pre], k[:n_pre], v[:n_pre], 0, kc, vc, H, scale_of(hd))]
    for p in range(n_pre, total):
        out.append(orc.attention_rows(q[p:p + 1], k[p:p + 1], v[p:p + 1], p, kc, vc, H, scale_of(hd)))
    out = np.concatenate(out)
    return dict(n_heads=H, n_kv=KV, head_dim=hd, n_prefill=n_pre, q=q, k=k, v=v, out=out, k_cache=kc, v_cache=vc,
                out_f64=brute_causal(q, k, v, 0, H, KV, hd, scale_of(hd)))


def c2_decode():
    """Config 2's heads (32 on 8, hd 128, theta 5e5) with 64 cached rows and
    one appended step at position 64."""
    H, KV, hd, ctx, base = 32, 8, 128, 64, 500000.0
    g = rng(2)
    k_rows = roped(g.standard_normal((ctx + 1, KV * hd)).astype(np.float32), hd, 0, base)
    v_rows = g.standard_normal((ctx + 1, KV * hd)).astype(np.float32)
    q = roped(g.standard_normal((1, H * hd)).astype(np.float32), hd, ctx, base)
    kc, vc = orc.new_cache(ctx + 1, KV, hd)
    kc[:ctx] = orc.float_to_fp16(k_rows[:ctx])
    vc[:ctx] = orc.float_to_fp16(v_rows[:ctx])
    k_cached, v_cached = kc[:ctx].copy(), vc[:ctx].copy()
    out = orc.attention_rows(q, k_rows[ctx:], v_rows[ctx:], ctx, kc, vc, H, scale_of(hd))
    return dict(n_heads=H, n_kv=KV, head_dim=hd, ctx=ctx, k_cached=k_cached, v_cached=v_cached, q=q,
                k=k_rows[ctx:], v=v_rows[ctx:], out=out,
                out_f64=brute_causal(q, k_rows, v_rows, ctx, H, KV, hd, scale_of(hd)))


def c3_prefill():
    """Config 3's heads with 16 binary16 tokens, RoPE theta 5e5, causal."""
    H, KV, hd, n, base = 32, 8, 128, 16, 500000.0
    g = rng(3)
    f = lambda x: x.astype(np.float16).astype(np.float32)
    q = f(roped(g.standard_normal((n, H * hd)).astype(np.float32), hd, 0, base))
    k = f(roped(g.standard_normal((n, KV * hd)).astype(np.float32), hd, 0, base))
    v = f(g.standard_normal((n, KV * hd)).astype(np.float32))
    kc, vc = orc.new_cache(n, KV, hd)
    out = orc.attention_rows(q, k, v, 0, kc, vc, H, scale_of(hd))
    return dict(n_heads=H, n_kv=KV, head_dim=hd, q=q.astype(np.float16), k=k.astype(np.float16),
                v=v.astype(np.float16), out=out, out_f64=brute_causal(q, k, v, 0, H, KV, hd, scale_of(hd)))


def c4_ragged():
    """Config 4's heads, 3 sequences of lengths 5, 33, 70 (already cached),
    one query each."""
    H, KV, hd = 32, 8, 128
    lengths = [5, 33, 70]
    g = rng(4)
    fx = {"n_heads": H, "n_kv": KV, "head_dim": hd, "lengths": np.array(lengths, np.int64)}
    for i, L in enumerate(lengths):
        k_rows = roped(g.standard_normal((L, KV * hd)).astype(np.float32), hd, 0, 500000.0)
        v_rows = g.standard_normal((L, KV * hd)).astype(np.float32)
        q = g.standard_normal((1, H * hd)).astype(np.float32)
        kc, vc = orc.float_to_fp16(k_rows), orc.float_to_fp16(v_rows)
        fx[f"k_cache{i}"], fx[f"v_cache{i}"], fx[f"q{i}"] = kc, vc, q
        fx[f"out{i}"] = orc.attend_rows(q, L - 1, kc, vc, H, scale_of(hd))
        fx[f"out_f64_{i}"] = brute_causal(q, k_rows, v_rows, L - 1, H, KV, hd, scale_of(hd))
    return fx


def c5_vit():
    """Config 5's heads (16 of 64, no RoPE, bidirectional), 2 images of 17
    rows, binary16 inputs ~ N(0, 0.5^2)."""
    H, hd, n, batch = 16, 64, 17, 2
    g = rng(5)
    q, k, v = ((g.standard_normal((batch * n, H * hd)) * 0.5).astype(np.float16) for _ in range(3))
    out = np.concatenate([orc.self_attention(q[b * n:(b + 1) * n].astype(np.float32),
                                             k[b * n:(b + 1) * n].astype(np.float32),
                                             v[b * n:(b + 1) * n].astype(np.float32), H, scale_of(hd), threads=4)
                          for b in range(batch)])
    ref = np.concatenate([brute_self(q[b * n:(b + 1) * n], k[b * n:(b + 1) * n], v[b * n:(b + 1) * n], H,
                                     scale_of(hd)) for b in range(batch)])
    return dict(n_heads=H, head_dim=hd, n=n, batch=batch, q=q, k=k, v=v, out=out, out_f64=ref)


def rope_vectors():
    """RoPE of 5 rows of 4 heads of 128 at positions 4090.., normal, neox and
    YaRN with frequency factors."""
    hd, pos, base = 128, 4090, 500000.0
    g = rng(6)
    x = g.standard_normal((5, 4 * hd)).astype(np.float32)
    ts = orc.rope_theta_scale(base, hd)
    ff = (1.0 + np.arange(hd // 2) % 4).astype(np.float32)
    yarn = np.array([0.25, 1.0, 0.9, 8.0, 23.0], np.float32)
    return dict(x=x, head_dim=hd, pos=pos, theta_scale=np.float32(ts), freq_factors=ff, yarn=yarn,
                normal=orc.rope_rows(x, hd, pos, ts), neox=orc.rope_rows(x, hd, pos, ts, mode=1),
                yarn_ff=orc.rope_rows(x, hd, pos, ts, freq_factors=ff, scaling=yarn))


FIXTURES = {"c1_tiny": c1_tiny, "c2_decode": c2_decode, "c3_prefill": c3_prefill, "c4_ragged": c4_ragged,
            "c5_vit": c5_vit, "rope": rope_vectors}


def main() -> None:
    for name, make in FIXTURES.items():
        fx = make()
        # double references are stored rounded to f32: ample for a 2e-3 check
        arrays = {k: (np.asarray(v, np.float32) if "f64" in k else np.asarray(v)) for k, v in fx.items()}
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print(f"wrote {name}.npz")


if __name__ == "__main__":
    main()
