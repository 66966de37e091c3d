"""The benchmark configurations and their seeded synthetic inputs.

Shapes are BASELINE.json's five configs; every input is drawn from numpy's
PCG64 generator with a recorded seed, so the GPU run and the CPU baseline
see identical data. RoPE on synthetic K and Q uses float64 angles
pos * base^(-2i/hd) in normal (interleaved-pair) mode; the inputs only need
to be RoPE-shaped data, not bit-exact rotations.
"""
from __future__ import annotations

import dataclasses

import numpy as np

SEED = 20261201


@dataclasses.dataclass(frozen=True)
class Decode:
    """One decode step: n_heads query heads over n_kv cached heads, `ctx`
    rows already cached; the step appends row `ctx` and attends ctx+1 rows."""
    name: str
    n_heads: int
    n_kv: int
    head_dim: int
    ctx: int
    theta: float

    @property
    def scale(self) -> float:
        return float(np.float32(1.0) / np.sqrt(np.float32(self.head_dim)))

    def kv_bytes(self) -> int:
        """Algorithmic HBM bytes of one step: K and V of ctx+1 rows (f16),
        q (f32), the new k, v rows (f32) and out (f32)."""
        row = self.n_kv * self.head_dim
        return 2 * (self.ctx + 1) * row * 2 + self.n_heads * self.head_dim * 4 * 2 + 2 * row * 4

    def flops(self) -> int:
        return 4 * self.n_heads * self.head_dim * (self.ctx + 1)


@dataclasses.dataclass(frozen=True)
class Prefill:
    name: str
    n_heads: int
    n_kv: int
    head_dim: int
    n: int
    theta: float

    @property
    def scale(self) -> float:
        return float(np.float32(1.0) / np.sqrt(np.float32(self.head_dim)))

    def flops(self) -> int:
        """Causal pairs only (j <= i): 4 * H * hd * n(n+1)/2."""
        return 4 * self.n_heads * self.head_dim * self.n * (self.n + 1) // 2


@dataclasses.dataclass(frozen=True)
class Ragged:
    name: str
    n_seqs: int
    n_heads: int
    n_kv: int
    head_dim: int
    lo: int
    hi: int
    theta: float

    @property
    def scale(self) -> float:
        return float(np.float32(1.0) / np.sqrt(np.float32(self.head_dim)))

    def lengths(self, seed: int = SEED) -> np.ndarray:
        return np.random.Generator(np.random.PCG64(seed + 4)).integers(self.lo, self.hi + 1, self.n_seqs)


@dataclasses.dataclass(frozen=True)
class Vision:
    name: str
    batch: int
    n: int
    n_heads: int
    head_dim: int
    sigma: float

    @property
    def scale(self) -> float:
        return float(np.float32(1.0) / np.sqrt(np.float32(self.head_dim)))

    def flops(self) -> int:
        return 4 * self.n_heads * self.head_dim * self.n * self.n * self.batch

    def bytes(self) -> int:
        rows = self.batch * self.n * self.n_heads * self.head_dim
        return 3 * rows * 2 + rows * 4


# BASELINE.json configs[0..4]
C1_PREFILL = Prefill("tiny-prefill", n_heads=8, n_kv=8, head_dim=32, n=32, theta=10000.0)
C1_DECODE_STEPS = 32
C2 = Decode("llama3-8b-decode-kv4096", n_heads=32, n_kv=8, head_dim=128, ctx=4096, theta=500000.0)
C3 = Prefill("llama3-8b-prefill-2048", n_heads=32, n_kv=8, head_dim=128, n=2048, theta=500000.0)
C4 = Ragged("ragged-decode-16", n_seqs=16, n_heads=32, n_kv=8, head_dim=128, lo=512, hi=32768, theta=500000.0)
C5 = Vision("clip-vit-l14", batch=32, n=257, n_heads=16, head_dim=64, sigma=0.5)


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def normal(g: np.random.Generator, shape, sigma: float = 1.0) -> np.ndarray:
    return (g.standard_normal(shape) * sigma).astype(np.float32)


def rope_rows(x: np.ndarray, head_dim: int, pos0: int, theta: float) -> np.ndarray:
    """Rows of heads rotated by positions pos0, pos0+1, ... (normal mode)."""
    n, size = x.shape
    i = np.arange(head_dim // 2, dtype=np.float64)
    ang = (pos0 + np.arange(n, dtype=np.float64))[:, None] * theta ** (-2.0 * i / head_dim)[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    h = x.reshape(n, size // head_dim, head_dim // 2, 2).astype(np.float64)
    x0, x1 = h[..., 0], h[..., 1]
    out = np.stack([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)
    return out.reshape(n, size).astype(np.float32)


def to_f16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> IEEE binary16 bit patterns (round to nearest even)."""
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def decode_inputs(cfg: Decode, seed: int = SEED, ctx: int | None = None):
    """Cached K (RoPE'd at 0..ctx-1, binary16) and V (binary16) rows, and the
    step's q (RoPE'd at ctx), k (RoPE'd at ctx), v rows, all f32."""
    ctx = cfg.ctx if ctx is None else ctx
    g = rng(seed)
    row = cfg.n_kv * cfg.head_dim
    k_cached = to_f16_bits(rope_rows(normal(g, (ctx, row)), cfg.head_dim, 0, cfg.theta))
    v_cached = to_f16_bits(normal(g, (ctx, row)))
    q = rope_rows(normal(g, (1, cfg.n_heads * cfg.head_dim)), cfg.head_dim, ctx, cfg.theta)
    k = rope_rows(normal(g, (1, row)), cfg.head_dim, ctx, cfg.theta)
    v = normal(g, (1, row))
    return k_cached, v_cached, q, k, v


def prefill_inputs(cfg: Prefill, seed: int = SEED, f16_exact: bool = True):
    """q, k, v rows [n][...] f32, RoPE'd at positions 0..n-1; with f16_exact
    every value is rounded to binary16 first (config 3's f16 inputs)."""
    g = rng(seed + 1)
    q = rope_rows(normal(g, (cfg.n, cfg.n_heads * cfg.head_dim)), cfg.head_dim, 0, cfg.theta)
    k = rope_rows(normal(g, (cfg.n, cfg.n_kv * cfg.head_dim)), cfg.head_dim, 0, cfg.theta)
    v = normal(g, (cfg.n, cfg.n_kv * cfg.head_dim))
    if f16_exact:
        q, k, v = (a.astype(np.float16).astype(np.float32) for a in (q, k, v))
    return q, k, v


def vision_inputs(cfg: Vision, seed: int = SEED, batch: int | None = None):
    """q, k, v [batch*n][n_heads*hd] as binary16 values (returned as f32)."""
    b = cfg.batch if batch is None else batch
    g = rng(seed + 5)
    shape = (b * cfg.n, cfg.n_heads * cfg.head_dim)
    return tuple(normal(g, shape, cfg.sigma).astype(np.float16).astype(np.float32) for _ in range(3))
