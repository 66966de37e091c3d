"""CPU restatement of the reference's image encoder (S/models/clip.hpp:300-417,
executed as S/graph/session.hpp does), to pin this build's reading of the
graph against llama.cpp's golden embeddings before the GPU runs it: numpy
float32 with the reference's accumulation where it is specified (layer
norm's double sums, S/kernels/elementwise.hpp:240-305; GELU through
binary16, :115-167) and the oracle's f32 self-attention. Test infrastructure
only."""
from __future__ import annotations

import math

import numpy as np

import binding as orc
from synapse_amd.clip import read_config, unfold_patches
from synapse_amd.gguf import GGUFFile

f32 = np.float32


def layer_norm(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray, eps: float) -> np.ndarray:
    out = np.empty_like(x)
    for r in range(x.shape[0]):
        row = x[r]
        s = 0.0
        for v in row.astype(np.float64):
            s += v
        mean = f32(s) / f32(row.size)
        d = (row - mean).astype(f32)
        q = 0.0
        for v in (d * d).astype(np.float64):
            q += v
        var = f32(q / row.size)
        scale = f32(1) / f32(math.sqrt(float(var + f32(eps))))
        out[r] = (d * scale) * gamma + beta
    return out.astype(f32)


def gelu(x: np.ndarray) -> np.ndarray:
    h = x.astype(np.float16).astype(f32)
    g = (f32(0.5) * h * (f32(1) + np.tanh(f32(0.79788456080286535587989211986876) * h *
                                         (f32(1) + f32(0.044715) * h * h)))).astype(f32)
    t = g.astype(np.float16).astype(f32)
    return np.where(x <= -10, f32(0), np.where(x >= 10, x, t)).astype(f32)


def pixel_shuffle(x: np.ndarray, grid: int, s: int) -> np.ndarray:
    n = x.shape[1]
    bw = grid // s
    out = np.empty((grid * grid // (s * s), s * s * n), f32)
    for by in range(grid // s):
        for bx in range(bw):
            for dy in range(s):
                for dx in range(s):
                    out[bx + bw * by, (dy * s + dx) * n:(dy * s + dx + 1) * n] = x[(bx * s + dx) + grid * (by * s + dy)]
    return out


def encode(f: GGUFFile, image: np.ndarray) -> np.ndarray:
    c = read_config(f)
    W = {name: np.asarray(f.tensor(name), dtype=f32) for name in f.tensors}
    E = c.n_embd

    def lin(w, x, b=None):
        y = (x @ w.reshape(w.shape[0], -1).T).astype(f32)
        return (y + b).astype(f32) if b is not None else y

    patches = unfold_patches(c, image)
    x = (lin(W["v.patch_embd.weight"].reshape(E, -1), patches, W["v.patch_embd.bias"]) +
         W["v.position_embd.weight"]).astype(f32)
    scale = float(f32(1) / np.sqrt(f32(E // c.n_head)))
    for l in range(c.n_layer):
        b = f"v.blk.{l}."
        swapped = W[b + "ffn_down.weight"].shape[1] == E and W[b + "ffn_down.weight"].shape[0] != E
        up, down = ("ffn_down", "ffn_up") if swapped else ("ffn_up", "ffn_down")
        h = layer_norm(x, W[b + "ln1.weight"], W[b + "ln1.bias"], c.eps)
        q = lin(W[b + "attn_q.weight"], h, W[b + "attn_q.bias"])
        k = lin(W[b + "attn_k.weight"], h, W[b + "attn_k.bias"])
        v = lin(W[b + "attn_v.weight"], h, W[b + "attn_v.bias"])
        attn = orc.self_attention(q, k, v, c.n_head, scale)
        x = (lin(W[b + "attn_out.weight"], attn, W[b + "attn_out.bias"]) + x).astype(f32)
        h = layer_norm(x, W[b + "ln2.weight"], W[b + "ln2.bias"], c.eps)
        act = gelu(lin(W[b + up + ".weight"], h, W[b + up + ".bias"]))
        x = (x + lin(W[b + down + ".weight"], act, W[b + down + ".bias"])).astype(f32)
    if "v.post_ln.weight" in W:
        x = layer_norm(x, W["v.post_ln.weight"], W["v.post_ln.bias"], c.eps)
    return lin(W["mm.model.fc.weight"], pixel_shuffle(x, c.grid, c.scale_factor))


def compare(ours: np.ndarray, ref: np.ndarray) -> list[float]:
    """Per output token: rms(ours - ref) / rms(ref), the reference test's
    measure (tests/sdk/clip_golden.cpp:22-35)."""
    res = []
    for o, r in zip(ours.astype(np.float64), ref.astype(np.float64)):
        res.append(float(np.sqrt(np.mean((o - r) ** 2)) / np.sqrt(np.mean(r ** 2))))
    return res
