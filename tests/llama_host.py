"""CPU restatement of the reference's Llama-family decode graph
(S/models/llama.hpp:405-473, executed as S/graph/session.hpp:287-378 does),
used to pin this build's reading of the graph against llama.cpp's golden
logits before the GPU runs it. Matrix products, norms and element-wise ops
are numpy float32 with the reference's accumulation where it is specified
(RMSNorm's squares summed in double, S/kernels/elementwise.hpp:208-235);
RoPE and the f16-cache attention are the oracle's (oracle/oracle.cpp).
Test infrastructure only."""
from __future__ import annotations

import numpy as np

import binding as orc
import quant_host as qh
from synapse_amd.gguf import GGUFFile
from synapse_amd.llama import attn_temperature, read_config, rope_theta_scale

f32 = np.float32


def rms_norm(x: np.ndarray, gamma: np.ndarray, eps: float) -> np.ndarray:
    sq = (x * x).astype(np.float64)  # float squares, double sum
    s = 0.0
    for v in sq:
        s += v
    mean = f32(s / x.size)
    scale = f32(1) / np.sqrt(mean + f32(eps))
    return ((x * scale) * gamma).astype(f32)


def silu(x: np.ndarray) -> np.ndarray:
    return (x / (f32(1) + np.exp(-x))).astype(f32)


class QuantMatrix:
    """A weight matrix kept in its GGUF format: rows of blocks."""

    def __init__(self, f: GGUFFile, name: str):
        self.raw, self.type, self.cols, self.rows = f.raw(name)
        self.row_bytes = self.raw.size // self.rows

    def row(self, r: int) -> np.ndarray:
        return self.raw[r * self.row_bytes:(r + 1) * self.row_bytes]

    def matvec(self, x: np.ndarray) -> np.ndarray:
        """ggml's quantized product: x quantized to the paired activation
        format, then one integer dot per row."""
        act = qh.quantize_act(x, self.type)
        return np.array([qh.vec_dot(self.row(r), self.type, act) for r in range(self.rows)], f32)

    def dequantize_row(self, r: int) -> np.ndarray:
        return qh.dequantize(self.row(r), self.type)


def _weights(f: GGUFFile) -> dict:
    W = {}
    for name, info in f.tensors.items():
        if info.type == 0:
            W[name] = np.asarray(f.tensor(name), dtype=f32)
        else:
            W[name] = QuantMatrix(f, name)
    return W


def decode_logits(f: GGUFFile, tokens, max_ctx: int = 32) -> np.ndarray:
    """Logits after each token, decoded one at a time from position 0."""
    c = read_config(f)
    hd = c.head_dim
    W = _weights(f)
    ff = W.get("rope_freqs.weight")
    s = c.rope_scaling
    scaling = np.array([s.freq_scale, s.ext_factor, s.attn_factor, s.corr_low, s.corr_high], f32)
    ts = rope_theta_scale(c.rope_base, hd)
    scale = float(f32(1) / np.sqrt(f32(hd)))
    caches = [orc.new_cache(max_ctx, c.n_head_kv, hd) for _ in range(c.n_layer)]

    def lin(name, x, bias=None):
        w = W[name]
        y = w.matvec(x) if isinstance(w, QuantMatrix) else (w @ x).astype(f32)
        return (y + W[bias]).astype(f32) if bias in W else y

    out = []
    for pos, tok in enumerate(tokens):
        embd = W["token_embd.weight"]
        x = embd.dequantize_row(tok) if isinstance(embd, QuantMatrix) else embd[tok].copy()
        for l in range(c.n_layer):
            b = f"blk.{l}."
            h = rms_norm(x, W[b + "attn_norm.weight"], c.rms_eps)
            q = lin(b + "attn_q.weight", h, b + "attn_q.bias")
            k = lin(b + "attn_k.weight", h, b + "attn_k.bias")
            v = lin(b + "attn_v.weight", h, b + "attn_v.bias")
            q = orc.rope(q, hd, pos, ts, freq_factors=ff, mode=c.rope_mode, scaling=scaling)
            k = orc.rope(k, hd, pos, ts, freq_factors=ff, mode=c.rope_mode, scaling=scaling)
            if c.attn_temp_scale != 0.0:
                q = (q * f32(attn_temperature(pos, c.attn_temp_scale, c.n_ctx_orig))).astype(f32)
            kc, vc = caches[l]
            attn = orc.attention_rows(q[None], k[None], v[None], pos, kc, vc, c.n_head, scale)[0]
            x = (lin(b + "attn_output.weight", attn, b + "attn_output.bias") + x).astype(f32)
            h = rms_norm(x, W[b + "ffn_norm.weight"], c.rms_eps)
            act = (silu(lin(b + "ffn_gate.weight", h, b + "ffn_gate.bias")) *
                   lin(b + "ffn_up.weight", h, b + "ffn_up.bias")).astype(f32)
            x = (lin(b + "ffn_down.weight", act, b + "ffn_down.bias") + x).astype(f32)
        h = rms_norm(x, W["output_norm.weight"], c.rms_eps)
        wout = "output.weight" if "output.weight" in W else "token_embd.weight"
        out.append(lin(wout, h, "output.bias"))
    return np.stack(out)


def compare(ours: np.ndarray, ref: np.ndarray) -> list[tuple[float, bool]]:
    """Per position: (max |ours - ref| / max |ref|, same argmax), the
    reference test's measures (tests/support/llama_golden.hpp)."""
    res = []
    for o, r in zip(ours, ref):
        err = float(np.max(np.abs(o.astype(np.float64) - r)) / np.max(np.abs(r)))
        res.append((err, int(np.argmax(o)) == int(np.argmax(r))))
    return res
