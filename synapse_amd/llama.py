"""A Llama-family decode graph (Llama, Qwen2, Mistral 3) run entirely on one
GPU through the C ABI: embedding, RMSNorm, F32 matrix products, RoPE, the
f16-cache attention, residual adds and the SiLU-gated FFN.

The graph is the reference's (S/models/llama.hpp:8-14, built at :405-473):

    x = embed(token_embd)
    per layer:
        h = rms_norm(x, attn_norm)
        q = rope(Wq h + bq) * temp(pos), k = rope(Wk h + bk), v = Wv h + bv
        x = x + Wo attention(q, k, v, kv_cache) + bo
        h = rms_norm(x, ffn_norm)
        x = x + Wdown (silu(Wgate h + bgate) * (Wup h + bup)) + bdown
    logits = Wout rms_norm(last_row(x), output_norm) + bout   (Wout = token_embd if tied)

`read_config` follows the reference's read_llama_config
(S/models/llama.hpp:125-319) for the keys the three architectures use, in
float arithmetic as the reference computes them. Norms, biases and RoPE
factors must be F32; the matrices (token embedding, projections, output)
may be F32 or one of the block formats Q4_0, Q5_0, Q8_0, Q4_K, Q6_K, which
stay in their GGUF bytes on the device and run through the quantized GEMV
(activation quantized to Q8_0 / Q8_K, integer block dots).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field

import numpy as np

from . import capi
from .capi import (NO_OFFSET, SYN_ADD, SYN_F32, SYN_SILU_MUL, Arena, AttnDesc, AttnRopeDesc, ElementwiseDesc, EmbedDesc,
                   MatmulDesc, MatmulQDesc, NormDesc, check, lib)
from .gguf import F32, Q4_0, Q4_K, Q5_0, Q6_K, Q8_0, TYPE_NAMES, GGUFError, GGUFFile

_f32 = np.float32

# Biases an architecture may carry, as the reference's loader accepts them
# (S/models/llama.hpp:376-389).
_BIASES = {
    "llama": (),
    "qwen2": ("attn_q.bias", "attn_k.bias", "attn_v.bias", "output.bias"),
    "mistral3": ("attn_q.bias", "attn_k.bias", "attn_v.bias", "attn_output.bias", "ffn_gate.bias", "ffn_up.bias",
                 "ffn_down.bias"),
}


@dataclass
class RopeScaling:
    """kernels::rope_scaling (S/kernels/attention.hpp:57-66); default = none."""
    freq_scale: float = 1.0
    ext_factor: float = 0.0
    attn_factor: float = 1.0
    corr_low: float = 0.0
    corr_high: float = 0.0


@dataclass
class LlamaConfig:
    arch: str
    rope_mode: int          # 0 normal, 1 neox
    n_layer: int
    n_embd: int
    n_ff: int
    n_head: int
    n_head_kv: int
    head_dim: int
    n_vocab: int
    n_ctx_train: int
    rms_eps: float
    rope_base: float
    n_ctx_orig: int
    rope_scaling: RopeScaling = field(default_factory=RopeScaling)
    attn_temp_scale: float = 0.0


def rope_theta_scale(base: float, head_dim: int) -> float:
    """base^(-2/head_dim) in float (S/kernels/attention.hpp:47-49)."""
    return float(_f32(base) ** (_f32(-2.0) / _f32(head_dim)))


def rope_yarn_corr_dims(n_dims: int, n_ctx_orig: int, base: float, beta_fast: float,
                        beta_slow: float) -> tuple[float, float]:
    """The YaRN ramp's pair range, in float (S/kernels/attention.hpp:71-81)."""
    pi = _f32(3.14159265358979323846)

    def corr_dim(n_rot):
        return _f32(n_dims) * np.log(_f32(n_ctx_orig) / (_f32(n_rot) * _f32(2) * pi)) / (_f32(2) * np.log(_f32(base)))

    start = np.floor(corr_dim(beta_fast))
    end = np.ceil(corr_dim(beta_slow))
    return float(max(_f32(0), start)), float(min(_f32(n_dims) - _f32(1), end))


def _yarn_mscale(factor, mscale):
    factor, mscale = _f32(factor), _f32(mscale)
    return _f32(1) if factor <= 1 else _f32(0.1) * mscale * np.log(factor) + _f32(1)


def attn_temperature(pos: int, scale: float, floor_len: int) -> float:
    """1 + scale * ln(floor(pos / floor_len) + 1): a float quotient, the log
    in double, rounded to float (S/kernels/elementwise.hpp:66-71)."""
    q = math.floor(float(_f32(pos) / _f32(floor_len)))
    return float(_f32(math.log(q + 1.0) * float(_f32(scale)) + 1.0))


def read_config(f: GGUFFile) -> LlamaConfig:
    arch = f.require("general.architecture")
    if arch not in _BIASES:
        raise GGUFError(f"general.architecture {arch!r}: not a Llama-family model")

    def key(k):
        return f"{arch}.{k}"

    def count(k, default=None):
        v = f.get(key(k), default)
        if v is None:
            raise GGUFError(f"missing {key(k)}")
        return int(v)

    n_head = count("attention.head_count")
    n_embd = count("embedding_length")
    head_dim = count("attention.key_length", n_embd // n_head)
    if count("rope.dimension_count", head_dim) != head_dim:
        raise GGUFError(f"{key('rope.dimension_count')}: partial rotary dimensions are not supported")
    n_ctx_train = count("context_length")
    c = LlamaConfig(
        arch=arch, rope_mode=1 if arch == "qwen2" else 0, n_layer=count("block_count"), n_embd=n_embd,
        n_ff=count("feed_forward_length"), n_head=n_head, n_head_kv=count("attention.head_count_kv", n_head),
        head_dim=head_dim, n_vocab=0, n_ctx_train=n_ctx_train,
        rms_eps=float(_f32(f.require(key("attention.layer_norm_rms_epsilon")))),
        rope_base=float(_f32(f.get(key("rope.freq_base"), 10000.0))),
        n_ctx_orig=count("rope.scaling.original_context_length", n_ctx_train))
    if c.n_head % c.n_head_kv:
        raise GGUFError(f"{key('attention.head_count_kv')}: {c.n_head_kv} does not divide {c.n_head}")
    # RoPE scaling (S/models/llama.hpp:125-183): none, or YaRN.
    stype = f.get(key("rope.scaling.type"), "linear")
    factor = _f32(f.get(key("rope.scaling.factor"), 0.0))
    freq_scale = _f32(1) if factor == 0 else _f32(1) / factor
    attn = _f32(f.get(key("rope.scaling.attn_factor"), 1.0))
    if stype == "none" or (stype == "linear" and freq_scale == 1):
        c.rope_scaling = RopeScaling(attn_factor=float(attn))
    elif stype == "yarn":
        mistral3 = arch == "mistral3"
        beta_fast = _f32(f.get(key("rope.scaling.yarn_beta_fast"), 32.0) if mistral3 else 32.0)
        beta_slow = _f32(f.get(key("rope.scaling.yarn_beta_slow"), 1.0) if mistral3 else 1.0)
        log_mul = _f32(f.get(key("rope.scaling.yarn_log_multiplier"), 0.0) if mistral3 else 0.0)
        yarn_factor = _f32(1) / freq_scale
        a = (_yarn_mscale(yarn_factor, 1.0) / _yarn_mscale(yarn_factor, log_mul) if log_mul != 0
             else _yarn_mscale(yarn_factor, 1.0))
        a = a * (_f32(1) / (_f32(1) + _f32(0.1) * np.log(yarn_factor)))
        a = a * attn
        low, high = rope_yarn_corr_dims(c.head_dim, c.n_ctx_orig, c.rope_base, float(beta_fast), float(beta_slow))
        c.rope_scaling = RopeScaling(float(freq_scale), 1.0, float(a), low, high)
    else:
        raise GGUFError(f"{key('rope.scaling.type')} {stype!r} is not supported")
    if arch == "mistral3":
        c.attn_temp_scale = float(_f32(f.get(key("attention.temperature_scale"), 0.0)))
    embd = f.tensors.get("token_embd.weight")
    if embd is None or embd.shape[0] != n_embd:
        raise GGUFError("token_embd.weight")
    c.n_vocab = int(embd.shape[1])
    return c


# Block formats the device GEMV and embedding read.
QUANT_TYPES = (Q4_0, Q5_0, Q8_0, Q4_K, Q6_K)


def _matrix(f: GGUFFile, name: str, rows: int, cols: int):
    """A weight matrix as (ggml type, array to upload): F32 values, or the
    rows of blocks exactly as the file stores them."""
    info = f.tensors.get(name)
    if info is None:
        raise GGUFError(f"missing tensor {name}")
    if info.type == F32:
        return F32, _f32_weight(f, name, (rows, cols))
    if info.type not in QUANT_TYPES:
        raise GGUFError(f"{name}: type {TYPE_NAMES.get(info.type, info.type)} is not supported")
    raw, t, row, n_rows = f.raw(name)
    if (n_rows, row) != (rows, cols):
        raise GGUFError(f"{name}: shape {(n_rows, row)}, expected {(rows, cols)}")
    return t, raw


def _f32_weight(f: GGUFFile, name: str, shape) -> np.ndarray:
    info = f.tensors.get(name)
    if info is None:
        raise GGUFError(f"missing tensor {name}")
    if info.type != F32:
        raise GGUFError(f"{name}: type {info.type}; this runner takes F32 weights")
    a = f.tensor(name)
    if a.shape != tuple(shape):
        raise GGUFError(f"{name}: shape {a.shape}, expected {tuple(shape)}")
    return np.ascontiguousarray(a, dtype=np.float32)


class DeviceLlama:
    """The decode graph on the GPU: one arena holding the weights, the
    activations, the RoPE factors, one KV state per layer and the attention
    scratch. step(token, pos) runs one token and returns its logits."""

    def __init__(self, f: GGUFFile, max_ctx: int):
        c = self.config = read_config(f)
        self.max_ctx = max_ctx
        hd, E, F, V = c.head_dim, c.n_embd, c.n_ff, c.n_vocab
        q_rows, kv_rows = c.n_head * hd, c.n_head_kv * hd
        # Tensors that change the result and that this architecture does not
        # read are refused, not ignored (S/models/llama.hpp:436-452, :469-471).
        biases = set(_BIASES[c.arch])
        for name in f.tensors:
            suffix = name.split(".", 2)[2] if name.startswith("blk.") else name
            if suffix in ("attn_q.bias", "attn_k.bias", "attn_v.bias", "attn_output.bias", "ffn_gate.bias",
                          "ffn_up.bias", "ffn_down.bias", "ffn_gate_inp.weight", "output.bias") \
                    and suffix not in biases:
                raise GGUFError(f"{name}: not supported for {c.arch}")
        self._host = {}
        self.wtype = {}  # matrix name -> (ggml type, columns)

        def w(name, shape):
            if len(shape) == 2:
                t, self._host[name] = _matrix(f, name, *shape)
                self.wtype[name] = (t, shape[1])
            else:
                self._host[name] = _f32_weight(f, name, shape)

        w("token_embd.weight", (V, E))
        w("output_norm.weight", (E,))
        self.tied = "output.weight" not in f.tensors
        if not self.tied:
            w("output.weight", (V, E))
        if "output.bias" in f.tensors:
            w("output.bias", (V,))
        self.freq_factors = None
        if "rope_freqs.weight" in f.tensors:
            if c.arch == "qwen2":
                raise GGUFError("rope_freqs.weight: not read for qwen2")
            w("rope_freqs.weight", (hd // 2,))
            self.freq_factors = "rope_freqs.weight"
        shapes = {"attn_norm.weight": (E,), "attn_q.weight": (q_rows, E), "attn_k.weight": (kv_rows, E),
                  "attn_v.weight": (kv_rows, E), "attn_output.weight": (E, q_rows), "ffn_norm.weight": (E,),
                  "ffn_gate.weight": (F, E), "ffn_up.weight": (F, E), "ffn_down.weight": (E, F),
                  "attn_q.bias": (q_rows,), "attn_k.bias": (kv_rows,), "attn_v.bias": (kv_rows,),
                  "attn_output.bias": (E,), "ffn_gate.bias": (F,), "ffn_up.bias": (F,), "ffn_down.bias": (E,)}
        for l in range(c.n_layer):
            for suffix, shape in shapes.items():
                name = f"blk.{l}.{suffix}"
                if suffix.endswith(".bias") and name not in f.tensors:
                    continue
                w(name, shape)

        # ---- arena layout: weights, activations, KV states, scratch ----------
        act = {"x": E, "h": E, "q": q_rows, "qr": q_rows, "k": kv_rows, "kr": kv_rows, "v": kv_rows,
               "attn": q_rows, "o": E, "gate": F, "up": F, "down": E, "logits": V}
        scratch_bytes = int(lib().syn_hip_attention_scratch_bytes(c.n_head, c.n_head_kv, hd, max_ctx, 1))
        # One activation-quantization buffer serves every quantized matrix.
        qact_bytes = max([int(lib().syn_hip_matmul_q_act_bytes(t, 1, cols))
                          for t, cols in self.wtype.values() if t != F32] or [0])
        total = sum(capi.align(a.nbytes) for a in self._host.values())
        total += sum(capi.align(n * 4) for n in act.values()) + capi.align(max(qact_bytes, 1))
        total += c.n_layer * capi.align(capi.kv_state_bytes(max_ctx, c.n_head_kv, hd)) + capi.align(scratch_bytes)
        self.arena = Arena(total + 4096)
        self.off = {name: self.arena.put(a) for name, a in self._host.items()}
        self.act = {name: self.arena.alloc(n * 4) for name, n in act.items()}
        self.qact = self.arena.alloc(max(qact_bytes, 1))
        self.caches = [capi.kv_state(self.arena, max_ctx, c.n_head_kv, hd) for _ in range(c.n_layer)]
        self.scratch = (self.arena.alloc(scratch_bytes), scratch_bytes)
        self.theta_scale = rope_theta_scale(c.rope_base, hd)
        self.scale = float(_f32(1) / np.sqrt(_f32(hd)))
        self.reset()

    def close(self) -> None:
        self.arena.close()

    def reset(self) -> None:
        """Zeroes the KV states, as before a new sequence."""
        for cache in self.caches:
            self.arena.fill(cache.k_offset, 0, capi.kv_state_bytes(self.max_ctx, self.config.n_head_kv,
                                                                    self.config.head_dim))

    # ---- one op each, through the C ABI ---------------------------------------
    def _bias(self, name):
        return self.off.get(name, NO_OFFSET)

    def _matmul(self, w, x, out, rows, cols, bias=None):
        bias_offset = self._bias(bias) if bias else NO_OFFSET
        t = self.wtype[w][0]
        if t == F32:
            d = MatmulDesc(w_offset=self.off[w], x_offset=self.act[x], bias_offset=bias_offset,
                           out_offset=self.act[out], n=1, rows=rows, cols=cols)
            check(lib().syn_hip_matmul(self.arena.handle, ctypes.byref(d)))
        else:
            d = MatmulQDesc(w_offset=self.off[w], x_offset=self.act[x], act_offset=self.qact, bias_offset=bias_offset,
                            out_offset=self.act[out], w_type=t, n=1, rows=rows, cols=cols)
            check(lib().syn_hip_matmul_q(self.arena.handle, ctypes.byref(d)))

    def _norm(self, x, weight, out):
        d = NormDesc(in_offset=self.act[x], weight_offset=self.off[weight], out_offset=self.act[out], n=1,
                     size=self.config.n_embd, eps=self.config.rms_eps)
        check(lib().syn_hip_rms_norm(self.arena.handle, ctypes.byref(d)))

    def _elementwise(self, op, a, b, out, count, scalar=0.0):
        d = ElementwiseDesc(a_offset=self.act[a], b_offset=self.act[b] if b else 0, out_offset=self.act[out],
                            count=count, op=op, scalar=scalar)
        check(lib().syn_hip_elementwise(self.arena.handle, ctypes.byref(d)))

    def _attention(self, layer, pos):
        """op_rope on q and k, op_attn_temperature, op_attention: one
        syn_hip_attention_rope call, which a decode step runs as one kernel."""
        c, s = self.config, self.config.rope_scaling
        ad = AttnDesc(cache=self.caches[layer], q_offset=self.act["q"], k_offset=self.act["k"],
                      v_offset=self.act["v"], out_offset=self.act["attn"], scratch_offset=self.scratch[0],
                      scratch_bytes=self.scratch[1], n_heads=c.n_head, pos=pos, n=1, scale=self.scale,
                      q_dtype=SYN_F32, kv_dtype=SYN_F32)
        rd = AttnRopeDesc(q_out_offset=self.act["qr"], k_out_offset=self.act["kr"],
                          freq_factors_offset=self.off[self.freq_factors] if self.freq_factors else NO_OFFSET,
                          theta_scale=self.theta_scale, mode=c.rope_mode, freq_scale=s.freq_scale,
                          ext_factor=s.ext_factor, attn_factor=s.attn_factor, corr_low=s.corr_low,
                          corr_high=s.corr_high, temp_scale=c.attn_temp_scale,
                          temp_floor_len=c.n_ctx_orig if c.attn_temp_scale != 0.0 else 0)
        check(lib().syn_hip_attention_rope(self.arena.handle, ctypes.byref(ad), ctypes.byref(rd)))

    def step(self, token: int, pos: int) -> np.ndarray:
        c = self.config
        hd, E, F, V = c.head_dim, c.n_embd, c.n_ff, c.n_vocab
        q_rows, kv_rows = c.n_head * hd, c.n_head_kv * hd
        if not 0 <= pos < self.max_ctx:
            raise ValueError(f"position {pos} outside the {self.max_ctx}-row cache")
        tok = (ctypes.c_uint32 * 1)(token)
        d = EmbedDesc(table_offset=self.off["token_embd.weight"], out_offset=self.act["x"], n_table_rows=V, size=E,
                      table_type=self.wtype["token_embd.weight"][0])
        check(lib().syn_hip_embed(self.arena.handle, ctypes.byref(d), tok, 1))
        for l in range(c.n_layer):
            b = f"blk.{l}."
            self._norm("x", b + "attn_norm.weight", "h")
            self._matmul(b + "attn_q.weight", "h", "q", q_rows, E, b + "attn_q.bias")
            self._matmul(b + "attn_k.weight", "h", "k", kv_rows, E, b + "attn_k.bias")
            self._matmul(b + "attn_v.weight", "h", "v", kv_rows, E, b + "attn_v.bias")
            self._attention(l, pos)  # RoPE, then the temperature after it (llm_build_mistral3), then attention
            self._matmul(b + "attn_output.weight", "attn", "o", E, q_rows, b + "attn_output.bias")
            self._elementwise(SYN_ADD, "o", "x", "x", E)
            self._norm("x", b + "ffn_norm.weight", "h")
            self._matmul(b + "ffn_gate.weight", "h", "gate", F, E, b + "ffn_gate.bias")
            self._matmul(b + "ffn_up.weight", "h", "up", F, E, b + "ffn_up.bias")
            self._elementwise(SYN_SILU_MUL, "gate", "up", "gate", F)
            self._matmul(b + "ffn_down.weight", "gate", "down", E, F, b + "ffn_down.bias")
            self._elementwise(SYN_ADD, "down", "x", "x", E)
        self._norm("x", "output_norm.weight", "h")
        out_w = "token_embd.weight" if self.tied else "output.weight"
        self._matmul(out_w, "h", "logits", V, E, "output.bias" if "output.bias" in self.off else None)
        return self.arena.download(self.act["logits"], (V,), np.float32)
