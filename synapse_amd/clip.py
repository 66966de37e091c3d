"""The reference's image encoder (a llama.cpp "idefics3" mmproj: SigLIP ViT,
pixel shuffle, linear projector) run entirely on one GPU through the C ABI.

The graph is the reference's (S/models/clip.hpp:8-16, built at :300-380):

    x = Wpatch patches + bpatch + pos_embd          (one row per patch)
    per layer:
        h = LN1(x);  x = x + Wo self_attention(Wq h + bq, Wk h + bk, Wv h + bv) + bo
        h = LN2(x);  x = x + Wdown gelu(Wup h + bup) + bdown
    embeddings = Wfc pixel_shuffle(LN_post(x), s)    (one row per s x s patches)

The image arrives normalized (what clip.cpp holds after preprocessing) and
is unfolded into patch rows on the host, as the reference's encode() does
(S/models/clip.hpp:383-417). Weights must be F32.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import capi
from .capi import (NO_OFFSET, SYN_ADD, SYN_F32, SYN_GELU, Arena, ElementwiseDesc, LayerNormDesc, MatmulDesc,
                   PixelShuffleDesc, SelfDesc, check, lib)
from .gguf import F32, GGUFError, GGUFFile

_f32 = np.float32


@dataclass
class ClipConfig:
    image_size: int
    patch_size: int
    n_embd: int
    n_ff: int
    n_layer: int
    n_head: int
    eps: float
    scale_factor: int
    n_embd_text: int

    @property
    def grid(self) -> int:
        return self.image_size // self.patch_size

    @property
    def n_patches(self) -> int:
        return self.grid * self.grid

    @property
    def n_tokens(self) -> int:
        return self.n_patches // (self.scale_factor * self.scale_factor)

    @property
    def patch_floats(self) -> int:
        return 3 * self.patch_size * self.patch_size


def read_config(f: GGUFFile) -> ClipConfig:
    """The keys and checks of the reference's clip config reader
    (S/models/clip.hpp:180-240) that this encoder needs."""
    if f.get("clip.projector_type") != "idefics3":
        raise GGUFError(f"clip.projector_type {f.get('clip.projector_type')!r}: only idefics3")
    if not f.get("clip.use_gelu", False):
        raise GGUFError("clip.use_gelu: only GELU")

    def count(k):
        v = f.require(k)
        if int(v) <= 0:
            raise GGUFError(f"{k}: {v}")
        return int(v)

    c = ClipConfig(image_size=count("clip.vision.image_size"), patch_size=count("clip.vision.patch_size"),
                   n_embd=count("clip.vision.embedding_length"), n_ff=count("clip.vision.feed_forward_length"),
                   n_layer=count("clip.vision.block_count"), n_head=count("clip.vision.attention.head_count"),
                   eps=float(_f32(f.require("clip.vision.attention.layer_norm_epsilon"))),
                   scale_factor=count("clip.vision.projector.scale_factor"),
                   n_embd_text=count("clip.vision.projection_dim"))
    if c.image_size % c.patch_size or c.n_embd % c.n_head:
        raise GGUFError("clip.vision: image/patch or width/heads do not divide")
    if c.scale_factor < 2 or c.grid % c.scale_factor:
        raise GGUFError("clip.vision.projector.scale_factor")
    return c


def unfold_patches(c: ClipConfig, image: np.ndarray) -> np.ndarray:
    """Image [y][x][channel] (image_size^2 * 3 floats) to one row per patch in
    the (channel, y, x) order of the patch kernel (S/models/clip.hpp:383-400)."""
    p, g = c.patch_size, c.grid
    img = np.asarray(image, np.float32).reshape(g, p, g, p, 3)          # py, y, px, x, ch
    return np.ascontiguousarray(img.transpose(0, 2, 4, 1, 3).reshape(c.n_patches, c.patch_floats))


def _weight(f: GGUFFile, name: str, shape) -> np.ndarray:
    info = f.tensors.get(name)
    if info is None:
        raise GGUFError(f"missing tensor {name}")
    if info.type != F32:
        raise GGUFError(f"{name}: type {info.type}; this encoder takes F32 weights")
    return np.ascontiguousarray(np.asarray(f.tensor(name), np.float32).reshape(shape))


class DeviceClip:
    """The encoder on the GPU, one arena per model; encode(image) returns the
    n_tokens x n_embd_text embeddings."""

    def __init__(self, f: GGUFFile):
        c = self.config = read_config(f)
        E, F, P = c.n_embd, c.n_ff, c.n_patches
        w = {}
        w["patch.w"] = _weight(f, "v.patch_embd.weight", (E, c.patch_floats))
        w["patch.b"] = _weight(f, "v.patch_embd.bias", (E,))
        w["pos"] = _weight(f, "v.position_embd.weight", (P, E))
        for l in range(c.n_layer):
            b = f"v.blk.{l}."
            for extra in ("attn_qkv.weight", "attn_q_norm.weight", "attn_k_norm.weight", "ls1.weight", "ls2.weight",
                          "ffn_gate.weight"):
                if b + extra in f.tensors:
                    raise GGUFError(f"{b + extra}: not supported")
            # The up projection reads n_embd-wide rows; files may store the
            # pair swapped (S/models/clip.hpp:318-323).
            swapped = f.tensors[b + "ffn_down.weight"].shape[0] == E
            up, down = ("ffn_down", "ffn_up") if swapped else ("ffn_up", "ffn_down")
            for s, shape in (("ln1.weight", (E,)), ("ln1.bias", (E,)), ("attn_q.weight", (E, E)),
                             ("attn_q.bias", (E,)), ("attn_k.weight", (E, E)), ("attn_k.bias", (E,)),
                             ("attn_v.weight", (E, E)), ("attn_v.bias", (E,)), ("attn_out.weight", (E, E)),
                             ("attn_out.bias", (E,)), ("ln2.weight", (E,)), ("ln2.bias", (E,))):
                w[b + s] = _weight(f, b + s, shape)
            w[b + "up.w"] = _weight(f, b + up + ".weight", (F, E))
            w[b + "up.b"] = _weight(f, b + up + ".bias", (F,))
            w[b + "down.w"] = _weight(f, b + down + ".weight", (E, F))
            w[b + "down.b"] = _weight(f, b + down + ".bias", (E,))
        self.post_ln = "v.post_ln.weight" in f.tensors
        if self.post_ln:
            w["post.w"] = _weight(f, "v.post_ln.weight", (E,))
            w["post.b"] = _weight(f, "v.post_ln.bias", (E,))
        merged = E * c.scale_factor * c.scale_factor
        w["fc"] = _weight(f, "mm.model.fc.weight", (c.n_embd_text, merged))

        act = {"patches": P * c.patch_floats, "x": P * E, "h": P * E, "q": P * E, "k": P * E, "v": P * E,
               "attn": P * E, "o": P * E, "up": P * F, "shuf": P * E, "emb": c.n_tokens * c.n_embd_text}
        total = sum(capi.align(a.nbytes) for a in w.values()) + sum(capi.align(n * 4) for n in act.values())
        self.arena = Arena(total + 4096)
        self.off = {k: self.arena.put(a) for k, a in w.items()}
        self.act = {k: self.arena.alloc(n * 4) for k, n in act.items()}
        self.scale = float(_f32(1) / np.sqrt(_f32(E // c.n_head)))

    def close(self) -> None:
        self.arena.close()

    def _matmul(self, w, x, out, n, rows, cols, bias=None):
        d = MatmulDesc(w_offset=self.off[w], x_offset=self.act[x],
                       bias_offset=self.off[bias] if bias else NO_OFFSET, out_offset=self.act[out], n=n, rows=rows,
                       cols=cols)
        check(lib().syn_hip_matmul(self.arena.handle, ctypes.byref(d)))

    def _ln(self, x, w, b, out):
        c = self.config
        d = LayerNormDesc(in_offset=self.act[x], weight_offset=self.off[w], bias_offset=self.off[b],
                          out_offset=self.act[out], n=c.n_patches, size=c.n_embd, eps=c.eps)
        check(lib().syn_hip_layer_norm(self.arena.handle, ctypes.byref(d)))

    def _ew(self, op, a, b, out, count, a_is_weight=False, b_is_weight=False):
        d = ElementwiseDesc(a_offset=self.off[a] if a_is_weight else self.act[a],
                            b_offset=(self.off[b] if b_is_weight else self.act[b]) if b else 0,
                            out_offset=self.act[out], count=count, op=op, scalar=0.0)
        check(lib().syn_hip_elementwise(self.arena.handle, ctypes.byref(d)))

    def encode(self, image: np.ndarray) -> np.ndarray:
        c = self.config
        E, F, P = c.n_embd, c.n_ff, c.n_patches
        self.arena.upload(self.act["patches"], unfold_patches(c, image))
        self._matmul("patch.w", "patches", "x", P, E, c.patch_floats, "patch.b")
        self._ew(SYN_ADD, "x", "pos", "x", P * E, b_is_weight=True)  # add_rows over the whole table
        for l in range(c.n_layer):
            b = f"v.blk.{l}."
            self._ln("x", b + "ln1.weight", b + "ln1.bias", "h")
            self._matmul(b + "attn_q.weight", "h", "q", P, E, E, b + "attn_q.bias")
            self._matmul(b + "attn_k.weight", "h", "k", P, E, E, b + "attn_k.bias")
            self._matmul(b + "attn_v.weight", "h", "v", P, E, E, b + "attn_v.bias")
            sd = SelfDesc(q_offset=self.act["q"], k_offset=self.act["k"], v_offset=self.act["v"],
                          out_offset=self.act["attn"], n=P, batch=1, n_heads=c.n_head, head_dim=E // c.n_head,
                          scale=self.scale, in_dtype=SYN_F32)
            check(lib().syn_hip_self_attention(self.arena.handle, ctypes.byref(sd)))
            self._matmul(b + "attn_out.weight", "attn", "o", P, E, E, b + "attn_out.bias")
            self._ew(SYN_ADD, "o", "x", "x", P * E)
            self._ln("x", b + "ln2.weight", b + "ln2.bias", "h")
            self._matmul(b + "up.w", "h", "up", P, F, E, b + "up.b")
            self._ew(SYN_GELU, "up", None, "up", P * F)
            self._matmul(b + "down.w", "up", "o", P, E, F, b + "down.b")
            self._ew(SYN_ADD, "x", "o", "x", P * E)
        if self.post_ln:
            self._ln("x", "post.w", "post.b", "h")
        src = "h" if self.post_ln else "x"
        d = PixelShuffleDesc(in_offset=self.act[src], out_offset=self.act["shuf"], n=E, grid_w=c.grid, grid_h=c.grid,
                             scale=c.scale_factor)
        check(lib().syn_hip_pixel_shuffle(self.arena.handle, ctypes.byref(d)))
        merged = E * c.scale_factor * c.scale_factor
        self._matmul("fc", "shuf", "emb", c.n_tokens, c.n_embd_text, merged)
        return self.arena.download(self.act["emb"], (c.n_tokens, c.n_embd_text), np.float32)
