"""Helpers that drive the HIP path through the C ABI (ctypes) for the GPU
parity tests. Every kernel call here goes through include/synapse_hip.h."""
from __future__ import annotations

import ctypes

import numpy as np

from synapse_amd import capi
from synapse_amd.capi import SYN_F16, SYN_F32, Arena, AttnDesc, SelfDesc, SeqDesc, check, lib


def f16(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16)


def put_rows(arena: Arena, x: np.ndarray, dtype: int) -> int:
    return arena.put(f16(x) if dtype == SYN_F16 else np.ascontiguousarray(x, dtype=np.float32))


def scratch_for(arena: Arena, n_heads: int, n_kv: int, hd: int, max_ctx: int) -> tuple[int, int]:
    nbytes = int(lib().syn_hip_attention_scratch_bytes(n_heads, n_kv, hd, max_ctx, 1))
    return (arena.alloc(max(nbytes, 256)), nbytes)


def attn_desc(cache, q_off, k_off, v_off, out_off, scratch, n_heads, pos, n, scale, q_dtype=SYN_F32,
              kv_dtype=SYN_F32) -> AttnDesc:
    return AttnDesc(cache=cache, q_offset=q_off, k_offset=k_off, v_offset=v_off, out_offset=out_off,
                    scratch_offset=scratch[0], scratch_bytes=scratch[1], n_heads=n_heads, pos=pos, n=n,
                    scale=scale, q_dtype=q_dtype, kv_dtype=kv_dtype)


def attention(arena: Arena, cache, scratch, q, k, v, pos, n_heads, scale, q_dtype=SYN_F32, kv_dtype=SYN_F32,
              append=True) -> np.ndarray:
    """syn_hip_attention (append + attend) or, with append=False, syn_hip_attend,
    for n rows at positions pos..pos+n-1. Returns the f32 output rows."""
    n = q.shape[0]
    mark = arena.top
    q_off = put_rows(arena, q, q_dtype)
    k_off = put_rows(arena, k, kv_dtype) if append else 0
    v_off = put_rows(arena, v, kv_dtype) if append else 0
    out_off = arena.alloc(q.shape[0] * q.shape[1] * 4)
    d = attn_desc(cache, q_off, k_off, v_off, out_off, scratch, n_heads, pos, n, scale, q_dtype, kv_dtype)
    fn = lib().syn_hip_attention if append else lib().syn_hip_attend
    check(fn(arena.handle, ctypes.byref(d)))
    out = arena.download(out_off, q.shape, np.float32)
    arena.top = mark  # the run's rows are free again
    return out


def self_attention(arena: Arena, q, k, v, n, batch, n_heads, scale, in_dtype=SYN_F16) -> np.ndarray:
    mark = arena.top
    offs = [put_rows(arena, x, in_dtype) for x in (q, k, v)]
    out_off = arena.alloc(q.shape[0] * q.shape[1] * 4)
    d = SelfDesc(q_offset=offs[0], k_offset=offs[1], v_offset=offs[2], out_offset=out_off, n=n, batch=batch,
                 n_heads=n_heads, head_dim=q.shape[1] // n_heads, scale=scale, in_dtype=in_dtype)
    check(lib().syn_hip_self_attention(arena.handle, ctypes.byref(d)))
    out = arena.download(out_off, q.shape, np.float32)
    arena.top = mark
    return out


def seq_array(seqs: list[SeqDesc]):
    arr = (SeqDesc * len(seqs))(*seqs)
    return arr


__all__ = ["f16", "put_rows", "scratch_for", "attn_desc", "attention", "self_attention", "seq_array", "capi",
           "SYN_F16", "SYN_F32", "Arena", "SeqDesc", "check", "lib"]
