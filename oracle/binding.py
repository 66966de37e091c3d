"""numpy binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the checker for the HIP path. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module.

KV caches here are in the reference layout: k_cache, v_cache are uint16
[max_ctx][n_kv*hd] binary16 bit patterns, V untransposed.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_HALF_PATH = HERE / "_ref" / "libref_half.so"

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_sz, _u32, _f32 = ctypes.c_size_t, ctypes.c_uint32, ctypes.c_float

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: run `make -C oracle`")
        L = ctypes.CDLL(str(LIB_PATH))
        L.orc_fp16_to_float_n.argtypes = [_u16p, _f32p, _sz]
        L.orc_float_to_fp16_n.argtypes = [_f32p, _u16p, _sz]
        L.orc_rope_theta_scale.argtypes = [_f32, _sz]
        L.orc_rope_theta_scale.restype = _f32
        L.orc_rope_yarn_corr_dims.argtypes = [_sz, _sz, _f32, _f32, _f32, _f32p]
        L.orc_rope.argtypes = [_f32p, _f32p, _sz, _sz, _u32, _f32, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        L.orc_softmax.argtypes = [_f32p, _f32p, _sz]
        L.orc_attention_group_floats.argtypes = [_sz, _sz, _sz, _sz]
        L.orc_attention_group_floats.restype = _sz
        L.orc_attention_scratch_floats.argtypes = [_sz, _sz, _sz, _sz]
        L.orc_attention_scratch_floats.restype = _sz
        L.orc_kv_append.argtypes = [_f32p, _f32p, _u16p, _u16p, _sz, _sz, _sz, _u32]
        L.orc_attend_group.argtypes = [_f32p, _u16p, _u16p, _sz, _sz, _sz, _u32, _sz, _f32, _f32p, _f32p, _sz]
        L.orc_attention.argtypes = [_f32p, _f32p, _f32p, _u16p, _u16p, _sz, _sz, _sz, _u32, _sz, _f32, _f32p, _f32p]
        L.orc_attention_rows.argtypes = [_f32p, _f32p, _f32p, _sz, _u32, _u16p, _u16p, _sz, _sz, _sz, _sz, _f32,
                                         _f32p, _f32p, ctypes.c_uint]
        L.orc_attend_rows.argtypes = [_f32p, _sz, _u32, _u16p, _u16p, _sz, _sz, _sz, _sz, _f32, _f32p, _f32p,
                                      ctypes.c_uint]
        L.orc_self_attention.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, _sz, _f32, _f32p, ctypes.c_uint]
        for fn in (L.orc_fp16_to_float_n, L.orc_float_to_fp16_n, L.orc_rope, L.orc_softmax, L.orc_kv_append,
                   L.orc_attend_group, L.orc_attention, L.orc_attention_rows, L.orc_attend_rows,
                   L.orc_self_attention, L.orc_rope_yarn_corr_dims):
            fn.restype = None
        _lib = L
    return _lib


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def fp16_to_float(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().orc_fp16_to_float_n(h.reshape(-1), out.reshape(-1), h.size)
    return out


def float_to_fp16(x: np.ndarray) -> np.ndarray:
    x = _f(x)
    out = np.empty(x.shape, np.uint16)
    lib().orc_float_to_fp16_n(x.reshape(-1), out.reshape(-1), x.size)
    return out


def round16(x: np.ndarray) -> np.ndarray:
    return fp16_to_float(float_to_fp16(x))


def rope_theta_scale(base: float, head_dim: int) -> float:
    return float(lib().orc_rope_theta_scale(base, head_dim))


def rope_yarn_corr_dims(n_dims, n_ctx_orig, base, beta_fast, beta_slow) -> tuple[float, float]:
    out = np.zeros(2, np.float32)
    lib().orc_rope_yarn_corr_dims(n_dims, n_ctx_orig, base, beta_fast, beta_slow, out)
    return float(out[0]), float(out[1])


def rope(x: np.ndarray, head_dim: int, pos: int, theta_scale: float, freq_factors=None, mode: int = 0,
         scaling=None) -> np.ndarray:
    """One row of heads rotated by position pos (S/kernels/attention.hpp:89-129)."""
    x = _f(x)
    out = np.empty_like(x)
    ff = _f(freq_factors) if freq_factors is not None else None
    sc = _f(scaling) if scaling is not None else None
    lib().orc_rope(x, out, x.size, head_dim, pos, theta_scale, ff.ctypes.data if ff is not None else None, mode,
                   sc.ctypes.data if sc is not None else None)
    return out


def rope_rows(x: np.ndarray, head_dim: int, pos: int, theta_scale: float, **kw) -> np.ndarray:
    """Row i of x rotated by position pos + i (op_rope, S/graph/session.hpp:337-342)."""
    return np.stack([rope(x[i], head_dim, pos + i, theta_scale, **kw) for i in range(x.shape[0])])


def softmax(x: np.ndarray) -> np.ndarray:
    x = _f(x)
    out = np.empty_like(x)
    lib().orc_softmax(x, out, x.size)
    return out


def scratch_floats(n_heads, n_kv, hd, max_ctx) -> int:
    return int(lib().orc_attention_scratch_floats(n_heads, n_kv, hd, max_ctx))


def new_cache(max_ctx: int, n_kv: int, hd: int) -> tuple[np.ndarray, np.ndarray]:
    return np.zeros((max_ctx, n_kv * hd), np.uint16), np.zeros((max_ctx, n_kv * hd), np.uint16)


def attention_rows(q, k, v, pos, k_cache, v_cache, n_heads, scale, threads=1) -> np.ndarray:
    """session::execute(op_attention): append n rows, then causal attention.
    Mutates k_cache, v_cache (uint16 [max_ctx][n_kv*hd])."""
    q, k, v = _f(q), _f(k), _f(v)
    n = q.shape[0]
    max_ctx, row = k_cache.shape
    hd = q.shape[1] // n_heads
    n_kv = row // hd
    out = np.zeros_like(q)
    scores = np.zeros(scratch_floats(n_heads, n_kv, hd, max_ctx), np.float32)
    lib().orc_attention_rows(q, k, v, n, pos, k_cache, v_cache, max_ctx, n_kv, hd, n_heads, scale, out, scores,
                             threads)
    return out


def attend_rows(q, pos, k_cache, v_cache, n_heads, scale, threads=1, scores=None) -> np.ndarray:
    """The attend half: rows 0..pos+n-1 already in the cache."""
    q = _f(q)
    n = q.shape[0]
    max_ctx, row = k_cache.shape
    hd = q.shape[1] // n_heads
    n_kv = row // hd
    out = np.zeros_like(q)
    if scores is None:
        scores = np.zeros(scratch_floats(n_heads, n_kv, hd, max_ctx), np.float32)
    lib().orc_attend_rows(q, n, pos, k_cache, v_cache, max_ctx, n_kv, hd, n_heads, scale, out, scores, threads)
    return out


def self_attention(q, k, v, n_heads, scale, threads=1) -> np.ndarray:
    """op_self_attention over one image's rows [n][n_heads*hd]."""
    q, k, v = _f(q), _f(k), _f(v)
    out = np.zeros_like(q)
    lib().orc_self_attention(q, k, v, q.shape[0], q.shape[1], n_heads, scale, out, threads)
    return out


def ref_half():
    """The reference's own binary16 conversions (oracle/_ref), or None where
    the reference tree was absent at build time."""
    if not REF_HALF_PATH.exists():
        return None
    L = ctypes.CDLL(str(REF_HALF_PATH))
    L.ref_fp16_to_float_n.argtypes = [_u16p, _f32p, _sz]
    L.ref_float_to_fp16_n.argtypes = [_f32p, _u16p, _sz]
    L.ref_fp16_to_float_n.restype = None
    L.ref_float_to_fp16_n.restype = None
    return L
