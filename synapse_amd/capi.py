"""ctypes binding of the C ABI in include/synapse_hip.h.

The library must have been built (python -m synapse_amd.build); loading fails
loudly otherwise -- there is no fallback path. Every call returning a status
raises SynHipError on a non-zero status, with the library's detail message.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
LIB_PATH = ROOT / "libsynapse_hip.so"

SYN_F32 = 0
SYN_F16 = 1
NO_OFFSET = (1 << 64) - 1

u64, u32, f32, i32 = ctypes.c_uint64, ctypes.c_uint32, ctypes.c_float, ctypes.c_int


class KvDesc(ctypes.Structure):
    _fields_ = [("k_offset", u64), ("v_offset", u64), ("max_ctx", u32), ("n_kv_heads", u32),
                ("head_dim", u32), ("ctx_stride", u32)]


class AttnDesc(ctypes.Structure):
    _fields_ = [("cache", KvDesc), ("q_offset", u64), ("k_offset", u64), ("v_offset", u64),
                ("out_offset", u64), ("scratch_offset", u64), ("scratch_bytes", u64), ("n_heads", u32),
                ("pos", u32), ("n", u32), ("scale", f32), ("q_dtype", u32), ("kv_dtype", u32)]


class SeqDesc(ctypes.Structure):
    _fields_ = [("cache", KvDesc), ("q_offset", u64), ("out_offset", u64), ("pos", u32), ("reserved", u32)]


class SelfDesc(ctypes.Structure):
    _fields_ = [("q_offset", u64), ("k_offset", u64), ("v_offset", u64), ("out_offset", u64), ("n", u32),
                ("batch", u32), ("n_heads", u32), ("head_dim", u32), ("scale", f32), ("in_dtype", u32)]


class RopeDesc(ctypes.Structure):
    _fields_ = [("in_offset", u64), ("out_offset", u64), ("freq_factors_offset", u64), ("n", u32), ("size", u32),
                ("head_dim", u32), ("pos", u32), ("theta_scale", f32), ("mode", u32), ("freq_scale", f32),
                ("ext_factor", f32), ("attn_factor", f32), ("corr_low", f32), ("corr_high", f32), ("period", u32)]


class AttnRopeDesc(ctypes.Structure):
    _fields_ = [("q_out_offset", u64), ("k_out_offset", u64), ("freq_factors_offset", u64), ("theta_scale", f32),
                ("mode", u32), ("freq_scale", f32), ("ext_factor", f32), ("attn_factor", f32), ("corr_low", f32),
                ("corr_high", f32), ("temp_scale", f32), ("temp_floor_len", u32)]


class TemperatureDesc(ctypes.Structure):
    _fields_ = [("in_offset", u64), ("out_offset", u64), ("n", u32), ("size", u32), ("pos", u32),
                ("floor_len", u32), ("scale", f32), ("reserved", u32)]


class EmbedDesc(ctypes.Structure):
    _fields_ = [("table_offset", u64), ("out_offset", u64), ("n_table_rows", u32), ("size", u32),
                ("table_type", u32), ("reserved", u32)]


class MatmulQDesc(ctypes.Structure):
    _fields_ = [("w_offset", u64), ("x_offset", u64), ("act_offset", u64), ("bias_offset", u64),
                ("out_offset", u64), ("w_type", u32), ("n", u32), ("rows", u32), ("cols", u32)]


class NormDesc(ctypes.Structure):
    _fields_ = [("in_offset", u64), ("weight_offset", u64), ("out_offset", u64), ("n", u32), ("size", u32),
                ("eps", f32), ("reserved", u32)]


class MatmulDesc(ctypes.Structure):
    _fields_ = [("w_offset", u64), ("x_offset", u64), ("bias_offset", u64), ("out_offset", u64), ("n", u32),
                ("rows", u32), ("cols", u32), ("reserved", u32)]


class ElementwiseDesc(ctypes.Structure):
    _fields_ = [("a_offset", u64), ("b_offset", u64), ("out_offset", u64), ("count", u64), ("op", u32),
                ("scalar", f32), ("period", u32), ("reserved", u32)]


class LayerNormDesc(ctypes.Structure):
    _fields_ = [("in_offset", u64), ("weight_offset", u64), ("bias_offset", u64), ("out_offset", u64), ("n", u32),
                ("size", u32), ("eps", f32), ("reserved", u32)]


class PixelShuffleDesc(ctypes.Structure):
    _fields_ = [("in_offset", u64), ("out_offset", u64), ("n", u32), ("grid_w", u32), ("grid_h", u32),
                ("scale", u32)]


class SoftmaxDesc(ctypes.Structure):
    _fields_ = [("in_offset", u64), ("out_offset", u64), ("n", u32), ("size", u32)]


SYN_ADD, SYN_MUL, SYN_SILU_MUL, SYN_SCALE, SYN_GELU, SYN_SILU, SYN_ADD_BIAS = 0, 1, 2, 3, 4, 5, 6


# name -> (restype, argtypes); every symbol include/synapse_hip.h declares.
SIGNATURES = {
    "syn_hip_error_string": (ctypes.c_char_p, [i32]),
    "syn_hip_last_error": (ctypes.c_char_p, []),
    "syn_hip_arena_create": (i32, [ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)]),
    "syn_hip_arena_destroy": (i32, [ctypes.c_void_p]),
    "syn_hip_arena_bytes": (ctypes.c_size_t, [ctypes.c_void_p]),
    "syn_hip_arena_stream": (ctypes.c_void_p, [ctypes.c_void_p]),
    "syn_hip_upload": (i32, [ctypes.c_void_p, u64, ctypes.c_void_p, ctypes.c_size_t]),
    "syn_hip_download": (i32, [ctypes.c_void_p, u64, ctypes.c_void_p, ctypes.c_size_t]),
    "syn_hip_fill": (i32, [ctypes.c_void_p, u64, i32, ctypes.c_size_t]),
    "syn_hip_copy": (i32, [ctypes.c_void_p, u64, u64, ctypes.c_size_t]),
    "syn_hip_synchronize": (i32, [ctypes.c_void_p]),
    "syn_hip_kv_ctx_stride": (u32, [u32]),
    "syn_hip_kv_state_bytes": (u64, [u32, u32, u32]),
    "syn_hip_attention_scratch_bytes": (u64, [u32, u32, u32, u32, u32]),
    "syn_hip_attention": (i32, [ctypes.c_void_p, ctypes.POINTER(AttnDesc)]),
    "syn_hip_attend": (i32, [ctypes.c_void_p, ctypes.POINTER(AttnDesc)]),
    "syn_hip_attention_noalloc": (i32, [ctypes.c_void_p, ctypes.POINTER(AttnDesc)]),
    "syn_hip_attention_noalloc_scratch_limit": (u64, []),
    "syn_hip_kv_append": (i32, [ctypes.c_void_p, ctypes.POINTER(KvDesc), u64, u64, u32, u32, u32]),
    "syn_hip_attend_batch_scratch_bytes": (u64, [ctypes.POINTER(SeqDesc), u32, u32]),
    "syn_hip_attend_batch": (i32, [ctypes.c_void_p, ctypes.POINTER(SeqDesc), u32, u32, f32, u32, u64, u64]),
    "syn_hip_self_attention": (i32, [ctypes.c_void_p, ctypes.POINTER(SelfDesc)]),
    "syn_hip_rope": (i32, [ctypes.c_void_p, ctypes.POINTER(RopeDesc)]),
    "syn_hip_attn_temperature": (i32, [ctypes.c_void_p, ctypes.POINTER(TemperatureDesc)]),
    "syn_hip_attention_rope": (i32, [ctypes.c_void_p, ctypes.POINTER(AttnDesc), ctypes.POINTER(AttnRopeDesc)]),
    "syn_hip_embed": (i32, [ctypes.c_void_p, ctypes.POINTER(EmbedDesc), ctypes.POINTER(u32), u32]),
    "syn_hip_rms_norm": (i32, [ctypes.c_void_p, ctypes.POINTER(NormDesc)]),
    "syn_hip_matmul": (i32, [ctypes.c_void_p, ctypes.POINTER(MatmulDesc)]),
    "syn_hip_elementwise": (i32, [ctypes.c_void_p, ctypes.POINTER(ElementwiseDesc)]),
    "syn_hip_matmul_q_act_bytes": (u64, [u32, u32, u32]),
    "syn_hip_matmul_q": (i32, [ctypes.c_void_p, ctypes.POINTER(MatmulQDesc)]),
    "syn_hip_softmax": (i32, [ctypes.c_void_p, ctypes.POINTER(SoftmaxDesc)]),
    "syn_hip_layer_norm": (i32, [ctypes.c_void_p, ctypes.POINTER(LayerNormDesc)]),
    "syn_hip_pixel_shuffle": (i32, [ctypes.c_void_p, ctypes.POINTER(PixelShuffleDesc)]),
}

_lib = None


class SynHipError(RuntimeError):
    def __init__(self, code: int, detail: str):
        super().__init__(f"synapse_hip error {code}: {detail}")
        self.code = code
        self.detail = detail


def lib() -> ctypes.CDLL:
    """The loaded library. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m synapse_amd.build`")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != 0:
        detail = lib().syn_hip_last_error().decode()
        raise SynHipError(status, detail or lib().syn_hip_error_string(status).decode())


class HipGraph:
    """A HIP graph captured from the C ABI calls `record()` makes on an
    arena's stream, replayed with `launch()`: for launch-bound loops (one
    decode step per layer, say), whose kernels the graph replays with one
    host call. Calls that allocate, synchronise or copy to the host cannot
    be captured; the attention, RoPE and model-op entry points only launch
    kernels on the arena's stream."""

    _CAPTURE_RELAXED = 2  # hipStreamCaptureModeRelaxed

    def __init__(self, arena: "Arena", record):
        rt = _hip_runtime()
        self._rt = rt
        self.stream = ctypes.c_void_p(arena.stream)
        graph = ctypes.c_void_p()
        self._exec = ctypes.c_void_p()
        _hip_ok(rt.hipStreamBeginCapture(self.stream, self._CAPTURE_RELAXED), "hipStreamBeginCapture")
        try:
            record()
        finally:
            _hip_ok(rt.hipStreamEndCapture(self.stream, ctypes.byref(graph)), "hipStreamEndCapture")
        try:
            count = ctypes.c_size_t(0)
            _hip_ok(rt.hipGraphGetNodes(graph, None, ctypes.byref(count)), "hipGraphGetNodes")
            self.nodes = count.value  # the captured launches (and any other recorded operations)
            _hip_ok(rt.hipGraphInstantiate(ctypes.byref(self._exec), graph, None, None, 0), "hipGraphInstantiate")
        finally:
            rt.hipGraphDestroy(graph)

    def launch(self) -> None:
        _hip_ok(self._rt.hipGraphLaunch(self._exec, self.stream), "hipGraphLaunch")

    def upload(self) -> None:
        """Moves the executable graph's launch resources to the device ahead
        of its first launch, so a timed first launch does not pay for that."""
        _hip_ok(self._rt.hipGraphUpload(self._exec, self.stream), "hipGraphUpload")

    def close(self) -> None:
        """Destroys the executable graph; the caller has synchronised every
        launch of it. Before the arena is closed, on every path: a graph
        left alive is otherwise torn down with the runtime at process exit."""
        if self._exec:
            self._rt.hipGraphExecDestroy(self._exec)
            self._exec = ctypes.c_void_p()

    def __enter__(self) -> "HipGraph":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        self.close()


_rt = None


def _hip_runtime() -> ctypes.CDLL:
    global _rt
    if _rt is None:
        rt = ctypes.CDLL("libamdhip64.so")
        vp = ctypes.c_void_p
        for name, args in {"hipStreamBeginCapture": [vp, ctypes.c_int],
                           "hipStreamEndCapture": [vp, ctypes.POINTER(vp)],
                           "hipGraphInstantiate": [ctypes.POINTER(vp), vp, vp, vp, ctypes.c_size_t],
                           "hipGraphLaunch": [vp, vp], "hipGraphUpload": [vp, vp], "hipGraphDestroy": [vp],
                           "hipGraphGetNodes": [vp, ctypes.POINTER(vp), ctypes.POINTER(ctypes.c_size_t)],
                           "hipGraphExecDestroy": [vp]}.items():
            getattr(rt, name).argtypes = args
            getattr(rt, name).restype = ctypes.c_int
        _rt = rt
    return _rt


def _hip_ok(status: int, what: str) -> None:
    if status != 0:
        raise SynHipError(status, f"{what} failed with HIP error {status}")


def align(x: int, a: int = 256) -> int:
    return (x + a - 1) // a * a


class Arena:
    """One device arena (one hipMalloc) with a bump allocator for offsets."""

    def __init__(self, nbytes: int):
        self.handle = ctypes.c_void_p()
        check(lib().syn_hip_arena_create(nbytes, ctypes.byref(self.handle)))
        self.nbytes = nbytes
        self.top = 0

    def alloc(self, nbytes: int, alignment: int = 256) -> int:
        off = align(self.top, alignment)
        if off + nbytes > self.nbytes:
            raise MemoryError(f"arena of {self.nbytes} bytes cannot hold {nbytes} more at {off}")
        self.top = off + nbytes
        return off

    def put(self, array: np.ndarray, alignment: int = 256) -> int:
        a = np.ascontiguousarray(array)
        off = self.alloc(a.nbytes, alignment)
        self.upload(off, a)
        return off

    def upload(self, offset: int, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array)
        check(lib().syn_hip_upload(self.handle, offset, a.ctypes.data, a.nbytes))

    def download(self, offset: int, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        check(lib().syn_hip_download(self.handle, offset, out.ctypes.data, out.nbytes))
        return out

    def fill(self, offset: int, value: int, nbytes: int) -> None:
        check(lib().syn_hip_fill(self.handle, offset, value, nbytes))

    def sync(self) -> None:
        check(lib().syn_hip_synchronize(self.handle))

    @property
    def stream(self) -> int:
        return lib().syn_hip_arena_stream(self.handle)

    def close(self) -> None:
        if self.handle:
            check(lib().syn_hip_arena_destroy(self.handle))
            self.handle = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def kv_state(arena: Arena, max_ctx: int, n_kv: int, hd: int) -> KvDesc:
    """Places one KV state in the arena (K block, then V^T block)."""
    stride = lib().syn_hip_kv_ctx_stride(max_ctx)
    k_bytes = align(max_ctx * n_kv * hd * 2)
    base = arena.alloc(lib().syn_hip_kv_state_bytes(max_ctx, n_kv, hd))
    return KvDesc(k_offset=base, v_offset=base + k_bytes, max_ctx=max_ctx, n_kv_heads=n_kv, head_dim=hd,
                  ctx_stride=stride)


def kv_state_bytes(max_ctx: int, n_kv: int, hd: int) -> int:
    return int(lib().syn_hip_kv_state_bytes(max_ctx, n_kv, hd))


def upload_cache(arena: Arena, c: KvDesc, k_rows16: np.ndarray, v_rows16: np.ndarray) -> None:
    """Writes binary16 K, V rows [L][n_kv*hd] (uint16 bit patterns) straight
    into a state's K and V^T blocks (positions 0..L-1)."""
    L = k_rows16.shape[0]
    row = c.n_kv_heads * c.head_dim
    assert k_rows16.shape == (L, row) and v_rows16.shape == (L, row) and L <= c.max_ctx
    arena.upload(c.k_offset, k_rows16.astype(np.uint16))
    vt = np.zeros((row, c.ctx_stride), dtype=np.uint16)
    vt[:, :L] = v_rows16.T
    arena.upload(c.v_offset, vt)


def download_cache(arena: Arena, c: KvDesc, L: int) -> tuple[np.ndarray, np.ndarray]:
    """Rows 0..L-1 of a state's K and V, as [L][n_kv*hd] uint16 (V untransposed)."""
    row = c.n_kv_heads * c.head_dim
    k = arena.download(c.k_offset, (c.max_ctx, row), np.uint16)[:L]
    vt = arena.download(c.v_offset, (row, c.ctx_stride), np.uint16)
    return k, np.ascontiguousarray(vt[:, :L].T)
