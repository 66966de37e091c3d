"""A read-only GGUF (v2/v3) parser over numpy: metadata and tensors, nothing
executed from the file.

The layout is GGUF's published one, which the reference's reader parses too
(S/gguf/reader.hpp): magic "GGUF", version, tensor count, metadata count;
typed key/value pairs; tensor infos (name, dims with ne[0] fastest, type,
offset); then the tensor data at `general.alignment` (default 32).

Only the tensor types this build consumes are decoded (F32, F16); other
types are listed but refused when read.
"""
from __future__ import annotations

import pathlib
import struct
from dataclasses import dataclass

import numpy as np

GGUF_MAGIC = b"GGUF"

# Metadata value types.
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_SCALAR = {_U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f", _BOOL: "<?",
           _U64: "<Q", _I64: "<q", _F64: "<d"}

# Tensor types (ggml_type) this build reads.
F32, F16 = 0, 1
Q4_0, Q5_0, Q8_0, Q4_K, Q6_K, Q8_K, BF16 = 2, 6, 8, 12, 14, 15, 30
_DTYPE = {F32: np.float32, F16: np.float16}

# ggml_type -> (elements per block, bytes per block): the published block
# layouts (ggml-common.h). Types not listed are refused.
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34),
         Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292)}
TYPE_NAMES = {F32: "F32", F16: "F16", BF16: "BF16", Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q4_K: "Q4_K",
              Q6_K: "Q6_K", Q8_K: "Q8_K"}


class GGUFError(ValueError):
    pass


@dataclass(frozen=True)
class TensorInfo:
    name: str
    shape: tuple[int, ...]  # ne[0] first (fastest-varying), as GGUF stores it
    type: int
    offset: int             # from the start of the data section

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n


class GGUFFile:
    """Parsed GGUF file: `metadata` (dict), `tensors` (name -> TensorInfo)."""

    def __init__(self, path: str | pathlib.Path):
        self.path = pathlib.Path(path)
        self._buf = self.path.read_bytes()
        self._pos = 0
        if self._take(4) != GGUF_MAGIC:
            raise GGUFError(f"{self.path}: not a GGUF file")
        self.version = self._scalar(_U32)
        if self.version not in (2, 3):
            raise GGUFError(f"{self.path}: GGUF version {self.version}")
        n_tensors = self._scalar(_U64)
        n_kv = self._scalar(_U64)
        self.metadata: dict[str, object] = {}
        for _ in range(n_kv):
            key = self._string()
            self.metadata[key] = self._value(self._scalar(_U32))
        self.tensors: dict[str, TensorInfo] = {}
        for _ in range(n_tensors):
            name = self._string()
            n_dims = self._scalar(_U32)
            shape = tuple(self._scalar(_U64) for _ in range(n_dims))
            ttype = self._scalar(_U32)
            offset = self._scalar(_U64)
            self.tensors[name] = TensorInfo(name, shape, ttype, offset)
        align = int(self.metadata.get("general.alignment", 32))
        if align <= 0 or align & (align - 1):
            raise GGUFError(f"{self.path}: alignment {align}")
        self.data_start = (self._pos + align - 1) // align * align

    # ---- metadata -----------------------------------------------------------
    def _take(self, n: int) -> bytes:
        if self._pos + n > len(self._buf):
            raise GGUFError(f"{self.path}: truncated at byte {self._pos}")
        b = self._buf[self._pos:self._pos + n]
        self._pos += n
        return b

    def _scalar(self, t: int):
        fmt = _SCALAR[t]
        return struct.unpack(fmt, self._take(struct.calcsize(fmt)))[0]

    def _string(self) -> str:
        n = self._scalar(_U64)
        return self._take(n).decode("utf-8")

    def _value(self, t: int):
        if t in _SCALAR:
            return self._scalar(t)
        if t == _STR:
            return self._string()
        if t == _ARR:
            et = self._scalar(_U32)
            n = self._scalar(_U64)
            return [self._value(et) for _ in range(n)]
        raise GGUFError(f"{self.path}: metadata type {t}")

    def get(self, key: str, default=None):
        return self.metadata.get(key, default)

    def require(self, key: str):
        if key not in self.metadata:
            raise GGUFError(f"{self.path}: missing metadata {key}")
        return self.metadata[key]

    # ---- tensors --------------------------------------------------------------
    def has(self, name: str) -> bool:
        return name in self.tensors

    def raw(self, name: str) -> tuple[np.ndarray, int, int, int]:
        """The tensor's bytes as stored: (uint8 array, ggml type, row length
        ne[0], number of rows). Rows are ne[0] / block elements blocks each."""
        info = self.tensors.get(name)
        if info is None:
            raise GGUFError(f"{self.path}: no tensor {name}")
        if info.type not in BLOCK:
            raise GGUFError(f"{self.path}: tensor {name} has unsupported type {info.type}")
        bs, ts = BLOCK[info.type]
        row = info.shape[0]
        if row % bs:
            raise GGUFError(f"{self.path}: tensor {name}: row of {row} is not whole blocks of {bs}")
        n_rows = info.n_elements // row
        nbytes = n_rows * (row // bs) * ts
        start = self.data_start + info.offset
        if start + nbytes > len(self._buf):
            raise GGUFError(f"{self.path}: tensor {name} past the end of the file")
        return np.frombuffer(self._buf, dtype=np.uint8, count=nbytes, offset=start), info.type, row, n_rows

    def tensor(self, name: str) -> np.ndarray:
        """The tensor as an array of shape reversed(ne): rows last-dimension
        fastest, so a [rows][cols] matrix comes back as (rows, cols)."""
        info = self.tensors.get(name)
        if info is None:
            raise GGUFError(f"{self.path}: no tensor {name}")
        dtype = _DTYPE.get(info.type)
        if dtype is None:
            raise GGUFError(f"{self.path}: tensor {name} has type {info.type}, not F32/F16")
        start = self.data_start + info.offset
        nbytes = info.n_elements * np.dtype(dtype).itemsize
        if start + nbytes > len(self._buf):
            raise GGUFError(f"{self.path}: tensor {name} past the end of the file")
        a = np.frombuffer(self._buf, dtype=dtype, count=info.n_elements, offset=start)
        return a.reshape(tuple(reversed(info.shape)))
