"""Minimal GGUF (v2/v3) writer used to build synthetic and hand-made models.

The byte format is the one the reference parser reads (src/gguf/file.rs:57-116,
src/gguf/value.rs:45-71, src/gguf/tensor.rs:52-75): magic ``GGUF``, u32 version,
u64 tensor count, u64 metadata count, typed metadata, tensor infos, then the
data region starting at the next multiple of 32 bytes.  Large payloads are
filled in place through a ``numpy.memmap`` so multi-GB models never sit in
Python memory.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Sequence

import numpy as np

# metadata value type ids (src/gguf/types.rs:7-21)
VT_U8, VT_I8, VT_U16, VT_I16, VT_U32, VT_I32, VT_F32, VT_BOOL, VT_STR, VT_ARR, VT_U64, VT_I64, VT_F64 = range(13)

# ggml tensor type ids (src/gguf/types.rs:70-100)
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K = 0, 1, 2, 7, 12, 14, 15
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K", Q8_K: "Q8_K"}

# element size or (block elements, block bytes) (src/gguf/types.rs:181-229)
_ELEM = {0: 4, 1: 2, 16: 1, 17: 2, 18: 4, 19: 8, 20: 8}
_BLOCK = {2: (32, 18), 3: (32, 20), 5: (32, 22), 6: (32, 24), 7: (32, 34), 8: (32, 36), 29: (32, 18),
          10: (256, 96), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
          15: (256, 292), 21: (256, 166), 22: (256, 184), 23: (256, 66), 24: (256, 104),
          25: (256, 176), 26: (256, 98), 27: (256, 166), 28: (256, 136), 30: (256, 116)}

_SCALAR_FMT = {VT_U8: "<B", VT_I8: "<b", VT_U16: "<H", VT_I16: "<h", VT_U32: "<I", VT_I32: "<i",
               VT_F32: "<f", VT_BOOL: "<B", VT_U64: "<Q", VT_I64: "<q", VT_F64: "<d"}


def byte_size(ggml_type: int, n_elements: int) -> int:
    """TensorInfo::byte_size (src/gguf/tensor.rs:30-40)."""
    if ggml_type in _ELEM:
        return n_elements * _ELEM[ggml_type]
    be, bb = _BLOCK[ggml_type]
    return -(-n_elements // be) * bb


def _gguf_string(s) -> bytes:
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _encode_value(vtype: int, value) -> bytes:
    if vtype == VT_STR:
        return _gguf_string(value)
    if vtype == VT_ARR:
        item_type, items = value
        out = struct.pack("<IQ", item_type, len(items))
        return out + b"".join(_encode_value(item_type, it) for it in items)
    return struct.pack(_SCALAR_FMT[vtype], value)


@dataclass
class _Tensor:
    name: str
    shape: List[int]
    ggml_type: int
    nbytes: int
    data: Optional[bytes] = None
    fill: Optional[Callable[[np.ndarray], None]] = None
    offset: int = 0


@dataclass
class GGUFWriter:
    version: int = 3
    alignment: int = 32
    meta: List[bytes] = field(default_factory=list)
    tensors: List[_Tensor] = field(default_factory=list)

    # ---- metadata ----
    def add(self, key: str, vtype: int, value) -> "GGUFWriter":
        self.meta.append(_gguf_string(key) + struct.pack("<I", vtype) + _encode_value(vtype, value))
        return self

    def add_raw(self, raw: bytes) -> "GGUFWriter":
        """Append pre-encoded metadata bytes (for malformed-file tests)."""
        self.meta.append(raw)
        return self

    def add_string(self, k, v): return self.add(k, VT_STR, v)
    def add_u32(self, k, v): return self.add(k, VT_U32, v)
    def add_u64(self, k, v): return self.add(k, VT_U64, v)
    def add_f32(self, k, v): return self.add(k, VT_F32, v)

    # ---- tensors ----
    def add_tensor(self, name: str, shape: Sequence[int], ggml_type: int, data: Optional[bytes] = None,
                   fill: Optional[Callable[[np.ndarray], None]] = None, nbytes: Optional[int] = None):
        n = int(np.prod(shape)) if len(shape) else 1
        size = byte_size(ggml_type, n) if nbytes is None else nbytes
        if data is not None and len(data) != size:
            raise ValueError(f"{name}: {len(data)} bytes given, {size} expected")
        self.tensors.append(_Tensor(name, list(shape), ggml_type, size, data, fill))
        return self

    def tensor_f32(self, name: str, shape: Sequence[int], values) -> "GGUFWriter":
        arr = np.ascontiguousarray(np.asarray(values, dtype="<f4"))
        return self.add_tensor(name, shape, F32, data=arr.tobytes())

    # ---- output ----
    def header_bytes(self) -> bytes:
        off = 0
        infos = []
        for t in self.tensors:
            off = -(-off // self.alignment) * self.alignment
            t.offset = off
            infos.append(_gguf_string(t.name) + struct.pack("<I", len(t.shape)) +
                         b"".join(struct.pack("<Q", d) for d in t.shape) +
                         struct.pack("<IQ", t.ggml_type, off))
            off += t.nbytes
        head = b"GGUF" + struct.pack("<IQQ", self.version, len(self.tensors), len(self.meta))
        head += b"".join(self.meta) + b"".join(infos)
        pad = (-len(head)) % 32
        self._data_len = off
        return head + b"\0" * pad

    def write(self, path: str) -> int:
        """Write the file; returns its size in bytes."""
        head = self.header_bytes()
        total = len(head) + self._data_len
        with open(path, "wb") as f:
            f.write(head)
            f.truncate(total)
        if self._data_len:
            mm = np.memmap(path, dtype=np.uint8, mode="r+", offset=len(head), shape=(self._data_len,))
            for t in self.tensors:
                view = mm[t.offset:t.offset + t.nbytes]
                if t.data is not None:
                    view[:] = np.frombuffer(t.data, dtype=np.uint8)
                elif t.fill is not None:
                    t.fill(view)
            mm.flush()
            del mm
        return total
