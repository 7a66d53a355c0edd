"""The byte-level BPE tokenizer of the text path, over the C ABI.

Mirrors ``inferox::tokenizer`` (src/tokenizer/mod.rs): ``BpeTokenizer.from_file``
/ ``from_json`` load a Hugging Face tokenizer.json of model type "BPE";
``encode`` / ``decode`` follow ``Tokenizer::encode`` / ``decode``.  Errors come
back as :class:`TokenizerError` with the C ABI status (``IFX_E_IO``,
``IFX_E_JSON``, ``IFX_E_UNSUPPORTED_TOKENIZER``), the reference's
``TokenizerError::{Io, Json, UnsupportedModel}``.  Host code only: no device
is touched.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from inferox_amd import _native

IFX_E_IO, IFX_E_JSON, IFX_E_UNSUPPORTED_TOKENIZER = 1, 13, 14


class TokenizerError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def _raise(rc: int):
    if rc != 0:
        raise TokenizerError(rc, _native.lib().ifx_last_error().decode(errors="replace"))


class BpeTokenizer:
    def __init__(self, handle: C.c_void_p):
        self._h = handle

    @classmethod
    def from_file(cls, path: str) -> "BpeTokenizer":
        h = C.c_void_p()
        _raise(_native.lib().ifx_tokenizer_from_file(str(path).encode(), C.byref(h)))
        return cls(h)

    @classmethod
    def from_json(cls, raw: str | bytes) -> "BpeTokenizer":
        data = raw.encode() if isinstance(raw, str) else bytes(raw)
        buf = C.create_string_buffer(data, len(data) + 1)
        h = C.c_void_p()
        _raise(_native.lib().ifx_tokenizer_from_json(C.cast(buf, C.c_void_p), len(data), C.byref(h)))
        return cls(h)

    def encode(self, text: str | bytes) -> list[int]:
        data = text.encode() if isinstance(text, str) else bytes(text)
        buf = C.create_string_buffer(data, len(data) + 1)
        n = C.c_uint64()
        _raise(_native.lib().ifx_tokenizer_encode(self._h, C.cast(buf, C.c_void_p), len(data), None, 0, C.byref(n)))
        ids = np.zeros(max(n.value, 1), np.uint32)
        _raise(_native.lib().ifx_tokenizer_encode(self._h, C.cast(buf, C.c_void_p), len(data),
                                                  ids.ctypes.data_as(C.c_void_p), n.value, C.byref(n)))
        return ids[: n.value].tolist()

    def decode(self, tokens) -> str:
        ids = np.ascontiguousarray(tokens, dtype=np.uint32)
        n = C.c_uint64()
        _raise(_native.lib().ifx_tokenizer_decode(self._h, ids.ctypes.data_as(C.c_void_p), ids.size, None, 0,
                                                  C.byref(n)))
        out = C.create_string_buffer(max(n.value, 1))
        _raise(_native.lib().ifx_tokenizer_decode(self._h, ids.ctypes.data_as(C.c_void_p), ids.size,
                                                  C.cast(out, C.c_void_p), n.value, C.byref(n)))
        return out.raw[: n.value].decode("utf-8")

    def vocab_size(self) -> int:
        n = C.c_uint64()
        _raise(_native.lib().ifx_tokenizer_vocab_size(self._h, C.byref(n)))
        return n.value

    def close(self):
        if self._h:
            _native.lib().ifx_tokenizer_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def byte_encoder() -> list[str]:
    """GPT-2 byte table (src/tokenizer/bytes.rs:9-27), for building vocabularies in tests."""
    out, n = [], 0
    for b in range(256):
        if 0x21 <= b <= 0x7E or 0xA1 <= b <= 0xAC or 0xAE <= b <= 0xFF:
            out.append(chr(b))
        else:
            out.append(chr(0x100 + n))
            n += 1
    return out
