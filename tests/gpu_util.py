"""Device buffers and sessions through the C ABI (ctypes), for the gpu tests."""
from __future__ import annotations

import ctypes as C

import numpy as np

from inferox_amd import _native
from inferox_amd._native import check


class Dev:
    """A device allocation made with ifx_malloc."""

    def __init__(self, nbytes: int):
        self.ptr = C.c_void_p()
        self.nbytes = max(int(nbytes), 4)
        check(_native.lib().ifx_malloc(C.byref(self.ptr), self.nbytes), "ifx_malloc")

    @classmethod
    def of(cls, arr: np.ndarray) -> "Dev":
        arr = np.ascontiguousarray(arr)
        d = cls(arr.nbytes)
        if arr.nbytes:
            check(_native.lib().ifx_memcpy_h2d(d.ptr, arr.ctypes.data_as(C.c_void_p), arr.nbytes), "h2d")
        return d

    def get(self, dtype, n: int) -> np.ndarray:
        out = np.empty(n, dtype=dtype)
        check(_native.lib().ifx_stream_synchronize(None), "sync")
        check(_native.lib().ifx_memcpy_d2h(out.ctypes.data_as(C.c_void_p), self.ptr, out.nbytes), "d2h")
        return out

    def free(self):
        if self.ptr:
            _native.lib().ifx_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Tensor:
    """An uploaded weight matrix (ifx_tensor_upload)."""

    def __init__(self, ggml_type: int, raw: np.ndarray, rows: int, cols: int):
        raw = np.ascontiguousarray(raw, dtype=np.uint8)
        self.h = C.c_void_p()
        self.rows, self.cols = rows, cols
        rc = _native.lib().ifx_tensor_upload(ggml_type, raw.ctypes.data_as(C.c_void_p), raw.size, rows, cols,
                                             C.byref(self.h))
        check(rc, "ifx_tensor_upload")

    def __del__(self):
        if getattr(self, "h", None):
            _native.lib().ifx_tensor_free(self.h)
            self.h = None


class GpuModel:
    def __init__(self, path: str):
        self.h = C.c_void_p()
        check(_native.lib().ifx_model_open(path.encode(), C.byref(self.h)), f"ifx_model_open({path})")
        self.cfg = _native.IfxConfig()
        check(_native.lib().ifx_model_config(self.h, C.byref(self.cfg)), "config")
        self.vocab = self.cfg.vocab_size

    def close(self):
        if self.h:
            _native.lib().ifx_model_close(self.h)
            self.h = None

    def batched_prefill(self) -> bool:
        e = C.c_int()
        check(_native.lib().ifx_model_batched_prefill(self.h, C.byref(e)), "batched_prefill")
        return bool(e.value)

    def session(self, max_seq: int, kv_f16: bool = False) -> "GpuSession":
        return GpuSession(self, max_seq, kv_f16)

    def forward(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.zeros(max(ids.size * self.vocab, 1), np.float32)
        rc = _native.lib().ifx_forward(self.h, ids.ctypes.data_as(C.c_void_p), ids.size,
                                       out.ctypes.data_as(C.c_void_p))
        return rc, out[: ids.size * self.vocab].reshape(ids.size, self.vocab)

    def forward_last_token_logits(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.zeros(self.vocab, np.float32)
        rc = _native.lib().ifx_forward_last_token_logits(self.h, ids.ctypes.data_as(C.c_void_p), ids.size,
                                                         out.ctypes.data_as(C.c_void_p))
        return rc, out


class GpuSession:
    def __init__(self, model: GpuModel, max_seq: int, kv_f16: bool = False):
        self.model = model
        self.h = C.c_void_p()
        check(_native.lib().ifx_session_create_kv(model.h, max_seq, 1 if kv_f16 else 0, C.byref(self.h)),
              "session_create_kv")

    def close(self):
        if self.h:
            _native.lib().ifx_session_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self):
        n = C.c_uint64()
        check(_native.lib().ifx_session_len(self.h, C.byref(n)), "len")
        return n.value

    def clear(self):
        check(_native.lib().ifx_session_clear(self.h), "clear")

    def set_rope_mode(self, mode: int):
        check(_native.lib().ifx_session_set_rope_mode(self.h, mode), "rope_mode")

    def set_deterministic(self, on: bool):
        check(_native.lib().ifx_session_set_deterministic(self.h, 1 if on else 0), "set_deterministic")

    def set_prefill_batch(self, min_rows: int):
        check(_native.lib().ifx_session_set_prefill_batch(self.h, min_rows), "prefill_batch")

    def decode_step(self, token: int, want_logits=True):
        out = np.zeros(self.model.vocab, np.float32) if want_logits else None
        rc = _native.lib().ifx_decode_step(self.h, token, out.ctypes.data_as(C.c_void_p) if want_logits else None)
        return rc, out

    def prefill(self, ids, want_logits=True):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.zeros(max(ids.size * self.model.vocab, 1), np.float32) if want_logits else None
        rc = _native.lib().ifx_prefill(self.h, ids.ctypes.data_as(C.c_void_p), ids.size,
                                       out.ctypes.data_as(C.c_void_p) if want_logits else None)
        if want_logits:
            out = out[: ids.size * self.model.vocab].reshape(ids.size, self.model.vocab)
        return rc, out

    def generate(self, prompt, max_tokens: int):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(max_tokens, 1), np.uint32)
        rc = _native.lib().ifx_generate(self.h, prompt.ctypes.data_as(C.c_void_p), prompt.size, max_tokens,
                                        out.ctypes.data_as(C.c_void_p))
        return rc, out[:max_tokens]

    def set_sampler(self, temperature: float, top_k: int, top_p: float, seed: int):
        check(_native.lib().ifx_session_set_sampler(self.h, temperature, top_k, top_p, seed), "set_sampler")

    def generate_sampled(self, prompt, max_tokens: int):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(max_tokens, 1), np.uint32)
        rc = _native.lib().ifx_generate_sampled(self.h, prompt.ctypes.data_as(C.c_void_p), prompt.size, max_tokens,
                                                out.ctypes.data_as(C.c_void_p))
        return rc, out[:max_tokens]

    def decode_greedy(self, token: int, n: int):
        out = np.zeros(max(n, 1), np.uint32)
        rc = _native.lib().ifx_decode_greedy(self.h, token, n, out.ctypes.data_as(C.c_void_p))
        return rc, out[:n]

    def kv_import(self, k, v, length):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        return _native.lib().ifx_kv_import(self.h, k.ctypes.data_as(C.c_void_p), v.ctypes.data_as(C.c_void_p),
                                           length)

    def kv_export(self, length):
        c = self.model.cfg
        n = c.n_layers * length * c.n_kv_heads * c.head_dim
        k = np.zeros(max(n, 1), np.float32)
        v = np.zeros_like(k)
        check(_native.lib().ifx_kv_export(self.h, k.ctypes.data_as(C.c_void_p), v.ctypes.data_as(C.c_void_p),
                                          length), "kv_export")
        return k[:n], v[:n]

    def last_ms(self) -> float:
        ms = C.c_float()
        check(_native.lib().ifx_session_last_elapsed_ms(self.h, C.byref(ms)), "elapsed")
        return ms.value
