"""ctypes binding of oracle/liboracle.so — TEST INFRASTRUCTURE ONLY.

The oracle is the CPU restatement of the reference token loop that the HIP
path is checked against.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

u32, u64, i32, f32 = C.c_uint32, C.c_uint64, C.c_int, C.c_float
vp, cp = C.c_void_p, C.c_char_p
P = C.POINTER

MODE_FAITHFUL, MODE_FAST = 0, 1
ROPE_REFERENCE, ROPE_ABSOLUTE = 0, 1


class OrcConfig(C.Structure):
    _fields_ = [("vocab_size", u32), ("hidden_size", u64), ("n_layers", u64), ("n_heads", u64),
                ("n_kv_heads", u64), ("head_dim", u64), ("intermediate_size", u64),
                ("norm_eps", f32), ("rope_base", f32), ("rope_dim", u64), ("context_length", u64)]


_SIGS = {
    "orc_f16_to_f32": (f32, [C.c_uint16]),
    "orc_block_layout": (i32, [u32, P(u64), P(u64)]),
    "orc_byte_size": (i32, [u32, u64, P(u64)]),
    "orc_dequantize_f32": (i32, [u32, u64, vp, u64, vp, u64]),
    "orc_matmul_t": (None, [vp, vp, vp, u64, u64, u64]),
    "orc_matmul_t_scalar": (None, [vp, vp, vp, u64, u64, u64]),
    "orc_rms_norm": (None, [vp, vp, u64, f32]),
    "orc_rms_norm_rows": (None, [vp, vp, u64, u64, f32]),
    "orc_silu": (None, [vp, u64]),
    "orc_swiglu": (None, [vp, vp, vp, u64]),
    "orc_add_in_place": (None, [vp, vp, u64]),
    "orc_softmax_rows": (None, [vp, u64, u64]),
    "orc_embedding_lookup": (i32, [vp, u64, vp, u64, u64, vp]),
    "orc_rope": (None, [vp, u64, u64, u64, u64, f32, u64]),
    "orc_argmax": (i32, [vp, u64, P(u32)]),
    "orc_attention_decode": (i32, [vp, vp, vp, u64, u64, u64, u64, vp]),
    "orc_attention_batch": (i32, [vp, vp, vp, u64, u64, u64, u64, i32, vp, i32]),
    "orc_model_open": (i32, [cp, P(vp)]),
    "orc_model_close": (None, [vp]),
    "orc_model_config": (i32, [vp, P(OrcConfig)]),
    "orc_model_n_tensors": (i32, [vp, P(u64)]),
    "orc_model_tensor_info": (i32, [vp, u64, cp, u64, P(u32), P(u64), P(u64), P(u64)]),
    "orc_model_tensor_bytes": (i32, [vp, u64, P(vp), P(u64)]),
    "orc_kv_new": (vp, [vp, u64]),
    "orc_kv_free": (None, [vp]),
    "orc_kv_clear": (None, [vp]),
    "orc_kv_set_f16": (None, [vp, i32]),
    "orc_round_f16": (f32, [f32]),
    "orc_kv_len": (u64, [vp]),
    "orc_kv_import": (i32, [vp, vp, vp, u64]),
    "orc_kv_export": (i32, [vp, vp, vp, u64]),
    "orc_set_threads": (None, [i32]),
    "orc_decode_step": (i32, [vp, vp, u32, vp, i32, i32]),
    "orc_prefill": (i32, [vp, vp, vp, u64, vp, i32, i32]),
    "orc_prefill_rows": (i32, [vp, vp, vp, u64, vp, u64, vp, i32, i32]),
    "orc_dequantize_fast": (i32, [u32, u64, vp, vp]),
    "orc_forward_rows": (i32, [vp, vp, u64, vp, u64, vp, i32]),
    "orc_forward": (i32, [vp, vp, u64, vp, i32]),
    "orc_generate": (i32, [vp, vp, vp, u64, u64, vp, i32, i32]),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: build with `make -C oracle`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(vp)


def dequantize(ggml_type: int, raw: np.ndarray, n_elements: int, n_out: int | None = None):
    """(status, f32 array) of gguf::dequantize_f32 restated."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    n_out = n_elements if n_out is None else n_out
    out = np.zeros(max(n_out, 1), dtype=np.float32)
    rc = lib().orc_dequantize_f32(ggml_type, n_elements, _ptr(raw), raw.size, _ptr(out), n_out)
    return rc, out[:n_out]


def dequantize_fast(ggml_type: int, raw: np.ndarray, n_elements: int):
    """The FAST-mode dequantization of whole blocks (equals dequantize)."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.zeros(max(n_elements, 1), dtype=np.float32)
    rc = lib().orc_dequantize_fast(ggml_type, n_elements, _ptr(raw), _ptr(out))
    return rc, out[:n_elements]


def matmul_t(a: np.ndarray, b: np.ndarray, m: int, n: int, k: int, scalar: bool = False):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    c = np.zeros(m * n, dtype=np.float32)
    fn = lib().orc_matmul_t_scalar if scalar else lib().orc_matmul_t
    fn(_ptr(a), _ptr(b), _ptr(c), m, n, k)
    return c


def attention_decode(q, k, v, n_rows, n_heads, n_kv_heads, head_dim):
    """The decode step's attention (src/model/forward.rs:383-414): q [n_heads*hd]
    over rows 0..n_rows-1 of k, v [t][n_kv_heads*hd]; returns out [n_heads*hd]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.zeros(n_heads * head_dim, dtype=np.float32)
    rc = lib().orc_attention_decode(_ptr(q), _ptr(k), _ptr(v), n_rows, n_heads, n_kv_heads, head_dim, _ptr(out))
    if rc != 0:
        raise ValueError(f"orc_attention_decode: status {rc}")
    return out


def attention_batch(q, k, v, seq, n_heads, n_kv_heads, head_dim, causal=True, mode=MODE_FAST):
    """A prefill (causal) or forward chunk's attention (src/model/forward.rs:
    255-303, 104-156): q [seq][n_heads*hd], k, v [seq][n_kv*hd] -> [seq][n_heads*hd]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.zeros(seq * n_heads * head_dim, dtype=np.float32)
    rc = lib().orc_attention_batch(_ptr(q), _ptr(k), _ptr(v), seq, n_heads, n_kv_heads, head_dim, int(causal),
                                   _ptr(out), mode)
    if rc != 0:
        raise ValueError(f"orc_attention_batch: status {rc}")
    return out


def rms_norm_rows(x, w, eps, rows=None):
    x = np.array(x, dtype=np.float32, copy=True)
    w = np.ascontiguousarray(w, dtype=np.float32)
    n = w.size
    rows = x.size // n if rows is None else rows
    lib().orc_rms_norm_rows(_ptr(x), _ptr(w), n, rows, eps)
    return x


def softmax_rows(x, rows, cols):
    x = np.array(x, dtype=np.float32, copy=True)
    lib().orc_softmax_rows(_ptr(x), rows, cols)
    return x


def swiglu(g, u):
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    o = np.zeros_like(g)
    lib().orc_swiglu(_ptr(g), _ptr(u), _ptr(o), g.size)
    return o


def silu(x):
    x = np.array(x, dtype=np.float32, copy=True)
    lib().orc_silu(_ptr(x), x.size)
    return x


def add_in_place(o, b):
    o = np.array(o, dtype=np.float32, copy=True)
    b = np.ascontiguousarray(b, dtype=np.float32)
    lib().orc_add_in_place(_ptr(o), _ptr(b), o.size)
    return o


def round_f16(x) -> np.ndarray:
    """Elementwise orc_round_f16 (binary16 rounding of the f16-KV mode), as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    f = lib().orc_round_f16
    return np.array([f(float(v)) for v in x], dtype=np.float32)


def rope(x, seq, heads, hd, rope_dim, base, pos0=0):
    x = np.array(x, dtype=np.float32, copy=True)
    lib().orc_rope(_ptr(x), seq, heads, hd, rope_dim, base, pos0)
    return x


def argmax(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = u32(0)
    rc = lib().orc_argmax(_ptr(x), x.size, C.byref(out))
    return rc, out.value


def f16_to_f32(h: int) -> float:
    return lib().orc_f16_to_f32(h)


class Model:
    """The oracle's Model + KvCache (src/model/{mod,cache,forward}.rs)."""

    def __init__(self, path: str):
        self.h = vp()
        rc = lib().orc_model_open(path.encode(), C.byref(self.h))
        if rc != 0:
            self.h = None
            raise OracleError(rc, f"orc_model_open({path})")
        c = OrcConfig()
        lib().orc_model_config(self.h, C.byref(c))
        self.cfg = c
        self.vocab = c.vocab_size

    @staticmethod
    def open_status(path: str) -> int:
        h = vp()
        rc = lib().orc_model_open(path.encode(), C.byref(h))
        if rc == 0:
            lib().orc_model_close(h)
        return rc

    def close(self):
        if self.h:
            lib().orc_model_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def tensor_infos(self):
        n = u64(0)
        lib().orc_model_n_tensors(self.h, C.byref(n))
        out = []
        for i in range(n.value):
            name = C.create_string_buffer(256)
            t, nd, off = u32(), u64(), u64()
            shape = (u64 * 4)()
            lib().orc_model_tensor_info(self.h, i, name, 256, C.byref(t), C.byref(nd), shape, C.byref(off))
            out.append((name.value.decode(), t.value, list(shape)[: nd.value], off.value))
        return out

    def tensor_bytes(self, idx: int) -> np.ndarray:
        p, n = vp(), u64()
        rc = lib().orc_model_tensor_bytes(self.h, idx, C.byref(p), C.byref(n))
        if rc != 0:
            raise OracleError(rc, "tensor_bytes")
        return np.ctypeslib.as_array(C.cast(p, P(C.c_uint8)), shape=(n.value,)).copy()

    def kv(self, max_seq_len: int, f16: bool = False) -> "KvCache":
        """A cache; f16=True rounds every row stored to binary16 (the f16-KV mode)."""
        kv = KvCache(self, max_seq_len)
        if f16:
            lib().orc_kv_set_f16(kv.h, 1)
        return kv

    def decode_step(self, kv: "KvCache", token: int, mode=MODE_FAST, rope_mode=ROPE_REFERENCE):
        logits = np.zeros(max(self.vocab, 1), dtype=np.float32)
        rc = lib().orc_decode_step(self.h, kv.h, token, _ptr(logits), mode, rope_mode)
        return rc, logits[: self.vocab]

    def prefill(self, kv: "KvCache", ids, mode=MODE_FAST, rope_mode=ROPE_REFERENCE):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        logits = np.zeros(max(ids.size * self.vocab, 1), dtype=np.float32)
        rc = lib().orc_prefill(self.h, kv.h, _ptr(ids), ids.size, _ptr(logits), mode, rope_mode)
        return rc, logits[: ids.size * self.vocab].reshape(ids.size, self.vocab)

    def prefill_rows(self, kv: "KvCache", ids, rows, mode=MODE_FAST, rope_mode=ROPE_REFERENCE):
        """prefill, with the logits of the listed rows only ([len(rows) x vocab])."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        rows = np.ascontiguousarray(rows, dtype=np.uint64)
        logits = np.zeros(max(rows.size * self.vocab, 1), dtype=np.float32)
        rc = lib().orc_prefill_rows(self.h, kv.h, _ptr(ids), ids.size, _ptr(rows), rows.size, _ptr(logits), mode,
                                    rope_mode)
        return rc, logits[: rows.size * self.vocab].reshape(rows.size, self.vocab)

    def forward_rows(self, ids, rows, mode=MODE_FAST):
        """forward, with the logits of the listed rows only ([len(rows) x vocab])."""
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        rows = np.ascontiguousarray(rows, dtype=np.uint64)
        logits = np.zeros(max(rows.size * self.vocab, 1), dtype=np.float32)
        rc = lib().orc_forward_rows(self.h, _ptr(ids), ids.size, _ptr(rows), rows.size, _ptr(logits), mode)
        return rc, logits[: rows.size * self.vocab].reshape(rows.size, self.vocab)

    def forward(self, ids, mode=MODE_FAST):
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        logits = np.zeros(max(ids.size * self.vocab, 1), dtype=np.float32)
        rc = lib().orc_forward(self.h, _ptr(ids), ids.size, _ptr(logits), mode)
        return rc, logits[: ids.size * self.vocab].reshape(ids.size, self.vocab)

    def generate(self, kv: "KvCache", prompt, max_tokens: int, mode=MODE_FAST, rope_mode=ROPE_REFERENCE):
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.zeros(max(max_tokens, 1), dtype=np.uint32)
        rc = lib().orc_generate(self.h, kv.h, _ptr(prompt), prompt.size, max_tokens, _ptr(out), mode, rope_mode)
        return rc, out[:max_tokens]


class KvCache:
    def __init__(self, model: Model, max_seq_len: int):
        self.model = model
        self.h = lib().orc_kv_new(model.h, max_seq_len)
        self.max_seq_len = max_seq_len

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_kv_free(self.h)
            self.h = None

    def clear(self):
        lib().orc_kv_clear(self.h)

    def __len__(self):
        return int(lib().orc_kv_len(self.h))

    def import_(self, k: np.ndarray, v: np.ndarray, length: int):
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        return lib().orc_kv_import(self.h, _ptr(k), _ptr(v), length)

    def export(self, length: int):
        c = self.model.cfg
        kvd = c.n_kv_heads * c.head_dim
        k = np.zeros(c.n_layers * length * kvd, dtype=np.float32)
        v = np.zeros_like(k)
        rc = lib().orc_kv_export(self.h, _ptr(k), _ptr(v), length)
        if rc != 0:
            raise OracleError(rc, "kv_export")
        return k, v


class OracleError(RuntimeError):
    def __init__(self, status, where):
        super().__init__(f"{where}: oracle status {status}")
        self.status = status


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)
