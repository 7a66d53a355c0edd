"""ctypes loading of the native libraries built in-tree by ``inferox_amd.build``.

``libinferox.so`` is the product (HIP kernels + C++ host behind include/inferox.h).
``libifx_synth.so`` is the host-only synthetic-model payload generator.
Loading fails loudly: there is no CPU fallback for the product library.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
PRODUCT_LIB = os.path.join(LIB_DIR, "libinferox.so")
SYNTH_LIB = os.path.join(LIB_DIR, "libifx_synth.so")

_lib = None
_synth = None

u32, u64, i32, f32 = C.c_uint32, C.c_uint64, C.c_int, C.c_float
vp, cp = C.c_void_p, C.c_char_p
P = C.POINTER


class IfxConfig(C.Structure):
    _fields_ = [("vocab_size", u32), ("hidden_size", u64), ("n_layers", u64), ("n_heads", u64),
                ("n_kv_heads", u64), ("head_dim", u64), ("intermediate_size", u64),
                ("norm_eps", f32), ("rope_base", f32), ("rope_dim", u64), ("context_length", u64),
                ("architecture", C.c_char * 32)]


# name -> (restype, argtypes); mirrors include/inferox.h
SIGNATURES = {
    "ifx_last_error": (cp, []),
    "ifx_status_string": (cp, [i32]),
    "ifx_model_open": (i32, [cp, P(vp)]),
    "ifx_model_close": (None, [vp]),
    "ifx_model_config": (i32, [vp, P(IfxConfig)]),
    "ifx_model_weight_bytes": (i32, [vp, P(u64), P(u64)]),
    "ifx_session_create": (i32, [vp, u64, P(vp)]),
    "ifx_session_create_kv": (i32, [vp, u64, i32, P(vp)]),
    "ifx_model_open_ex": (i32, [cp, u32, P(vp)]),
    "ifx_tensor_upload_ex": (i32, [u32, vp, u64, u64, u64, u32, P(vp)]),
    "ifx_tokenizer_from_file": (i32, [cp, P(vp)]),
    "ifx_tokenizer_from_json": (i32, [vp, u64, P(vp)]),
    "ifx_tokenizer_free": (None, [vp]),
    "ifx_tokenizer_encode": (i32, [vp, vp, u64, vp, u64, P(u64)]),
    "ifx_tokenizer_decode": (i32, [vp, vp, u64, vp, u64, P(u64)]),
    "ifx_tokenizer_vocab_size": (i32, [vp, P(u64)]),
    "ifx_session_destroy": (None, [vp]),
    "ifx_session_clear": (i32, [vp]),
    "ifx_session_len": (i32, [vp, P(u64)]),
    "ifx_session_set_rope_mode": (i32, [vp, i32]),
    "ifx_session_set_prefill_batch": (i32, [vp, u64]),
    "ifx_model_batched_prefill": (i32, [vp, P(i32)]),
    "ifx_decode_step": (i32, [vp, u32, vp]),
    "ifx_prefill": (i32, [vp, vp, u64, vp]),
    "ifx_forward": (i32, [vp, vp, u64, vp]),
    "ifx_forward_last_token_logits": (i32, [vp, vp, u64, vp]),
    "ifx_generate": (i32, [vp, vp, u64, u64, vp]),
    "ifx_decode_greedy": (i32, [vp, u32, u64, vp]),
    "ifx_session_set_sampler": (i32, [vp, C.c_float, u32, C.c_float, u64]),
    "ifx_generate_sampled": (i32, [vp, vp, u64, u64, vp]),
    "ifx_sample_logits": (i32, [vp, u32, C.c_float, u32, C.c_float, u64, u32, vp]),
    "ifx_kv_import": (i32, [vp, vp, vp, u64]),
    "ifx_kv_export": (i32, [vp, vp, vp, u64]),
    "ifx_session_last_elapsed_ms": (i32, [vp, P(f32)]),
    "ifx_session_last_token": (i32, [vp, P(u32)]),
    "ifx_session_profile": (i32, [vp, u32, u64, P(f32), P(u64), P(u64)]),
    "ifx_session_profile_ordered": (i32, [vp, u32, u64, P(f32)]),
    "ifx_device_info": (i32, [cp, u64, P(i32), P(u64)]),
    "ifx_malloc": (i32, [P(vp), u64]),
    "ifx_free": (i32, [vp]),
    "ifx_memcpy_h2d": (i32, [vp, vp, u64]),
    "ifx_memcpy_d2h": (i32, [vp, vp, u64]),
    "ifx_memcpy_d2d": (i32, [vp, vp, u64]),
    "ifx_stream_synchronize": (i32, [vp]),
    "ifx_timer_start": (i32, [vp]),
    "ifx_timer_stop": (i32, [vp, P(f32)]),
    "ifx_dequantize_f32": (i32, [u32, u64, vp, u64, vp, u64, vp]),
    "ifx_tensor_upload": (i32, [u32, vp, u64, u64, u64, P(vp)]),
    "ifx_tensor_free": (None, [vp]),
    "ifx_tensor_bytes": (i32, [vp, P(u64), P(u64)]),
    "ifx_tensor_dequant": (i32, [vp, vp, vp]),
    "ifx_gemv": (i32, [vp, vp, vp, vp]),
    "ifx_matmul_qt": (i32, [vp, u64, vp, vp, vp]),
    "ifx_matmul_qt_noalloc": (i32, [vp, u64, vp, vp, vp]),
    "ifx_ops_matmul_t": (i32, [vp, vp, vp, u64, u64, u64, vp]),
    "ifx_ops_rms_norm_rows": (i32, [vp, vp, u64, u64, f32, vp]),
    "ifx_ops_swiglu": (i32, [vp, vp, vp, u64, vp]),
    "ifx_ops_add_in_place": (i32, [vp, vp, u64, vp]),
    "ifx_ops_softmax_rows": (i32, [vp, u64, u64, vp]),
    "ifx_ops_rope": (i32, [vp, u64, u64, u64, u64, f32, u64, vp]),
    "ifx_ops_embedding_lookup": (i32, [vp, vp, u64, vp, vp]),
    "ifx_ops_argmax": (i32, [vp, u64, vp, vp, vp]),
    "ifx_ops_attention_decode": (i32, [vp, vp, vp, i32, u64, u64, u64, u64, u64, vp, vp]),
    "ifx_ops_attention_decode_o": (i32, [vp, vp, vp, i32, u64, u64, u64, u64, u64, vp, vp, u32, vp, vp]),
    "ifx_ops_attention_prefill": (i32, [vp, vp, vp, i32, u64, u64, u64, u64, u64, u64, i32, vp, vp]),
    "ifx_ops_gemv_residual": (i32, [vp, vp, vp, i32, P(i32), vp]),
    "ifx_ops_qkv": (i32, [vp, vp, vp, vp, vp, f32, u64, u64, f32, u64, vp, vp, vp, i32, u64, u64, i32, P(i32), vp]),
    "ifx_session_set_deterministic": (i32, [vp, i32]),
}


def lib() -> C.CDLL:
    """The product library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(PRODUCT_LIB):
            raise RuntimeError(f"{PRODUCT_LIB} is missing: run __graft_entry__.build() first "
                               "(there is no CPU fallback)")
        L = C.CDLL(PRODUCT_LIB)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def synth() -> C.CDLL:
    global _synth
    if _synth is None:
        if not os.path.exists(SYNTH_LIB):
            raise RuntimeError(f"{SYNTH_LIB} is missing: run __graft_entry__.build() first")
        L = C.CDLL(SYNTH_LIB)
        L.ifx_synth_fill.restype = i32
        L.ifx_synth_fill.argtypes = [vp, u32, u64, u64, C.c_double, C.c_double, C.c_double, C.c_double]
        L.ifx_synth_fill_centred.restype = i32
        L.ifx_synth_fill_centred.argtypes = [vp, u32, u64, u64, C.c_double, C.c_double, C.c_double]
        L.ifx_synth_token_ids.restype = None
        L.ifx_synth_token_ids.argtypes = [vp, u64, u32, u64]
        L.ifx_synth_normal_f32.restype = None
        L.ifx_synth_normal_f32.argtypes = [vp, u64, u64, f32, f32]
        L.ifx_synth_f32_to_f16.restype = C.c_uint16
        L.ifx_synth_f32_to_f16.argtypes = [f32]
        _synth = L
    return _synth


class IfxError(RuntimeError):
    def __init__(self, status: int, where: str):
        msg = ""
        try:
            raw = lib().ifx_last_error()
            msg = raw.decode() if raw else ""
        except Exception:  # pragma: no cover - message is best effort
            pass
        super().__init__(f"{where}: status {status} ({STATUS_NAMES.get(status, '?')}) {msg}")
        self.status = status


STATUS_NAMES = {0: "OK", 1: "Io", 2: "InvalidMagic", 3: "UnsupportedVersion", 4: "UnknownValueType",
                5: "UnknownTensorType", 6: "InvalidUtf8", 7: "InvalidShape", 8: "UnexpectedEof",
                9: "TensorNotFound", 10: "InvalidTensorIndex", 11: "TensorOffsetOverflow",
                12: "UnsupportedArchitecture", 20: "InvalidArg", 21: "KvFull", 22: "Hip", 23: "Oom",
                24: "NanLogit", 25: "NoDevice"}


def check(status: int, where: str) -> None:
    if status != 0:
        raise IfxError(status, where)
