"""Seeded synthetic llama GGUF models.

Shapes, weight types and value distributions follow the benchmark workloads:
  * ``tiny``: dim 288, ffn 768, 6 layers, 6/6 heads (head_dim 48), vocab 32000,
    rope_theta 1e4, all linear weights and the embedding/output in Q8_0
    (delta f16 ~ U[0.001, 0.01], quants ~ U[-127, 127]).
  * ``llama3-8b``: dim 4096, 32 layers, 32/8 heads (head_dim 128), ffn 14336,
    vocab 128256, rope_theta 5e5; Q4_K for attn_q/k/o, ffn_gate/up and the
    embedding, Q6_K for attn_v, ffn_down and output.
  * ``llama3-70b``: dim 8192, 80 layers, 64/8 heads, ffn 28672, same quant mix.
Norm weights are f32 ~ N(1, 0.02).  Q4_K blocks: d ~ U[1e-3, 1e-2],
dmin ~ U[0, 5e-3], uniform scale and quant bytes.  Q6_K blocks (reference
layout, d first): d ~ U[1e-4, 1e-3], scales i8 ~ U[-32, 31], uniform ql/qh.

Payloads come from ``libifx_synth.so`` (counter-based per-block streams), so a
(spec, seed) pair names exactly one file regardless of thread count.

A spec with ``centred=True`` is a parity-test model instead: its Q4_K and
Q6_K matrices are zero-mean (``ifx_synth_fill_centred``) and scaled so that a
matrix-vector product with a unit-RMS input has output std ``CENTRED_GAIN``
of its role.  With the uniform bytes above every Q4_K element has mean ~1.2,
so a token's own key dominates the attention scores and the greedy pick
hardly moves; in a centred model q.k / sqrt(head_dim) has std ~1.5, the
softmax spreads over many cache rows and the logits follow the attention.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field, replace
from typing import Dict, Optional

import numpy as np

from . import _native
from .gguf_writer import F16, F32, Q4_0, Q4_K, Q6_K, Q8_0, GGUFWriter, byte_size

DIST = {  # per-type payload parameters (p0, p1, p2, p3) for ifx_synth_fill
    Q4_K: (1e-3, 1e-2, 0.0, 5e-3),
    Q6_K: (1e-4, 1e-3, 0.0, 0.0),
    Q8_0: (1e-3, 1e-2, 0.0, 0.0),
    Q4_0: (1e-3, 1e-2, 0.0, 0.0),
    F16: (0.0, 0.02, 0.0, 0.0),
    F32: (0.0, 0.02, 0.0, 0.0),
}

ROLES = ("q", "k", "v", "o", "gate", "up", "down")


@dataclass(frozen=True)
class LlamaSpec:
    name: str
    dim: int
    ffn: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    vocab: int
    rope_theta: float
    ctx: int
    eps: float = 1e-5
    types: Dict[str, int] = field(default_factory=dict)
    tied_output: bool = False
    centred: bool = False
    # per-layer type overrides: {layer: {role: type}} (real Q4_K_M files give
    # attn_v / ffn_down Q6_K in some layers only)
    layer_types: Dict[int, Dict[str, int]] = field(default_factory=dict)

    @property
    def head_dim(self) -> int:
        return self.dim // self.n_heads

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    def t(self, role: str, layer: Optional[int] = None) -> int:
        if layer is not None and role in self.layer_types.get(layer, {}):
            return self.layer_types[layer][role]
        return self.types[role]

    def shapes(self):
        """(name, ggml shape [ne0=cols, ne1=rows], type, rows, cols) for every tensor."""
        D, Fd, V, KV = self.dim, self.ffn, self.vocab, self.kv_dim
        out = [("token_embd.weight", self.t("embd"), V, D), ("output_norm.weight", F32, 1, D)]
        if not self.tied_output:
            out.append(("output.weight", self.t("output"), V, D))
        for i in range(self.n_layers):
            p = f"blk.{i}."
            t = lambda role: self.t(role, i)  # noqa: E731
            out += [(p + "attn_norm.weight", F32, 1, D), (p + "attn_q.weight", t("q"), D, D),
                    (p + "attn_k.weight", t("k"), KV, D), (p + "attn_v.weight", t("v"), KV, D),
                    (p + "attn_output.weight", t("o"), D, D), (p + "ffn_norm.weight", F32, 1, D),
                    (p + "ffn_gate.weight", t("gate"), Fd, D), (p + "ffn_up.weight", t("up"), Fd, D),
                    (p + "ffn_down.weight", t("down"), D, Fd)]
        return [(n, ([c] if r == 1 else [c, r]), t, r, c) for (n, t, r, c) in out]

    def gguf_bytes(self) -> int:
        return sum(byte_size(t, r * c) for (_, _, t, r, c) in self.shapes())


_ALL_Q8 = {r: Q8_0 for r in ROLES} | {"embd": Q8_0, "output": Q8_0}
_Q4KM = {"q": Q4_K, "k": Q4_K, "o": Q4_K, "gate": Q4_K, "up": Q4_K, "v": Q6_K, "down": Q6_K,
         "embd": Q4_K, "output": Q6_K}

TINY = LlamaSpec("tiny", 288, 768, 6, 6, 6, 32000, 10000.0, 256, types=_ALL_Q8)
LLAMA3_8B = LlamaSpec("llama3-8b", 4096, 14336, 32, 32, 8, 128256, 500000.0, 2560, types=_Q4KM)
LLAMA3_70B = LlamaSpec("llama3-70b", 8192, 28672, 80, 64, 8, 128256, 500000.0, 8448, types=_Q4KM)
SPECS = {s.name: s for s in (TINY, LLAMA3_8B, LLAMA3_70B)}


# centred models: output std of each role's matrix-vector product for a
# unit-RMS input (the embedding: std of its elements)
CENTRED_GAIN = {"embd": 1.0, "q": 1.25, "k": 1.25, "v": 1.0, "o": 1.0, "gate": 1.0, "up": 1.0, "down": 1.0,
                "output": 2.0}
CENTRED_Q6_SC_MAX = 3  # Q6_K scale bytes 1..3: d stays in f16's normal range at 28672 columns
_ELEM_STD_PER_D = {Q4_K: 168.5, Q6_K: 40.0}  # element std / d of the centred blocks


def role_of(name: str) -> str:
    if name == "token_embd.weight":
        return "embd"
    if name == "output.weight":
        return "output"
    base = name.split(".")[-2]  # blk.{i}.<base>.weight
    return {"attn_q": "q", "attn_k": "k", "attn_v": "v", "attn_output": "o", "ffn_gate": "gate",
            "ffn_up": "up", "ffn_down": "down"}.get(base, base)


def centred_params(ggml_type: int, cols: int, role: str):
    """(d_lo, d_hi, q6_scale_max) of a centred matrix of `cols` columns."""
    std = CENTRED_GAIN[role] if role == "embd" else CENTRED_GAIN[role] / float(np.sqrt(cols))
    d = std / _ELEM_STD_PER_D[ggml_type]
    return (0.75 * d, 1.25 * d, float(CENTRED_Q6_SC_MAX))


def fnv1a64(s: str) -> int:
    h = 0xCBF29CE484222325
    for b in s.encode():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def tensor_seed(master: int, name: str) -> int:
    return (fnv1a64(name) ^ ((master * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF)) & 0xFFFFFFFFFFFFFFFF


def _filler(ggml_type: int, n: int, seed: int, params=None):
    p = params if params is not None else DIST[ggml_type]

    def fill(view: np.ndarray) -> None:
        ptr = view.ctypes.data_as(C.c_void_p)
        rc = _native.synth().ifx_synth_fill(ptr, ggml_type, n, seed, *p)
        if rc != 0:
            raise ValueError(f"synth fill failed for type {ggml_type}")
    return fill


def _centred_filler(ggml_type: int, n: int, seed: int, params):
    def fill(view: np.ndarray) -> None:
        rc = _native.synth().ifx_synth_fill_centred(view.ctypes.data_as(C.c_void_p), ggml_type, n, seed, *params)
        if rc != 0:
            raise ValueError(f"synth centred fill failed for type {ggml_type}")
    return fill


def write_llama(path: str, spec: LlamaSpec, seed: int = 1234, norm_mean: float = 1.0,
                norm_std: float = 0.02) -> int:
    """Write `spec` as a GGUF file at `path`; returns the file size."""
    w = GGUFWriter()
    w.add_string("general.architecture", "llama").add_string("general.name", f"synthetic-{spec.name}")
    w.add_u32("llama.vocab_size", spec.vocab).add_u32("llama.embedding_length", spec.dim)
    w.add_u32("llama.block_count", spec.n_layers).add_u32("llama.attention.head_count", spec.n_heads)
    w.add_u32("llama.attention.head_count_kv", spec.n_kv_heads)
    w.add_u32("llama.feed_forward_length", spec.ffn)
    w.add_f32("llama.attention.layer_norm_rms_epsilon", spec.eps)
    w.add_f32("llama.rope.freq_base", spec.rope_theta)
    w.add_u32("llama.context_length", spec.ctx)
    w.add_u64("inferox.synth.seed", seed)
    if spec.centred:
        w.add_u32("inferox.synth.centred", 1)
    for name, shape, t, r, c in spec.shapes():
        n = r * c
        if spec.centred and t in (Q4_K, Q6_K):
            fill = _centred_filler(t, n, tensor_seed(seed, name), centred_params(t, c, role_of(name)))
        else:
            params = (norm_mean, norm_std, 0.0, 0.0) if t == F32 and name.endswith("norm.weight") else None
            fill = _filler(t, n, tensor_seed(seed, name), params)
        w.add_tensor(name, shape, t, fill=fill)
    return w.write(path)


def token_ids(n: int, vocab: int, seed: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    _native.synth().ifx_synth_token_ids(out.ctypes.data_as(C.c_void_p), n, vocab, seed)
    return out


def normal_f32(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _native.synth().ifx_synth_normal_f32(out.ctypes.data_as(C.c_void_p), n, seed, mean, std)
    return out


def random_blocks(ggml_type: int, n_elements: int, seed: int, params=None) -> np.ndarray:
    """Seeded raw block bytes of one tensor (same generator as the model files)."""
    buf = np.zeros(byte_size(ggml_type, n_elements), dtype=np.uint8)
    _filler(ggml_type, n_elements, seed, params)(buf)
    return buf


def random_centred_blocks(ggml_type: int, n_elements: int, cols: int, role: str, seed: int) -> np.ndarray:
    """Seeded zero-mean Q4_K / Q6_K block bytes of a [n_elements / cols x cols]
    matrix of `role`, as a centred model's (same generator)."""
    buf = np.zeros(byte_size(ggml_type, n_elements), dtype=np.uint8)
    _centred_filler(ggml_type, n_elements, seed, centred_params(ggml_type, cols, role))(buf)
    return buf


def reduced(spec: LlamaSpec, **kw) -> LlamaSpec:
    """A copy of `spec` with fields replaced (e.g. fewer layers for parity runs)."""
    return replace(spec, **kw)
