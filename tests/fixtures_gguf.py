"""GGUF fixtures rebuilt from the reference's own test builders (as data):

* ``weights_test_gguf``  — one F32 tensor [1.5, 2.5] (src/gguf/weights.rs:121-149)
* ``llama_wiring_gguf``  — 9 metadata keys, 21 F32 [1,1] tensors (src/model/mod.rs:136-195)
* ``builder_llama_gguf`` — TestGgufBuilder model of src/model/forward.rs:729-839
"""
from __future__ import annotations

import numpy as np

from inferox_amd.gguf_writer import GGUFWriter


def weights_test_gguf(path: str) -> None:
    w = GGUFWriter()
    w.tensor_f32("token_embeddings", [2], [1.5, 2.5])
    w.write(path)


def _llama_meta(w: GGUFWriter, vocab, dim, layers, heads, kv_heads, ffn, ctx):
    w.add_string("general.architecture", "llama")
    w.add_u32("llama.vocab_size", vocab)
    w.add_u32("llama.embedding_length", dim)
    w.add_u32("llama.block_count", layers)
    w.add_u32("llama.attention.head_count", heads)
    w.add_u32("llama.attention.head_count_kv", kv_heads)
    w.add_u32("llama.feed_forward_length", ffn)
    w.add_f32("llama.attention.layer_norm_rms_epsilon", 1e-5)
    w.add_u32("llama.context_length", ctx)


def llama_wiring_gguf(path: str) -> None:
    w = GGUFWriter()
    _llama_meta(w, 100, 64, 2, 4, 2, 128, 512)
    names = ["token_embd.weight", "output_norm.weight", "output.weight"]
    for i in range(2):
        names += [f"blk.{i}.{r}.weight" for r in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                                  "ffn_norm", "ffn_gate", "ffn_up", "ffn_down")]
    for n in names:
        w.tensor_f32(n, [1, 1], [0.0])
    w.write(path)


def builder_llama_gguf(path: str, fill: float, hidden=8, inter=16, vocab=100, ctx=128, heads=2,
                       with_output=True, layers=1) -> None:
    """The 1-layer model of the reference's forward tests.  `fill` is the value
    of the projection weights (1.0 in layer_forward_runs_without_panic, 0.0 in
    generate_with_kv_cache_runs); embeddings/output are zeros, norms ones."""
    w = GGUFWriter()
    _llama_meta(w, vocab, hidden, layers, heads, heads, inter, ctx)
    w.tensor_f32("token_embd.weight", [vocab, hidden], np.zeros(vocab * hidden))
    w.tensor_f32("output_norm.weight", [hidden], np.ones(hidden))
    if with_output:
        w.tensor_f32("output.weight", [vocab, hidden], np.zeros(vocab * hidden))
    for i in range(layers):
        p = f"blk.{i}."
        w.tensor_f32(p + "attn_norm.weight", [hidden], np.ones(hidden))
        for r in ("attn_q", "attn_k", "attn_v", "attn_output"):
            w.tensor_f32(p + r + ".weight", [hidden, hidden], np.full(hidden * hidden, fill))
        w.tensor_f32(p + "ffn_norm.weight", [hidden], np.ones(hidden))
        w.tensor_f32(p + "ffn_gate.weight", [inter, hidden], np.full(inter * hidden, fill))
        w.tensor_f32(p + "ffn_up.weight", [inter, hidden], np.full(inter * hidden, fill))
        w.tensor_f32(p + "ffn_down.weight", [hidden, inter], np.full(hidden * inter, fill))
    w.write(path)


def f16_bytes(*vals) -> bytes:
    return np.asarray(vals, dtype="<f2").tobytes()


# Known-answer blocks of src/gguf/dequant.rs:247-382, restated as bytes.
def kat_blocks():
    """[(ggml_type, raw bytes, n_elements, expected f32 array)]"""
    out = []
    # Q4_0: delta 0.5, byte (j<<4)|j  ->  ((j%16)-8)*0.5
    raw = f16_bytes(0.5) + bytes(((j << 4) | j) for j in range(16))
    out.append((2, raw, 32, np.array([((j % 16) - 8) * 0.5 for j in range(32)], np.float32)))
    # Q8_0: delta 0.25, q = 0..31  ->  j*0.25
    raw = f16_bytes(0.25) + bytes(range(32))
    out.append((7, raw, 32, np.arange(32, dtype=np.float32) * 0.25))
    # F16 [1, 2, -3]
    out.append((1, f16_bytes(1.0, 2.0, -3.0), 3, np.array([1, 2, -3], np.float32)))
    # F32 [1, 2, -3]
    out.append((0, np.array([1, 2, -3], "<f4").tobytes(), 3, np.array([1, 2, -3], np.float32)))
    # Q4_K: d=1, dmin=0, scales [1,1,1,1,0,0,0,0,1,1,1,1], qs pairs (low=2p, high=(2p+1)%32)
    qs = bytes((((((2 * p + 1) % 32) << 4) & 0xFF) | (2 * p)) for _ in range(8) for p in range(16))
    raw = f16_bytes(1.0, 0.0) + bytes([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]) + qs
    out.append((12, raw, 256, np.array([(j % 32) % 16 for j in range(256)], np.float32)))
    # Q6_K: d=1, 16 scales of 1, ql zeros, qh 0b10101010  ->  q=32  ->  zeros
    raw = f16_bytes(1.0) + bytes([1] * 16) + bytes(128) + bytes([0b10101010] * 64)
    out.append((14, raw, 256, np.zeros(256, np.float32)))
    # Q8_K: d=1, dmin=0, 32 scales of 1, qs = j as i8
    raw = f16_bytes(1.0, 0.0) + bytes([1] * 32) + bytes(j & 0xFF for j in range(256))
    out.append((15, raw, 256, np.array([np.int8(np.uint8(j)) for j in range(256)], np.float32)))
    return out
