"""Test helpers for the ggml K-quant layout mode: reference-layout blocks
rewritten in ggml's layout (the inverse of the library's host conversion), and
a small Q4_K/Q6_K model written twice: once in ggml's layout with signed Q6_K
scales, once as F32 weights holding the same values (ggml's dequantization,
oracle/numpy_ref.py) for the CPU oracle."""
from __future__ import annotations

import numpy as np

from inferox_amd import synth
from inferox_amd.gguf_writer import F32, Q4_K, Q6_K, GGUFWriter
from oracle import numpy_ref as nr


def q4k_ref_to_ggml(ref: np.ndarray) -> np.ndarray:
    """Reference Q4_K blocks -> ggml's: same header; sub-block g element l (the
    reference's nibble l % 2 of qs[16 g + l / 2]) goes to the low (g even) or
    high (g odd) nibble of qs[32 (g / 2) + l]."""
    b = ref.reshape(-1, 144)
    out = b.copy()
    qs = b[:, 16:144].reshape(-1, 8, 16)
    vals = np.stack([qs & 15, qs >> 4], axis=-1).reshape(-1, 8, 32)      # [nb, g, l]
    g = np.zeros((b.shape[0], 4, 32), np.uint8)
    g |= vals[:, 0::2, :]
    g |= (vals[:, 1::2, :] << 4).astype(np.uint8)
    out[:, 16:144] = g.reshape(-1, 128)
    return out.reshape(-1)


def q6k_ref_to_ggml(ref: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Reference Q6_K blocks (their q values and d) -> ggml's, with the given
    int8 scales [nb, 16] in place of the reference's u8 ones."""
    b = ref.reshape(-1, 210)
    nb = b.shape[0]
    ql = b[:, 18:146]
    qh = b[:, 146:210]
    lo = np.stack([ql & 15, ql >> 4], axis=-1).reshape(nb, 256).astype(np.uint8)
    hi = np.stack([(qh >> s) & 3 for s in (0, 2, 4, 6)], axis=-1).reshape(nb, 256).astype(np.uint8)
    out = np.zeros((nb, 210), np.uint8)
    e = np.arange(256)
    h, j, l = e // 128, (e % 128) // 32, e % 32
    for k in range(256):
        byte = 64 * h[k] + l[k] + 32 * (j[k] & 1)
        out[:, byte] |= (lo[:, k] << (0 if j[k] < 2 else 4)).astype(np.uint8)
        out[:, 128 + 32 * h[k] + l[k]] |= (hi[:, k] << (2 * j[k])).astype(np.uint8)
    out[:, 192:208] = np.asarray(scales, np.int8).view(np.uint8)
    out[:, 208:210] = b[:, 0:2]
    return out.reshape(-1)


def _meta(w: GGUFWriter, spec):
    w.add_string("general.architecture", "llama").add_string("general.name", f"ggml-{spec.name}")
    w.add_u32("llama.vocab_size", spec.vocab).add_u32("llama.embedding_length", spec.dim)
    w.add_u32("llama.block_count", spec.n_layers).add_u32("llama.attention.head_count", spec.n_heads)
    w.add_u32("llama.attention.head_count_kv", spec.n_kv_heads)
    w.add_u32("llama.feed_forward_length", spec.ffn)
    w.add_f32("llama.attention.layer_norm_rms_epsilon", spec.eps)
    w.add_f32("llama.rope.freq_base", spec.rope_theta)
    w.add_u32("llama.context_length", spec.ctx)


SMALL = synth.LlamaSpec("small-kq", 256, 512, 2, 4, 2, 1024, 10000.0, 128, types=dict(synth._Q4KM))


def write_ggml_pair(path_ggml: str, path_f32: str, seed: int = 5):
    """SMALL in ggml's layout (Q6_K scales random int8 in [-40, 40], both signs)
    and as F32 weights of the same values."""
    rng = np.random.default_rng(seed)
    wg, wf = GGUFWriter(), GGUFWriter()
    _meta(wg, SMALL)
    _meta(wf, SMALL)
    for name, shape, t, r, c in SMALL.shapes():
        n = r * c
        raw = np.zeros(synth.byte_size(t, n), np.uint8)
        synth._filler(t, n, synth.tensor_seed(seed, name),
                      (1.0, 0.02, 0.0, 0.0) if t == F32 else None)(raw)
        if t == Q4_K:
            g = q4k_ref_to_ggml(raw)
            vals = nr.dequant_q4_k_ggml(g)
        elif t == Q6_K:
            sc = rng.integers(-40, 41, size=(raw.size // 210, 16))
            g = q6k_ref_to_ggml(raw, sc)
            vals = nr.dequant_q6_k_ggml(g)
        else:
            g = raw
            vals = nr.dequant(t, raw)
        wg.add_tensor(name, shape, t, data=g.tobytes())
        wf.add_tensor(name, shape, F32, data=np.ascontiguousarray(vals, "<f4").tobytes())
    wg.write(path_ggml)
    wf.write(path_f32)
