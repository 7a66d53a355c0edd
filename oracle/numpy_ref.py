"""Independent numpy restatement of the reference dequantizers — TEST
INFRASTRUCTURE ONLY (cross-checks oracle.c bit for bit).

Written vectorised and separately from oracle.c so that a slip in one (a
nibble order, a shift, a signedness) shows up as a mismatch against the other.
numpy float32 arithmetic is one IEEE rounding per operation with no fused
multiply-add, like the Rust reference.

Also a float64 forward of the llama block (no quantization rounding of the
activations) used as a loose brute-force check of the oracle's model code,
and restatements of ggml's Q4_K / Q6_K dequantizers (llama.cpp
ggml-quants.c, the published block_q4_K / block_q6_K definitions; not part of
the reference), the checker of the ggml-layout mode.
"""
from __future__ import annotations

import numpy as np

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K = 0, 1, 2, 7, 12, 14, 15


def _f16(b: np.ndarray) -> np.ndarray:
    """little-endian f16 byte pairs -> f32 (exact)."""
    return np.ascontiguousarray(b).view("<f2").astype(np.float32).reshape(b.shape[:-1])


def dequant_q4_0(raw: np.ndarray) -> np.ndarray:
    """src/gguf/dequant.rs:62-84"""
    blk = raw.reshape(-1, 18)
    d = _f16(blk[:, 0:2])[:, None]
    qs = blk[:, 2:18].astype(np.int32)
    lo = ((qs & 15) - 8).astype(np.float32) * d
    hi = ((qs >> 4) - 8).astype(np.float32) * d
    return np.concatenate([lo, hi], axis=1).reshape(-1)


def dequant_q8_0(raw: np.ndarray) -> np.ndarray:
    """src/gguf/dequant.rs:93-111"""
    blk = raw.reshape(-1, 34)
    d = _f16(blk[:, 0:2])[:, None]
    q = blk[:, 2:34].view(np.int8).astype(np.float32)
    return (q * d).reshape(-1)


def q4k_scales(s: np.ndarray):
    """6-bit (scale, min) per group from the 12 packed bytes (dequant.rs:141-149)."""
    s = s.astype(np.uint32)
    sc = np.empty(s.shape[:-1] + (8,), np.uint32)
    mn = np.empty_like(sc)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, mn


def dequant_q4_k(raw: np.ndarray) -> np.ndarray:
    """src/gguf/dequant.rs:123-163 (group-contiguous nibble order)."""
    blk = raw.reshape(-1, 144)
    d = _f16(blk[:, 0:2])[:, None]
    dmin = _f16(blk[:, 2:4])[:, None]
    sc, mn = q4k_scales(blk[:, 4:16])
    dall = d * sc.astype(np.float32)        # [nb, 8]
    dm = dmin * mn.astype(np.float32)
    qs = blk[:, 16:144].reshape(-1, 8, 16)
    q = np.stack([qs & 15, qs >> 4], axis=-1).reshape(-1, 8, 32).astype(np.float32)
    return (dall[:, :, None] * q - dm[:, :, None]).reshape(-1)


def dequant_q6_k(raw: np.ndarray) -> np.ndarray:
    """src/gguf/dequant.rs:174-199 (d first, u8 scales)."""
    blk = raw.reshape(-1, 210)
    d = _f16(blk[:, 0:2])[:, None]
    sc = blk[:, 2:18].astype(np.float32)            # u8, not i8
    ql = blk[:, 18:146]
    qh = blk[:, 146:210]
    lo = np.stack([ql & 15, ql >> 4], axis=-1).reshape(-1, 256).astype(np.int32)
    hi = np.stack([(qh >> s) & 3 for s in (0, 2, 4, 6)], axis=-1).reshape(-1, 256).astype(np.int32)
    q = (lo | (hi << 4)) - 32
    scale = np.repeat(sc, 16, axis=1)
    return ((d * scale) * q.astype(np.float32)).reshape(-1)


def dequant_q4_k_ggml(raw: np.ndarray) -> np.ndarray:
    """ggml's Q4_K (llama.cpp ggml-quants.c dequantize_row_q4_K; no reference
    counterpart: the checker of IFX_OPEN_GGML_KQUANTS).  The 144-byte block
    has the reference's header (d, dmin, 12 packed scale/min bytes, which
    get_scale_min_k4 unpacks as q4k_scales does); each 64-element chunk i takes
    qs[32 i .. 32 i + 32]: low nibbles for sub-block 2 i, high for 2 i + 1.
    y = d1 q - m1, d1 = d sc, m1 = dmin m."""
    blk = raw.reshape(-1, 144)
    d = _f16(blk[:, 0:2])[:, None]
    dmin = _f16(blk[:, 2:4])[:, None]
    sc, mn = q4k_scales(blk[:, 4:16])
    dall = d * sc.astype(np.float32)
    dm = dmin * mn.astype(np.float32)
    qs = blk[:, 16:144].reshape(-1, 4, 1, 32)
    q = np.concatenate([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32).astype(np.float32)
    return (dall[:, :, None] * q - dm[:, :, None]).reshape(-1)


def dequant_q6_k_ggml(raw: np.ndarray) -> np.ndarray:
    """ggml's Q6_K (llama.cpp ggml-quants.c dequantize_row_q6_K; no reference
    counterpart): block ql[128], qh[64], int8 scales[16], f16 d.  Element
    128 h + 32 j + l (j < 4, l < 32): low 4 bits from ql[64 h + l + 32 (j & 1)]
    (low nibble for j < 2, high for j >= 2), high 2 bits at bit 2 j of
    qh[32 h + l]; scale scales[8 h + l / 16 + 2 j]; y = (d sc) (q - 32)."""
    blk = raw.reshape(-1, 210)
    nb = blk.shape[0]
    ql = blk[:, 0:128].reshape(nb, 2, 64).astype(np.int32)
    qh = blk[:, 128:192].reshape(nb, 2, 32).astype(np.int32)
    sc = blk[:, 192:208].view(np.int8).astype(np.float32)
    d = _f16(blk[:, 208:210])[:, None]
    q = np.empty((nb, 2, 4, 32), np.int32)
    for j in range(4):
        lo = ql[:, :, 32 * (j & 1): 32 * (j & 1) + 32]
        nib = (lo & 15) if j < 2 else (lo >> 4)
        q[:, :, j, :] = (nib | (((qh >> (2 * j)) & 3) << 4)) - 32
    l = np.arange(32)
    sidx = (8 * np.arange(2)[:, None, None] + 2 * np.arange(4)[None, :, None] + (l // 16)[None, None, :])
    scale = sc[:, sidx]                                # [nb, 2, 4, 32]
    return ((d[:, :, None, None] * scale) * q.astype(np.float32)).reshape(-1)


def dequant_q8_k(raw: np.ndarray) -> np.ndarray:
    """src/gguf/dequant.rs:210-232"""
    blk = raw.reshape(-1, 292)
    d = _f16(blk[:, 0:2])[:, None]
    dmin = _f16(blk[:, 2:4])[:, None]
    sc = np.repeat(blk[:, 4:36].astype(np.float32), 8, axis=1)
    q = blk[:, 36:292].view(np.int8).astype(np.float32)
    return ((d * sc) * q - dmin).reshape(-1)


def dequant(ggml_type: int, raw: np.ndarray) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    if ggml_type == F32:
        return raw.view("<f4").astype(np.float32)
    if ggml_type == F16:
        return raw.view("<f2").astype(np.float32)
    return {Q4_0: dequant_q4_0, Q8_0: dequant_q8_0, Q4_K: dequant_q4_k, Q6_K: dequant_q6_k,
            Q8_K: dequant_q8_k}[ggml_type](raw)


# ---- float64 brute-force model (structure check, not bit-exact) ----

def _rms(x, w, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def _rope(x, heads, hd, rope_dim, base, positions):
    x = x.reshape(len(positions), heads, hd).copy()
    i = np.arange(0, rope_dim, 2)
    inv = 1.0 / base ** (i / rope_dim)
    ang = np.asarray(positions, dtype=np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    a, b = x[:, :, i].copy(), x[:, :, i + 1].copy()
    x[:, :, i] = a * c - b * s
    x[:, :, i + 1] = a * s + b * c
    return x.reshape(len(positions), heads * hd)


def forward64(weights: dict, cfg: dict, ids, causal: bool, positions=None):
    """float64 llama forward over `ids` with chunk-local attention.

    weights: name -> float64 array ([rows, cols] for matrices, [n] for norms);
    cfg: dim, n_heads, n_kv_heads, head_dim, rope_dim, rope_base, eps, n_layers.
    Returns logits [len(ids), vocab].
    """
    D, H, KVH, hd = cfg["dim"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    n = len(ids)
    pos = np.arange(n) if positions is None else np.asarray(positions)
    x = weights["token_embd.weight"][np.asarray(ids)]
    grp = H // KVH
    for l in range(cfg["n_layers"]):
        p = f"blk.{l}."
        r = x
        h = _rms(x, weights[p + "attn_norm.weight"], cfg["eps"])
        q = h @ weights[p + "attn_q.weight"].T
        k = h @ weights[p + "attn_k.weight"].T
        v = h @ weights[p + "attn_v.weight"].T
        q = _rope(q, H, hd, cfg["rope_dim"], cfg["rope_base"], pos)
        k = _rope(k, KVH, hd, cfg["rope_dim"], cfg["rope_base"], pos)
        out = np.zeros((n, D))
        for hq in range(H):
            hk = hq // grp
            qh = q[:, hq * hd:(hq + 1) * hd]
            kh = k[:, hk * hd:(hk + 1) * hd]
            vh = v[:, hk * hd:(hk + 1) * hd]
            s = qh @ kh.T / np.sqrt(hd)
            if causal:
                s = np.where(np.tril(np.ones((n, n), bool)), s, -np.inf)
            s = np.exp(s - s.max(axis=1, keepdims=True))
            s /= s.sum(axis=1, keepdims=True)
            out[:, hq * hd:(hq + 1) * hd] = s @ vh
        x = out @ weights[p + "attn_output.weight"].T + r
        r = x
        h = _rms(x, weights[p + "ffn_norm.weight"], cfg["eps"])
        g = h @ weights[p + "ffn_gate.weight"].T
        u = h @ weights[p + "ffn_up.weight"].T
        m = g / (1.0 + np.exp(-np.clip(g, -80, 80))) * u
        x = m @ weights[p + "ffn_down.weight"].T + r
    h = _rms(x, weights["output_norm.weight"], cfg["eps"])
    w_out = weights.get("output.weight", weights["token_embd.weight"])
    return h @ w_out.T


def sampler_probs(logits, temperature: float, top_k: int, top_p: float) -> np.ndarray:
    """Sampler::sample (src/sampler.rs:28-76) as the distribution it draws
    from, with the maxima shifted out of exp as the device sampler does
    (exp((z - m) / T) / sum = exp(z / T) / sum in exact arithmetic).  The list
    is sorted by decreasing probability with ties in index order (Rust's
    stable sort_by); top-k truncates it, top-p keeps the prefix whose running
    sum of the whole-vocabulary probabilities first reaches top_p; the kept
    probabilities renormalised.  float64 throughout."""
    z = np.asarray(logits, np.float64)
    p = np.exp((z - z.max()) / temperature)
    p /= p.sum()
    order = sorted(range(len(p)), key=lambda i: -p[i])  # stable: ties keep index order
    if top_k > 0:
        order = order[:top_k]
    if top_p < 1.0:
        c, cut = 0.0, len(order)
        for pos, i in enumerate(order):
            c += p[i]
            if c >= top_p:
                cut = pos + 1
                break
        order = order[:cut]
    out = np.zeros_like(p)
    out[order] = p[order]
    return out / out.sum()
