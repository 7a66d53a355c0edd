"""Seeded attention inputs, their float64 evaluation and sensitivity guards,
shared by the oracle pins (CPU) and the GPU attention parity tests.

The decode attention of Layer::decode_step (src/model/forward.rs:383-414)
gives query head h (kv head h // group) o_h = sum_t p_t v_t with
p = softmax_t(q_h . k_t / sqrt(head_dim)).  Kinds of input:

  flat    scores std ~0.3: every cache row carries weight, and the V rows of
          each 64-row chunk share an offset (3 x N(0, 1) per element), so
          removing any one chunk moves the output.
  spread  scores std ~1.7: the softmax spreads over hundreds of rows.
  onehot  one row's key aligned with its kv head's queries (score ~+40): the
          output is that row's V.
  tie     two rows in different chunks with that same aligned key: the
          output is the mean of their two V rows.

In flat and spread the last row holds an "own key" aligned with the queries
(score ~+4 above the rest), as the row a decode step appends, so that a short
last chunk carries weight too.  K and V are [n][n_kv * head_dim] f32 (the
KvCache row layout, src/model/cache.rs:8-24); with f16=True they are rounded
to binary16 first (what an f16 cache holds).
"""
from __future__ import annotations

import numpy as np

CHUNK = 64  # rows per chunk record of the decode attention kernel


def _aligned(q_heads: np.ndarray, score: float, hd: int) -> np.ndarray:
    """The smallest key whose score q_g . k / sqrt(hd) is `score` for every
    query g of the group (the group's queries are independent: g <= 8 < hd)."""
    qm = q_heads.astype(np.float64)
    rhs = np.full(qm.shape[0], score * np.sqrt(hd))
    return (qm.T @ np.linalg.solve(qm @ qm.T, rhs)).astype(np.float32)


def decode_case(n: int, n_heads: int, n_kv: int, hd: int, kind: str, seed: int, f16: bool = False):
    """(q [n_heads*hd], k, v [n][n_kv*hd], special rows) of one case."""
    rng = np.random.default_rng(seed)
    group = n_heads // n_kv
    sigma = {"flat": 0.3, "spread": 1.7, "onehot": 1.0, "tie": 1.0}[kind]
    q = (sigma * rng.standard_normal((n_heads, hd))).astype(np.float32)
    k = rng.standard_normal((n, n_kv, hd)).astype(np.float32)
    off = rng.standard_normal(((n + CHUNK - 1) // CHUNK, n_kv, hd)).astype(np.float32)
    v = rng.standard_normal((n, n_kv, hd)).astype(np.float32)
    if kind == "flat":
        v += 3.0 * np.repeat(off, CHUNK, axis=0)[:n]
    special = []
    if kind in ("flat", "spread"):
        special = [n - 1]
        for hk in range(n_kv):
            k[n - 1, hk] = _aligned(q[hk * group:(hk + 1) * group], 4.0 + (3.0 if kind == "spread" else 0.0), hd)
    elif kind == "onehot":
        special = [int(rng.integers(0, n))]
    elif kind == "tie":
        if n < 2 * CHUNK:
            special = [0, n - 1] if n > 1 else [0]
        else:
            a = int(rng.integers(0, n // 2))
            b = int(rng.integers(n // 2, n))
            if a // CHUNK == b // CHUNK:
                b = min(n - 1, (a // CHUNK + 1) * CHUNK)
            special = [a, b]
    if kind in ("onehot", "tie"):
        for hk in range(n_kv):
            key = _aligned(q[hk * group:(hk + 1) * group], 40.0, hd)
            for t in special:
                k[t, hk] = key
    k = k.reshape(n, n_kv * hd)
    v = v.reshape(n, n_kv * hd)
    if f16:
        k = round_f16(k)
        v = round_f16(v)
    return q.reshape(-1), k, v, special


def round_f16(x: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def weights64(q, k, n_heads, n_kv, hd):
    """Softmax weights in float64: p [n_heads][n] and the unnormalised e, with
    the row max subtracted."""
    n = k.shape[0]
    group = n_heads // n_kv
    q = np.asarray(q, np.float64).reshape(n_heads, hd)
    k = np.asarray(k, np.float64).reshape(n, n_kv, hd)
    e = np.empty((n_heads, n))
    for h in range(n_heads):
        s = k[:, h // group] @ q[h] / np.sqrt(hd)
        e[h] = np.exp(s - s.max())
    return e / e.sum(1, keepdims=True), e


def eval64(q, k, v, n_heads, n_kv, hd):
    """(o [n_heads][hd], scale [n_heads], amag [n_heads][hd]) in float64:
    scale_h = sum_t p_t |v_t|_2 (the size an f32 evaluation's rounding error
    is measured against), amag_hd = sum_t p_t |v_td|."""
    n = k.shape[0]
    group = n_heads // n_kv
    p, _ = weights64(q, k, n_heads, n_kv, hd)
    v3 = np.asarray(v, np.float64).reshape(n, n_kv, hd)
    o = np.empty((n_heads, hd))
    scale = np.empty(n_heads)
    amag = np.empty((n_heads, hd))
    for h in range(n_heads):
        vh = v3[:, h // group]
        o[h] = p[h] @ vh
        scale[h] = p[h] @ np.linalg.norm(vh, axis=1)
        amag[h] = p[h] @ np.abs(vh)
    return o, scale, amag


def chunk_removal(q, k, v, n_heads, n_kv, hd):
    """[n_heads][n_chunks]: |o without chunk c - o|_2 / scale_h, in float64, for
    every 64-row chunk c (the last one may be short)."""
    n = k.shape[0]
    group = n_heads // n_kv
    _, e = weights64(q, k, n_heads, n_kv, hd)
    v3 = np.asarray(v, np.float64).reshape(n, n_kv, hd)
    starts = np.arange(0, n, CHUNK)
    out = np.empty((n_heads, len(starts)))
    for h in range(n_heads):
        vh = v3[:, h // group]
        E = np.add.reduceat(e[h], starts)
        S = np.add.reduceat(e[h][:, None] * vh, starts, axis=0)
        Et, St = e[h].sum(), (e[h][:, None] * vh).sum(0)
        o = St / Et
        rest = Et - E
        with np.errstate(invalid="ignore", divide="ignore"):
            om = (St[None] - S) / rest[:, None]
        d = np.linalg.norm(om - o[None], axis=1)
        # removing the only chunk leaves no softmax at all: as large a change as any
        d[rest <= 0] = np.inf
        scale = (e[h] / Et) @ np.linalg.norm(vh, axis=1)
        out[h] = d / scale
    return out


def guard_decode(kind, removal):
    """The chunk effect a test of this kind relies on, over every head: the
    smallest over all chunks (flat: any dropped chunk is seen), the median
    chunk (spread: the weight is uneven over chunks, a typical one is seen)
    or the largest (onehot, tie: the chunks holding the aligned rows)."""
    if kind == "flat":
        return float(removal.min())
    if kind == "spread":
        return float(np.median(removal, axis=1).min())
    return float(removal.max(1).min())
