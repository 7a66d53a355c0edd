"""Pins of the oracle's attention loops (orc_attention_decode,
orc_attention_batch), the checker of tests/test_gpu_attention.py.

* float64: at every case the GPU tests use (head dims 48/128, groups 1/4/8,
  lengths 1..20000, flat / spread / one-hot / tie inputs) the oracle is
  within 1e-6 * sum_t p_t |v_t| of a float64 evaluation written
  independently in numpy (tests/attn_cases.py: its own head-to-kv-head map
  h // group and 1/sqrt(head_dim) scale).
* closed forms: one row gives v_0 exactly; a one-hot score gives that row's
  v; two tied rows give their mean.
* invariants: the causal chunk's row p equals the decode attention over
  rows 0..p bit for bit (src/model/forward.rs:255-303 and 383-414 share the
  loop order); FAST equals FAITHFUL bit for bit; the non-causal last row
  equals the causal last row; decode output is invariant (to rounding) under
  a permutation of the cache rows.
* the guards: dropping a chunk's rows from the oracle's input moves its
  output by what the float64 chunk-removal figure predicts.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import binding as orc
from tests import attn_cases as ac

PIN = 1e-6


@pytest.mark.parametrize("hd,group", [(48, 1), (48, 8), (128, 4), (128, 8)])
@pytest.mark.parametrize("kind", ["flat", "spread", "onehot", "tie"])
def test_oracle_decode_attention_vs_float64(hd, group, kind):
    for n in (1, 63, 65, 2048, 8193, 20000):
        nh, nkv = 2 * group, 2
        q, k, v, _ = ac.decode_case(n, nh, nkv, hd, kind, seed=n + hd + group)
        o = orc.attention_decode(q, k, v, n, nh, nkv, hd).reshape(nh, hd)
        o64, scale, _ = ac.eval64(q, k, v, nh, nkv, hd)
        err = np.linalg.norm(o - o64, axis=1) / scale
        assert err.max() <= PIN, (n, kind, float(err.max()))


def test_oracle_decode_attention_closed_forms():
    rng = np.random.default_rng(3)
    hd, nh, nkv = 64, 8, 2
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal((1, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((1, nkv * hd)).astype(np.float32)
    o = orc.attention_decode(q, k, v, 1, nh, nkv, hd).reshape(nh, hd)
    for h in range(nh):  # softmax of one score is exactly 1: o = 1 * v
        assert np.array_equal(o[h], v[0, (h // 4) * hd:(h // 4 + 1) * hd])
    for kind in ("onehot", "tie"):
        q, k, v, special = ac.decode_case(3000, nh, nkv, hd, kind, seed=11)
        o = orc.attention_decode(q, k, v, 3000, nh, nkv, hd).reshape(nh, hd)
        v3 = v.reshape(3000, nkv, hd)
        for h in range(nh):
            want = v3[special, h // 4].astype(np.float64).mean(0)
            assert np.abs(o[h] - want).max() <= 1e-5 * np.abs(want).max()


def test_oracle_decode_attention_row_permutation():
    rng = np.random.default_rng(5)
    n, hd, nh, nkv = 500, 48, 6, 2
    q, k, v, _ = ac.decode_case(n, nh, nkv, hd, "spread", seed=5)
    perm = rng.permutation(n)
    a = orc.attention_decode(q, k, v, n, nh, nkv, hd)
    b = orc.attention_decode(q, k[perm], v[perm], n, nh, nkv, hd)
    assert np.abs(a - b).max() <= 1e-5 * np.abs(a).max()


@pytest.mark.parametrize("hd,group", [(48, 1), (128, 4)])
def test_oracle_batch_attention_invariants(hd, group):
    rng = np.random.default_rng(hd)
    n, nkv = 150, 2
    nh = nkv * group
    q = rng.standard_normal((n, nh * hd)).astype(np.float32)
    k = rng.standard_normal((n, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((n, nkv * hd)).astype(np.float32)
    causal = orc.attention_batch(q, k, v, n, nh, nkv, hd, causal=True, mode=orc.MODE_FAITHFUL).reshape(n, -1)
    fast = orc.attention_batch(q, k, v, n, nh, nkv, hd, causal=True, mode=orc.MODE_FAST).reshape(n, -1)
    assert np.array_equal(causal.view(np.uint32), fast.view(np.uint32))
    full = orc.attention_batch(q, k, v, n, nh, nkv, hd, causal=False, mode=orc.MODE_FAITHFUL).reshape(n, -1)
    full_fast = orc.attention_batch(q, k, v, n, nh, nkv, hd, causal=False, mode=orc.MODE_FAST).reshape(n, -1)
    assert np.array_equal(full.view(np.uint32), full_fast.view(np.uint32))
    # row p of the causal chunk is the decode attention over rows 0..p, bit for bit
    for p in (0, 1, 63, 64, 149):
        d = orc.attention_decode(q[p], k[:p + 1], v[:p + 1], p + 1, nh, nkv, hd)
        assert np.array_equal(d.view(np.uint32), causal[p].view(np.uint32)), p
    # the last row sees every key either way
    assert np.array_equal(full[-1].view(np.uint32), causal[-1].view(np.uint32))
    # and the mask matters to the others
    assert np.abs(full[:-1] - causal[:-1]).max() > 0.1
    # float64 of a few rows
    q3 = q.astype(np.float64).reshape(n, nh, hd)
    k3, v3 = k.astype(np.float64).reshape(n, nkv, hd), v.astype(np.float64).reshape(n, nkv, hd)
    for p in (0, 70, 149):
        for h in range(nh):
            s = k3[:p + 1, h // group] @ q3[p, h] / np.sqrt(hd)
            e = np.exp(s - s.max())
            want = (e / e.sum()) @ v3[:p + 1, h // group]
            got = causal[p].reshape(nh, hd)[h]
            assert np.linalg.norm(got - want) <= PIN * np.linalg.norm(v3[:p + 1, h // group], axis=1).max()


def test_chunk_removal_matches_the_oracle():
    """The guard's float64 chunk-removal figure is what the oracle does when a
    chunk's rows are left out."""
    n, hd, nh, nkv = 1000, 128, 8, 2
    q, k, v, _ = ac.decode_case(n, nh, nkv, hd, "flat", seed=9)
    rem = ac.chunk_removal(q, k, v, nh, nkv, hd)
    o = orc.attention_decode(q, k, v, n, nh, nkv, hd).reshape(nh, hd)
    _, scale, _ = ac.eval64(q, k, v, nh, nkv, hd)
    for c in (0, 7, 15):
        keep = np.ones(n, bool)
        keep[64 * c:64 * c + 64] = False
        o2 = orc.attention_decode(q, k[keep], v[keep], int(keep.sum()), nh, nkv, hd).reshape(nh, hd)
        moved = np.linalg.norm(o2.astype(np.float64) - o, axis=1) / scale
        assert np.allclose(moved, rem[:, c], rtol=1e-3), (c, moved, rem[:, c])
