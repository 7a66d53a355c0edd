"""The decode step's K-split launches on their own, through
ifx_ops_gemv_residual and ifx_ops_qkv, at the benchmark widths.

* h += W x (the attn_output and ffn_down projections with the residual add,
  src/model/forward.rs:415-419,432-437): K cut into 8 slices whose partial
  sums are added into h with atomics (mode 0), against the tiled launch
  (mode 1, one summation order: two runs are bit-identical).
* q/k/v of one token (src/model/forward.rs:357-378): RMSNorm, the three
  GEMVs, RoPE at position `pos` (src/ops.rs:265-287) and the K/V append at a
  cache row.  The K-split launch rotates each slice's partial sums (RoPE is
  linear) and adds them into q and the cache row; at position 0 the rotation
  is the identity, so positions 1, 2047 and 8191 are what check it.

Bar: every output element within 1e-5 * sum_j |w_ij| |x_j| of the float64
product of the oracle's dequantized weights (after RoPE: the bound of the
pair's two rows), plus one f32 rounding of the residual add.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from inferox_amd import _native, synth
from inferox_amd.gguf_writer import Q4_K, Q6_K
from oracle import binding as orc
from tests.gpu_util import Dev, Tensor

pytestmark = pytest.mark.gpu

BOUND = 1e-5


def _matrix(t, rows, cols, seed):
    raw = synth.random_blocks(t, rows * cols, seed)
    rc, w = orc.dequantize(t, raw, rows * cols)
    assert rc == 0
    return raw, w.reshape(rows, cols).astype(np.float64)


@pytest.mark.parametrize("t,rows,cols", [(Q4_K, 4096, 4096), (Q6_K, 4096, 14336), (Q4_K, 4096, 14336),
                                         (Q6_K, 4096, 4096), (Q4_K, 8192, 8192), (Q6_K, 8192, 28672),
                                         (Q4_K, 8192, 28672)])
def test_gemv_residual_ksplit(t, rows, cols):
    print(f"gemv_residual type={t} {rows}x{cols}", flush=True)
    raw, w = _matrix(t, rows, cols, seed=rows * 3 + cols + t)
    wt = Tensor(t, raw, rows, cols)
    rng = np.random.default_rng(cols)
    x = rng.standard_normal(cols).astype(np.float32)
    h0 = rng.standard_normal(rows).astype(np.float32)
    ref = h0.astype(np.float64) + w @ x.astype(np.float64)
    tol = BOUND * (np.abs(w) @ np.abs(x).astype(np.float64)) + 2.0 ** -23 * (np.abs(h0) + np.abs(ref))
    del w
    dx = Dev.of(x)
    outs = []
    for mode, runs in ((0, 1), (1, 2)):
        for _ in range(runs):
            dh = Dev.of(h0)
            path = C.c_int(-1)
            rc = _native.lib().ifx_ops_gemv_residual(wt.h, dx.ptr, dh.ptr, mode, C.byref(path), None)
            assert rc == 0, _native.lib().ifx_last_error()
            assert path.value == (1 if mode == 0 else 0)
            got = dh.get(np.float32, rows)
            err = np.abs(got.astype(np.float64) - ref)
            assert (err <= tol).all(), (mode, int((err > tol).sum()), float((err / tol).max()))
            outs.append(got)
    # the tiled launch sums in one order
    assert (outs[1].view(np.uint32) == outs[2].view(np.uint32)).all()


def _rope_ref(x, heads, hd, rope_dim, base, pos):
    return orc.rope(x.astype(np.float32), 1, heads, hd, rope_dim, base, pos).astype(np.float64)


def _pair_bound(b, hd, rope_dim):
    """After RoPE an element mixes its row and the pair's other row."""
    i = np.arange(b.size) % hd
    partner = np.arange(b.size) ^ 1
    return np.where(i < rope_dim, b + b[partner], b)


QKV_TYPES = [(4096, Q4_K, Q6_K), (4096, Q4_K, Q4_K), (4096, Q6_K, Q6_K), (4096, Q6_K, Q4_K), (8192, Q4_K, Q6_K)]


@pytest.mark.parametrize("dim,tqk,tv", QKV_TYPES)
def test_qkv_ksplit_rope(dim, tqk, tv):
    hd, n_kv, base, eps = 128, 8, 500000.0, 1e-5
    kvd = n_kv * hd
    rq, wq = _matrix(tqk, dim, dim, seed=dim + 1)
    rk, wk = _matrix(tqk, kvd, dim, seed=dim + 2)
    rv, wv = _matrix(tv, kvd, dim, seed=dim + 3)
    tq, tk, tvv = Tensor(tqk, rq, dim, dim), Tensor(tqk, rk, kvd, dim), Tensor(tv, rv, kvd, dim)
    rng = np.random.default_rng(dim + tqk + tv)
    x = (3.0 * rng.standard_normal(dim)).astype(np.float32)
    nw = (1.0 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    xn = orc.rms_norm_rows(x, nw, eps).astype(np.float64)
    bq, bk, bv = (BOUND * (np.abs(w) @ np.abs(xn)) for w in (wq, wk, wv))
    dx, dnw = Dev.of(x), Dev.of(nw)
    max_seq = 8200
    for pos, row in ((0, 0), (1, 5), (2047, 2047), (8191, 8191)):
        q_ref = _rope_ref(wq @ xn, dim // hd, hd, hd, base, pos)
        k_ref = _rope_ref(wk @ xn, n_kv, hd, hd, base, pos)
        v_ref = wv @ xn
        tq_b, tk_b = _pair_bound(bq, hd, hd), _pair_bound(bk, hd, hd)
        for mode, f16 in ((0, False), (1, False), (0, True)):
            print(f"qkv dim={dim} types={tqk}/{tv} pos={pos} row={row} mode={mode} f16={f16}", flush=True)
            et = np.float16 if f16 else np.float32
            sentinel = np.full((n_kv, max_seq, hd), np.nan, et)
            dk, dv = Dev.of(sentinel), Dev.of(sentinel)
            dq = Dev(dim * 4)
            path = C.c_int(-1)
            rc = _native.lib().ifx_ops_qkv(tq.h, tk.h, tvv.h, dx.ptr, dnw.ptr, eps, hd, hd, base, pos, dq.ptr,
                                           dk.ptr, dv.ptr, 1 if f16 else 0, max_seq, row, mode, C.byref(path), None)
            assert rc == 0, _native.lib().ifx_last_error()
            assert path.value == (1 if (mode == 0 and not f16) else 0)
            q = dq.get(np.float32, dim).astype(np.float64)
            kc = dk.get(et, n_kv * max_seq * hd).reshape(n_kv, max_seq, hd)
            vc = dv.get(et, n_kv * max_seq * hd).reshape(n_kv, max_seq, hd)
            # only row `row` of each kv head was written
            others = np.ones(max_seq, bool)
            others[row] = False
            assert np.isnan(kc[:, others].astype(np.float32)).all() and np.isnan(vc[:, others].astype(np.float32)).all()
            k = kc[:, row].reshape(-1).astype(np.float64)
            v = vc[:, row].reshape(-1).astype(np.float64)
            assert (np.abs(q - q_ref) <= tq_b).all(), float((np.abs(q - q_ref) / tq_b).max())
            # an f16 cache holds the rounding of the f32 row: half an f16 ulp more
            slack_k = np.abs(k_ref) * 2.0 ** -11 if f16 else 0.0
            slack_v = np.abs(v_ref) * 2.0 ** -11 if f16 else 0.0
            assert (np.abs(k - k_ref) <= tk_b + slack_k).all(), float((np.abs(k - k_ref) / (tk_b + slack_k)).max())
            assert (np.abs(v - v_ref) <= bv + slack_v).all(), float((np.abs(v - v_ref) / (bv + slack_v)).max())
        if pos > 0:
            # the check can see the rotation: the unrotated rows are far outside the bound
            k0 = wk @ xn
            assert np.abs(k0 - k_ref).max() > 100 * tk_b.max()
