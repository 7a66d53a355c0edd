"""Kernel-level parity on the GPU, through the C ABI, against the oracle.

Bar: bit-exact for dequantization (every type, raw stream and device layout)
and the embedding gather; for the fused GEMV and the f32 operators, relative
L2 <= 1e-5 against the oracle's matmul_t of the oracle-dequantized weights
(the GEMV sums in a different order and factors the block scales).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from inferox_amd import _native, synth
from inferox_amd.gguf_writer import F16, F32, Q4_0, Q4_K, Q6_K, Q8_0, Q8_K
from oracle import binding as orc
from oracle import numpy_ref
from tests import fixtures_gguf as fx
from tests.conftest import rel_l2
from tests.gpu_util import Dev, Tensor

pytestmark = pytest.mark.gpu

BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292)}
ALL = [F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K]


def _same_bits(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    ok = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
    return bool(ok.all()), int((~ok).sum())


def _raw(t, n, rng, special=False):
    if t == F32:
        return (rng.standard_normal(n).astype(np.float32)).view(np.uint8)
    if t == F16:
        if special:
            return rng.integers(0, 65536, n, dtype=np.uint64).astype(np.uint16).view(np.uint8)
        return rng.standard_normal(n).astype("<f2").view(np.uint8)
    be, bb = BLOCK[t]
    nb = n // be
    raw = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    if not special:
        nd = 2 if t in (Q4_K, Q8_K) else 1
        raw[:, :2 * nd] = rng.uniform(1e-4, 1e-1, (nb, nd)).astype("<f2").view(np.uint8).reshape(nb, 2 * nd)
    return raw.reshape(-1)


def _gpu_dequant(t, raw, n, n_out=None):
    n_out = n if n_out is None else n_out
    d_in, d_out = Dev.of(raw), Dev(4 * max(n_out, 1))
    rc = _native.lib().ifx_dequantize_f32(t, n, d_in.ptr, raw.size, d_out.ptr, n_out, None)
    return rc, (d_out.get(np.float32, n_out) if rc == 0 else None)


@pytest.mark.parametrize("t", ALL)
def test_dequant_raw_bit_exact(t):
    rng = np.random.default_rng(100 + t)
    for special in (False, True):
        n = 256 * 4096
        raw = _raw(t, n, rng, special)
        rc, got = _gpu_dequant(t, raw, n)
        assert rc == 0
        orc_rc, ref = orc.dequantize(t, raw, n)
        assert orc_rc == 0
        ok, bad = _same_bits(got, ref)
        assert ok, f"{bad} elements differ"


@pytest.mark.parametrize("case", range(7))
def test_dequant_kats_on_gpu(case):
    t, raw, n, expected = fx.kat_blocks()[case]
    rc, got = _gpu_dequant(t, np.frombuffer(raw, np.uint8), n)
    assert rc == 0
    np.testing.assert_array_equal(got, expected)


def test_dequant_errors_on_gpu():
    assert _gpu_dequant(5, np.zeros(22, np.uint8), 32)[0] == 5       # Q5_0: UnknownTensorType
    assert _gpu_dequant(7, np.zeros(33, np.uint8), 32)[0] == 8       # byte length: UnexpectedEof
    assert _gpu_dequant(7, np.zeros(34, np.uint8), 32, 31)[0] == 10  # out length: InvalidTensorIndex
    assert _gpu_dequant(16, np.zeros(32, np.uint8), 32)[0] == 5      # I8: sizes fine, type refused


@pytest.mark.parametrize("t", ALL)
def test_device_layout_roundtrip_bit_exact(t):
    """Upload (with the SoA / qh re-order repack) then dequantize from the device layout."""
    rng = np.random.default_rng(200 + t)
    rows, cols = 96, 512
    raw = _raw(t, rows * cols, rng, special=True)
    w = Tensor(t, raw, rows, cols)
    out = Dev(4 * rows * cols)
    assert _native.lib().ifx_tensor_dequant(w.h, out.ptr, None) == 0
    got = out.get(np.float32, rows * cols)
    _, ref = orc.dequantize(t, raw, rows * cols)
    ok, bad = _same_bits(got, ref)
    assert ok, f"{bad} elements differ"
    dev_b, gguf_b = C.c_uint64(), C.c_uint64()
    _native.lib().ifx_tensor_bytes(w.h, C.byref(dev_b), C.byref(gguf_b))
    assert gguf_b.value == raw.size and dev_b.value == raw.size  # same bytes, different placement


def _gemv_check(t, rows, cols, rng, x_scale=1.0, tol=1e-5):
    raw = _raw(t, rows * cols, rng)
    w = Tensor(t, raw, rows, cols)
    x = (rng.standard_normal(cols) * x_scale).astype(np.float32)
    dx, dy = Dev.of(x), Dev(4 * rows)
    assert _native.lib().ifx_gemv(w.h, dx.ptr, dy.ptr, None) == 0
    y = dy.get(np.float32, rows)
    _, wf = orc.dequantize(t, raw, rows * cols)
    ref = orc.matmul_t(x, wf, 1, rows, cols)
    err = rel_l2(y, ref)
    # elementwise bound scaled by sum |w||x| of each row
    bound = np.abs(wf.reshape(rows, cols)).astype(np.float64) @ np.abs(x).astype(np.float64)
    assert err < tol, err
    assert np.all(np.abs(y.astype(np.float64) - ref) <= 1e-5 * bound + 1e-30)


@pytest.mark.parametrize("t", ALL)
@pytest.mark.parametrize("shape", [(64, 256), (1024, 4096), (36, 2048), (4, 14336), (1002, 4096), (6, 16384)])
def test_gemv_vs_oracle(t, shape):
    rng = np.random.default_rng(300 + t + shape[0])
    _gemv_check(t, shape[0], shape[1], rng)


@pytest.mark.parametrize("t", [Q8_0, Q4_0, F32, F16])
def test_gemv_small_k(t):
    """Row lengths below one 64-group sweep (the tiny model's 288 / 768)."""
    rng = np.random.default_rng(7)
    _gemv_check(t, 288, 288, rng)
    _gemv_check(t, 768, 288, rng)
    _gemv_check(t, 288, 768, rng)


@pytest.mark.parametrize("rows,cols,t", [(4096, 4096, Q4_K), (14336, 4096, Q4_K), (4096, 14336, Q4_K)])
def test_gemv_microbench_shapes(rows, cols, t):
    """The GEMV microbench shapes with the benchmark's block distributions."""
    raw = synth.random_blocks(t, rows * cols, seed=rows * 7 + cols)
    w = Tensor(t, raw, rows, cols)
    x = synth.normal_f32(cols, seed=11)
    dx, dy = Dev.of(x), Dev(4 * rows)
    assert _native.lib().ifx_gemv(w.h, dx.ptr, dy.ptr, None) == 0
    y = dy.get(np.float32, rows)
    wf = numpy_ref.dequant(t, raw).reshape(rows, cols)
    ref = wf.astype(np.float64) @ x.astype(np.float64)
    assert rel_l2(y, ref) < 1e-5


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
def test_gemv_half_tiles_in_last_round(t, monkeypatch):
    """5691 rows (356 tiles, the last with 11 rows) on 256 workgroups: one
    round of whole tiles, then 200 half tiles. Every row within the oracle's
    bound, and the same bits as the launch on whole tiles only
    (IFX_GEMV_HALVES=0): a half tile computes each row from the same unit
    data and x digits in the same order."""
    rows, cols = 16 * 356 - 5, 4096
    rng = np.random.default_rng(356 + t)
    raw = _raw(t, rows * cols, rng)
    w = Tensor(t, raw, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    dx, y1, y0 = Dev.of(x), Dev(4 * rows), Dev(4 * rows)
    assert _native.lib().ifx_gemv(w.h, dx.ptr, y1.ptr, None) == 0
    monkeypatch.setenv("IFX_GEMV_HALVES", "0")
    assert _native.lib().ifx_gemv(w.h, dx.ptr, y0.ptr, None) == 0
    got, whole = y1.get(np.float32, rows), y0.get(np.float32, rows)
    assert np.array_equal(got.view(np.uint32), whole.view(np.uint32))
    _, wf = orc.dequantize(t, raw, rows * cols)
    ref = orc.matmul_t(x, wf, 1, rows, cols)
    bound = np.abs(wf.reshape(rows, cols)).astype(np.float64) @ np.abs(x).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - ref) <= 1e-5 * bound + 1e-30)


def test_gemv_lm_head_q6k_rows():
    """[128256 x 4096] Q6_K: all rows computed, a seeded sample of 8192 rows checked."""
    rows, cols = 128256, 4096
    raw = synth.random_blocks(Q6_K, rows * cols, seed=77)
    w = Tensor(Q6_K, raw, rows, cols)
    x = synth.normal_f32(cols, seed=12)
    dx, dy = Dev.of(x), Dev(4 * rows)
    assert _native.lib().ifx_gemv(w.h, dx.ptr, dy.ptr, None) == 0
    y = dy.get(np.float32, rows)
    sel = np.sort(np.random.default_rng(5).choice(rows, 8192, replace=False))
    blk = raw.reshape(rows, cols // 256 * 210)[sel].reshape(-1)
    wf = numpy_ref.dequant(Q6_K, blk).reshape(len(sel), cols)
    ref = wf.astype(np.float64) @ x.astype(np.float64)
    assert rel_l2(y[sel], ref) < 1e-5
    assert np.isfinite(y).all()


def test_ops_vs_oracle():
    rng = np.random.default_rng(9)
    L = _native.lib()
    # rms_norm_rows
    x = (rng.standard_normal(4 * 4096) * 50).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(4096)).astype(np.float32)
    dx, dw = Dev.of(x), Dev.of(w)
    assert L.ifx_ops_rms_norm_rows(dx.ptr, dw.ptr, 4096, 4, 1e-5, None) == 0
    assert rel_l2(dx.get(np.float32, x.size), orc.rms_norm_rows(x, w, 1e-5)) < 1e-6
    # softmax_rows
    s = (rng.standard_normal(3 * 1000) * 8).astype(np.float32)
    ds = Dev.of(s)
    assert L.ifx_ops_softmax_rows(ds.ptr, 3, 1000, None) == 0
    assert rel_l2(ds.get(np.float32, s.size), orc.softmax_rows(s, 3, 1000)) < 1e-5
    # swiglu and add
    g = (rng.standard_normal(5000) * 20).astype(np.float32)
    u = rng.standard_normal(5000).astype(np.float32)
    dg, du, do = Dev.of(g), Dev.of(u), Dev(4 * 5000)
    assert L.ifx_ops_swiglu(dg.ptr, du.ptr, do.ptr, 5000, None) == 0
    assert rel_l2(do.get(np.float32, 5000), orc.swiglu(g, u)) < 1e-6
    assert L.ifx_ops_add_in_place(dg.ptr, du.ptr, 5000, None) == 0
    np.testing.assert_array_equal(dg.get(np.float32, 5000), orc.add_in_place(g, u))
    # rope at positions 3..5 and the identity at 0
    r = rng.standard_normal(3 * 8 * 128).astype(np.float32)
    dr = Dev.of(r)
    assert L.ifx_ops_rope(dr.ptr, 3, 8, 128, 128, 500000.0, 3, None) == 0
    assert rel_l2(dr.get(np.float32, r.size), orc.rope(r, 3, 8, 128, 128, 500000.0, 3)) < 1e-6
    dr0 = Dev.of(r[: 8 * 128])
    assert L.ifx_ops_rope(dr0.ptr, 1, 8, 128, 128, 500000.0, 0, None) == 0
    np.testing.assert_array_equal(dr0.get(np.float32, 8 * 128), r[: 8 * 128])
    # matmul_t f32 (the KATs plus a random case)
    a, b = np.array([1, 2, 3, 4], np.float32), np.array([0, 1, 2, 3], np.float32)
    da, db, dc = Dev.of(a), Dev.of(b), Dev(16)
    assert L.ifx_ops_matmul_t(da.ptr, db.ptr, dc.ptr, 2, 2, 2, None) == 0
    assert dc.get(np.float32, 4).tolist() == [2.0, 8.0, 4.0, 18.0]
    a = rng.standard_normal(3 * 300).astype(np.float32)
    b = rng.standard_normal(70 * 300).astype(np.float32)
    da, db, dc = Dev.of(a), Dev.of(b), Dev(4 * 210)
    assert L.ifx_ops_matmul_t(da.ptr, db.ptr, dc.ptr, 3, 70, 300, None) == 0
    assert rel_l2(dc.get(np.float32, 210), orc.matmul_t(a, b, 3, 70, 300)) < 1e-6


def test_argmax_tie_rule_and_nan():
    L = _native.lib()
    out, st = Dev(4), Dev(4)

    def run(x):
        dx = Dev.of(np.asarray(x, np.float32))
        assert L.ifx_ops_argmax(dx.ptr, len(x), out.ptr, st.ptr, None) == 0
        return int(out.get(np.uint32, 1)[0]), int(st.get(np.int32, 1)[0])

    assert run([0.0] * 128256) == (128255, 0)
    assert run([1.0, 5.0, 5.0, 2.0]) == (2, 0)
    assert run([-0.0, 0.0]) == (1, 0)
    assert run([-3.0, -1.0, -2.0]) == (1, 0)
    assert run([1.0, float("nan"), 2.0])[1] == 24
    rng = np.random.default_rng(1)
    x = rng.standard_normal(128256).astype(np.float32)
    assert run(x) == (orc.argmax(x)[1], 0)


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K, F32])
def test_embedding_rows_bit_exact(t):
    rng = np.random.default_rng(40 + t)
    rows, cols = 300, 512
    raw = _raw(t, rows * cols, rng)
    w = Tensor(t, raw, rows, cols)
    ids = np.array([0, 299, 17, 17, 150], np.uint32)
    did, dout = Dev.of(ids), Dev(4 * ids.size * cols)
    assert _native.lib().ifx_ops_embedding_lookup(w.h, did.ptr, ids.size, dout.ptr, None) == 0
    got = dout.get(np.float32, ids.size * cols).reshape(ids.size, cols)
    _, full = orc.dequantize(t, raw, rows * cols)
    np.testing.assert_array_equal(got, full.reshape(rows, cols)[ids])


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
def test_gemv_wide_dynamic_range_within_groups(t):
    """The int8-MFMA GEMV stages x per 32-element group in fixed point scaled
    to the group's largest magnitude (22 bits): an element 2^k below it keeps
    22 - k bits.  Groups spanning 2^20 (one element of 1, the others ~2^-20)
    still meet the per-row bound 1e-5 * sum |w||x|: what the small elements
    lose is below 2^-22 of the group's largest term."""
    rng = np.random.default_rng(2 ** 20 + t)
    rows, cols = 512, 4096
    raw = _raw(t, rows * cols, rng)
    w = Tensor(t, raw, rows, cols)
    x = (rng.standard_normal(cols) * 2.0 ** -20).astype(np.float32)
    x[::32] = rng.choice([-1.0, 1.0], cols // 32).astype(np.float32)  # one large element per group
    x[5::64] *= 2.0 ** 19                                            # intermediate magnitudes too
    dx, dy = Dev.of(x), Dev(4 * rows)
    assert _native.lib().ifx_gemv(w.h, dx.ptr, dy.ptr, None) == 0
    y = dy.get(np.float32, rows)
    _, wf = orc.dequantize(t, raw, rows * cols)
    ref = orc.matmul_t(x, wf, 1, rows, cols)
    bound = np.abs(wf.reshape(rows, cols)).astype(np.float64) @ np.abs(x).astype(np.float64)
    assert np.all(np.abs(y.astype(np.float64) - ref) <= 1e-5 * bound + 1e-30)
    assert rel_l2(y, ref) < 1e-5
