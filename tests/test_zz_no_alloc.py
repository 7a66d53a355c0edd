"""ifx_matmul_qt_noalloc (no reference counterpart: for callers that cannot
allocate device memory) against ifx_matmul_qt, through the C ABI.

Two calls in a row on the same GPU, the second with a smaller input, each
compared with ifx_matmul_qt on the same operands: every element within
1e-5 * sum_k |a||w| of it (the two may split K differently, so the partial
sums can be added in another order; with the same split they are equal) and
rows at 1e-5 relative L2; a shape past the fixed scratch is refused with
IFX_E_INVALID_ARG; one-row calls, and several rows against a matrix the GEMM
does not take (F32, F16, Q8_K), take the GEMV row by row as ifx_matmul_qt
does, with the same bits.
"""
from __future__ import annotations

import numpy as np
import pytest

from inferox_amd import _native, synth
from tests.conftest import rel_l2
from tests.gpu_util import Dev, Tensor

pytestmark = pytest.mark.gpu

Q4_K, Q6_K = 12, 14


def _fn():
    return _native.lib().ifx_matmul_qt_noalloc


def _both(t, m, rows, cols, seed):
    rng = np.random.default_rng(seed)
    raw = synth.random_blocks(t, rows * cols, seed=seed)
    w = Tensor(t, raw, rows, cols)
    a = (rng.standard_normal((m, cols)) * (10.0 ** rng.uniform(-2, 3, size=(m, 1)))).astype(np.float32)
    da = Dev.of(a)
    d_ref, d_na = Dev(4 * m * rows), Dev(4 * m * rows)
    assert _native.lib().ifx_matmul_qt(da.ptr, m, w.h, d_ref.ptr, None) == 0
    assert _fn()(da.ptr, m, w.h, d_na.ptr, None) == 0
    ref = d_ref.get(np.float32, m * rows).reshape(m, rows).astype(np.float64)
    got = d_na.get(np.float32, m * rows).reshape(m, rows).astype(np.float64)
    return a, raw, ref, got


def _check(t, m, rows, cols, seed):
    from oracle import numpy_ref
    a, raw, ref, got = _both(t, m, rows, cols, seed)
    wf = numpy_ref.dequant(t, raw).reshape(rows, cols).astype(np.float64)
    bound = np.abs(a).astype(np.float64) @ np.abs(wf).T
    assert np.all(np.abs(got - ref) <= 1e-5 * bound + 1e-30)
    assert max(rel_l2(got[i], ref[i]) for i in range(m)) < 1e-5
    return ref, got


def test_noalloc_two_calls_second_smaller():
    # first call: 300 rows of 4096 against 1024 Q4_K rows (12 tiles: both split K, differently)
    _check(Q4_K, 300, 1024, 4096, seed=1)
    # second, smaller call on the same scratch: 40 rows against a Q6_K matrix
    _check(Q6_K, 40, 512, 4096, seed=2)


def test_noalloc_same_result_without_split():
    """256 output tiles (1024 x 8192): neither entry point splits K, so the
    same kernels on the same operands give the same bits."""
    ref, got = _check(Q4_K, 1024, 8192, 4096, seed=3)
    np.testing.assert_array_equal(got, ref)


def test_noalloc_limits_and_gemv_rows():
    rng = np.random.default_rng(4)
    raw = synth.random_blocks(Q4_K, 256 * 4096, seed=4)
    w = Tensor(Q4_K, raw, 256, 4096)
    # past the scratch: 1025 rows of 4096 (> 2^22 elements)
    big = Dev(4 * 1025 * 4096)
    out = Dev(4 * 1025 * 256)
    assert _fn()(big.ptr, 1025, w.h, out.ptr, None) == 20
    # one row: the GEMV, equal to ifx_matmul_qt's one-row result
    x = rng.standard_normal((1, 4096)).astype(np.float32)
    dx, y1, y2 = Dev.of(x), Dev(4 * 256), Dev(4 * 256)
    assert _native.lib().ifx_matmul_qt(dx.ptr, 1, w.h, y1.ptr, None) == 0
    assert _fn()(dx.ptr, 1, w.h, y2.ptr, None) == 0
    np.testing.assert_array_equal(y1.get(np.float32, 256), y2.get(np.float32, 256))


@pytest.mark.parametrize("t", [0, 1, 15])  # F32, F16, Q8_K: no GEMM operand form
def test_noalloc_gemv_rows_for_other_types(t):
    """m = 3 against a matrix the GEMM does not take: the row-by-row GEMV of
    both entry points, bit for bit."""
    rows, cols, m = 160, 1024, 3
    rng = np.random.default_rng(40 + t)
    if t == 0:
        raw = rng.standard_normal(rows * cols).astype(np.float32).view(np.uint8)
    elif t == 1:
        raw = (0.05 * rng.standard_normal(rows * cols)).astype("<f2").view(np.uint8)
    else:
        nb = rows * cols // 256
        raw = rng.integers(0, 256, size=(nb, 292), dtype=np.uint8)
        raw[:, :4] = rng.uniform(1e-3, 1e-2, (nb, 2)).astype("<f2").view(np.uint8).reshape(nb, 4)
        raw = raw.reshape(-1)
    w = Tensor(t, raw, rows, cols)
    a = rng.standard_normal((m, cols)).astype(np.float32)
    da, y1, y2 = Dev.of(a), Dev(4 * m * rows), Dev(4 * m * rows)
    assert _native.lib().ifx_matmul_qt(da.ptr, m, w.h, y1.ptr, None) == 0
    assert _fn()(da.ptr, m, w.h, y2.ptr, None) == 0
    ref, got = y1.get(np.float32, m * rows), y2.get(np.float32, m * rows)
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))
    # and the rows are the product, to the GEMV bar
    from oracle import numpy_ref
    wf = numpy_ref.dequant(t, raw).reshape(rows, cols).astype(np.float64)
    want = a.astype(np.float64) @ wf.T
    bound = np.abs(a).astype(np.float64) @ np.abs(wf).T
    assert np.all(np.abs(got.reshape(m, rows) - want) <= 1e-5 * bound)
