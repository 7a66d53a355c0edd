"""The ggml K-quant layout mode (IFX_OPEN_GGML_KQUANTS) on the GPU.

Bars: device dequantization of ggml-layout Q4_K / Q6_K blocks (Q6_K scales of
both signs) bit-exact to the numpy restatement of ggml's dequantizers; the
GEMV and the prefill GEMM within the same bounds as the reference-layout
kernels; a small Q4_K/Q6_K model in ggml's layout against the CPU oracle
running the same weights as F32: logits within 1e-3 relative L2 per decode
step and per prefill row, greedy tokens equal.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from inferox_amd import _native, synth
from oracle import binding as orc
from oracle import numpy_ref as nr
from tests.conftest import rel_l2
from tests.ggml_layout import q4k_ref_to_ggml, q6k_ref_to_ggml, write_ggml_pair
from tests.gpu_util import Dev, GpuModel

pytestmark = pytest.mark.gpu

Q4_K, Q6_K, Q8_K = 12, 14, 15
GGML = 1  # IFX_OPEN_GGML_KQUANTS


class GgmlTensor:
    def __init__(self, t, raw, rows, cols, flags=GGML):
        raw = np.ascontiguousarray(raw, np.uint8)
        self.h = C.c_void_p()
        self.rc = _native.lib().ifx_tensor_upload_ex(t, raw.ctypes.data_as(C.c_void_p), raw.size, rows, cols,
                                                     flags, C.byref(self.h))

    def __del__(self):
        if self.h:
            _native.lib().ifx_tensor_free(self.h)


def ggml_blocks(t, rows, cols, seed):
    ref = synth.random_blocks(t, rows * cols, seed=seed)
    if t == Q4_K:
        g = q4k_ref_to_ggml(ref)
        return g, nr.dequant_q4_k_ggml(g)
    rng = np.random.default_rng(seed)
    sc = rng.integers(-128, 128, size=(ref.size // 210, 16))
    g = q6k_ref_to_ggml(ref, sc)
    return g, nr.dequant_q6_k_ggml(g)


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("rows,cols", [(16, 256), (37, 512), (300, 1024)])
def test_ggml_dequant_bit_exact(t, rows, cols):
    g, ref = ggml_blocks(t, rows, cols, seed=rows + cols + t)
    w = GgmlTensor(t, g, rows, cols)
    assert w.rc == 0
    out = Dev(4 * rows * cols)
    assert _native.lib().ifx_tensor_dequant(w.h, out.ptr, None) == 0
    got = out.get(np.float32, rows * cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("rows,cols", [(64, 256), (1024, 4096), (36, 2048)])
def test_ggml_gemv(t, rows, cols):
    g, wf = ggml_blocks(t, rows, cols, seed=rows * 7 + cols + t)
    w = GgmlTensor(t, g, rows, cols)
    assert w.rc == 0
    x = np.random.default_rng(rows).standard_normal(cols).astype(np.float32)
    dx, dy = Dev.of(x), Dev(4 * rows)
    assert _native.lib().ifx_gemv(w.h, dx.ptr, dy.ptr, None) == 0
    y = dy.get(np.float32, rows).astype(np.float64)
    W = wf.reshape(rows, cols).astype(np.float64)
    ref = W @ x.astype(np.float64)
    bound = np.abs(W) @ np.abs(x).astype(np.float64)
    assert np.all(np.abs(y - ref) <= 1e-5 * bound + 1e-30)


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("m,rows,cols", [(2, 16, 256), (130, 300, 512), (64, 129, 4096)])
def test_ggml_gemm(t, m, rows, cols):
    g, wf = ggml_blocks(t, rows, cols, seed=m + rows + cols + t)
    w = GgmlTensor(t, g, rows, cols)
    assert w.rc == 0
    rng = np.random.default_rng(m)
    a = (rng.standard_normal((m, cols)) * (10.0 ** rng.uniform(-3, 3, size=(m, 1)))).astype(np.float32)
    da, dc = Dev.of(a), Dev(4 * m * rows)
    assert _native.lib().ifx_matmul_qt(da.ptr, m, w.h, dc.ptr, None) == 0
    c = dc.get(np.float32, m * rows).reshape(m, rows).astype(np.float64)
    W = wf.reshape(rows, cols).astype(np.float64)
    ref = a.astype(np.float64) @ W.T
    bound = np.abs(a).astype(np.float64) @ np.abs(W).T
    assert np.all(np.abs(c - ref) <= 1e-5 * bound + 1e-30)


def test_ggml_flags_and_q8k_refused():
    raw = np.zeros(292 * 4, np.uint8)  # four all-zero Q8_K blocks
    assert GgmlTensor(Q8_K, raw, 4, 256).rc == 5          # IFX_E_UNKNOWN_TENSOR_TYPE
    assert GgmlTensor(Q8_K, raw, 4, 256, flags=0).rc == 0
    assert GgmlTensor(Q8_K, raw, 4, 256, flags=2).rc == 20  # unknown flag


def test_ggml_model_against_f32_oracle(tmp_path):
    pg, pf = str(tmp_path / "small_ggml.gguf"), str(tmp_path / "small_f32.gguf")
    write_ggml_pair(pg, pf)
    h = C.c_void_p()
    assert _native.lib().ifx_model_open_ex(pg.encode(), GGML, C.byref(h)) == 0
    g = GpuModel.__new__(GpuModel)
    g.h = h
    g.cfg = _native.IfxConfig()
    assert _native.lib().ifx_model_config(h, C.byref(g.cfg)) == 0
    g.vocab = g.cfg.vocab_size
    o = orc.Model(pf)
    assert g.batched_prefill()
    s, kv = g.session(128), o.kv(128)
    ids = synth.token_ids(64, g.vocab, seed=9)
    rc, lg = s.prefill(ids)
    orc_rc, ref = o.prefill(kv, ids)
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg[t], ref[t]) for t in range(len(ids))) < 1e-3
    tok = orc.argmax(ref[-1])[1]
    for step in range(16):
        rc, lg = s.decode_step(tok)
        _, r = o.decode_step(kv, tok)
        assert rc == 0 and rel_l2(lg, r) < 1e-3, step
        tok = orc.argmax(r)[1]
        assert len(lg) - 1 - int(np.argmax(lg[::-1])) == tok
    s.close()
    # the same file read in the reference's layout is a different model
    h2 = C.c_void_p()
    assert _native.lib().ifx_model_open(pg.encode(), C.byref(h2)) == 0
    g2 = GpuModel.__new__(GpuModel)
    g2.h, g2.cfg, g2.vocab = h2, g.cfg, g.vocab
    s2 = g2.session(128)
    rc, lg2 = s2.prefill(ids)
    assert rc == 0 and not rel_l2(lg2[-1], ref[-1]) < 1e-2  # (garbage scales may give NaN logits)
    s2.close()
    g2.close()
    g.close()
    o.close()
