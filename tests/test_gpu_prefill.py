"""Batched prefill on the GPU: the dequant-to-LDS fp16-MFMA GEMM (the weights'
integer parts as exact fp16 values with the block scales applied in f32, the
activations as fp16 hi/lo pairs) and the batched causal attention, against the
oracle.  The Q6_K cases carry u8 scales up to 255, so they run the split
weight plane; the Q4_K cases run the min-term MFMA.

Bars: the GEMM within 1e-5 relative L2 of a float64 product of the oracle's
dequantized weights, and every element within 1e-5 * sum_k |a||w| of it; model
outputs within the token loop's 1e-3 relative L2 per row, greedy tokens equal.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from inferox_amd import _native, synth
from oracle import binding as orc
from oracle import numpy_ref
from tests.conftest import rel_l2
from tests.gpu_util import Dev, GpuModel, Tensor

pytestmark = pytest.mark.gpu

TOL = 1e-3
Q4_0, Q8_0, Q4_K, Q6_K = 2, 7, 12, 14


def _rows(m, cols, rng):
    """Rows of very different magnitudes (1e-3 .. 1e6), one all-zero row."""
    a = rng.standard_normal((m, cols)) * (10.0 ** rng.uniform(-3, 6, size=(m, 1)))
    a[m // 2] = 0.0
    return a.astype(np.float32)


def _gemm_check(t, m, rows, cols, seed):
    rng = np.random.default_rng(seed)
    raw = synth.random_blocks(t, rows * cols, seed=seed)
    w = Tensor(t, raw, rows, cols)
    a = _rows(m, cols, rng)
    da, dc = Dev.of(a), Dev(4 * m * rows)
    assert _native.lib().ifx_matmul_qt(da.ptr, m, w.h, dc.ptr, None) == 0
    c = dc.get(np.float32, m * rows).reshape(m, rows).astype(np.float64)
    wf = numpy_ref.dequant(t, raw).reshape(rows, cols).astype(np.float64)
    ref = a.astype(np.float64) @ wf.T
    bound = np.abs(a).astype(np.float64) @ np.abs(wf).T
    assert np.all(np.abs(c - ref) <= 1e-5 * bound + 1e-30), np.max(np.abs(c - ref) / (bound + 1e-30))
    nz = np.linalg.norm(ref, axis=1) > 0
    assert max(rel_l2(c[i], ref[i]) for i in np.flatnonzero(nz)) < 1e-5
    assert np.all(c[~nz] == 0)


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
@pytest.mark.parametrize("m,rows,cols", [(2, 16, 256), (130, 300, 512), (257, 1024, 4096), (64, 129, 14336)])
def test_gemm_kquant(t, m, rows, cols):
    _gemm_check(t, m, rows, cols, seed=rows + cols + m + t)


@pytest.mark.parametrize("t", [Q8_0, Q4_0])
@pytest.mark.parametrize("m,rows,cols", [(3, 288, 288), (100, 768, 288), (129, 288, 768)])
def test_gemm_q8_q4(t, m, rows, cols):
    _gemm_check(t, m, rows, cols, seed=rows * 3 + cols + m + t)


@pytest.fixture(scope="module")
def tiny(tiny_path):
    g = GpuModel(tiny_path)
    o = orc.Model(tiny_path)
    assert g.batched_prefill()
    yield g, o
    g.close()
    o.close()


def test_tiny_batched_prefill_logits_and_kv(tiny, tiny_prompt):
    """Model::prefill as whole-chunk GEMMs: every row's logits, then a second
    chunk (positions restart, attention inside the chunk: Q2), the KV rows."""
    g, o = tiny
    s, kv = g.session(256), o.kv(256)
    s.set_prefill_batch(1)
    ids = synth.token_ids(100, synth.TINY.vocab, seed=77)
    rc, lg = s.prefill(ids)
    orc_rc, ref = o.prefill(kv, ids)
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg[t], ref[t]) for t in range(len(ids))) < TOL
    rc, lg2 = s.prefill(tiny_prompt)
    orc_rc, ref2 = o.prefill(kv, tiny_prompt)
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg2[t], ref2[t]) for t in range(len(tiny_prompt))) < TOL
    assert len(s) == 116
    k, v = s.kv_export(116)
    kr, vr = kv.export(116)
    assert rel_l2(k, kr) < 1e-4 and rel_l2(v, vr) < 1e-4
    # decode continues from the batched state: same greedy picks as the oracle
    tok = orc.argmax(ref2[-1])[1]
    for step in range(8):
        rc, lg = s.decode_step(tok)
        _, r = o.decode_step(kv, tok)
        assert rc == 0 and rel_l2(lg, r) < TOL, step
        tok = orc.argmax(r)[1]
        assert len(lg) - 1 - int(np.argmax(lg[::-1])) == tok


def test_tiny_batched_generate(tiny, tiny_prompt):
    """Model::generate with the prompt through the batched path."""
    g, o = tiny
    s, kv = g.session(256), o.kv(256)
    s.set_prefill_batch(1)
    rc, toks = s.generate(tiny_prompt, 128)
    orc_rc, ref = o.generate(kv, tiny_prompt, 128)
    assert rc == 0 and orc_rc == 0
    assert toks.tolist() == ref.tolist()
    assert len(s) == 16 + 128


def test_tiny_batched_equals_token_path(tiny):
    """The two GPU prefill paths agree (GEMM + batched attention vs the decode
    step replayed per id)."""
    g, _ = tiny
    ids = synth.token_ids(70, synth.TINY.vocab, seed=5)
    a, b = g.session(128), g.session(128)
    a.set_prefill_batch(1)
    b.set_prefill_batch(0)
    rca, la = a.prefill(ids)
    rcb, lb = b.prefill(ids)
    assert rca == 0 and rcb == 0
    assert max(rel_l2(la[t], lb[t]) for t in range(len(ids))) < TOL
    ka, va = a.kv_export(70)
    kb, vb = b.kv_export(70)
    assert rel_l2(ka, kb) < 1e-4 and rel_l2(va, vb) < 1e-4


def test_tiny_batched_rope_absolute(tiny):
    g, o = tiny
    s, kv = g.session(256), o.kv(256)
    s.set_prefill_batch(1)
    s.set_rope_mode(1)
    ids = synth.token_ids(40, synth.TINY.vocab, seed=8)
    for chunk in (ids[:24], ids[24:]):
        rc, lg = s.prefill(chunk)
        orc_rc, ref = o.prefill(kv, chunk, rope_mode=orc.ROPE_ABSOLUTE)
        assert rc == 0 and orc_rc == 0
        assert max(rel_l2(lg[t], ref[t]) for t in range(len(chunk))) < TOL


def test_tiny_batched_forward(tiny):
    """Model::forward (non-causal, no cache) through the batched path (>= 64 ids)."""
    g, o = tiny
    ids = synth.token_ids(80, synth.TINY.vocab, seed=9)
    rc, lg = g.forward(ids)
    orc_rc, ref = o.forward(ids)
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg[t], ref[t]) for t in range(len(ids))) < TOL


@pytest.mark.parametrize("n", [8, 80])
def test_tiny_forward_last_token_logits(tiny, n):
    """Model::forward_last_token_logits (src/model/forward.rs:484-489): the
    forward's last row, with the output head run for that row alone (8 ids:
    layer-major token replays; 80: the batched path), against the oracle's
    forward and against ifx_forward's last row; an empty prompt and an id
    past the vocabulary are refused."""
    g, o = tiny
    ids = synth.token_ids(n, synth.TINY.vocab, seed=40 + n)
    rc, last = g.forward_last_token_logits(ids)
    orc_rc, ref = o.forward(ids)
    rc_all, lg = g.forward(ids)
    assert rc == 0 and orc_rc == 0 and rc_all == 0
    assert rel_l2(last, ref[-1]) < TOL
    assert rel_l2(last, lg[-1]) < 1e-5
    assert g.forward_last_token_logits(np.zeros(0, np.uint32))[0] == 20
    assert g.forward_last_token_logits(np.array([1, synth.TINY.vocab], np.uint32))[0] == 10


def test_8b_shape_batched_prefill(tmpdir_session):
    """Full-width Llama-3-8B shape, two layers: a 96-id chunk through the
    Q4_K/Q6_K GEMMs (default threshold), logits of every row and the KV rows."""
    spec = synth.reduced(synth.LLAMA3_8B, n_layers=2, ctx=512)
    p = str(tmpdir_session / "l8b_2l_prefill.gguf")
    synth.write_llama(p, spec, seed=8)
    g, o = GpuModel(p), orc.Model(p)
    assert g.batched_prefill()
    s, kv = g.session(256), o.kv(256)
    ids = synth.token_ids(96, spec.vocab, seed=31)
    rc, lg = s.prefill(ids)
    orc_rc, ref = o.prefill(kv, ids)
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg[t], ref[t]) for t in range(len(ids))) < TOL
    k, v = s.kv_export(96)
    kr, vr = kv.export(96)
    assert rel_l2(k, kr) < 1e-4 and rel_l2(v, vr) < 1e-4
    last = C.c_uint32()
    assert _native.lib().ifx_session_last_token(s.h, C.byref(last)) == 0
    assert last.value == orc.argmax(ref[-1])[1]
    g.close()
