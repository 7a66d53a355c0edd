"""Sessions with the f16 KV cache (ifx_session_create_kv(..., IFX_KV_F16)).

The mode has no counterpart in the reference: keys (after RoPE) and values
are rounded to binary16 as they are stored, before any attention reads them.
Its oracle is the reference algorithm with the same rounding (the oracle's
f16-KV mode, orc_kv_set_f16; its rounding is pinned against numpy's on the
CPU).  Rounding to binary16 is discontinuous: where the device's f32 value of
a key or value and the oracle's lie on either side of a rounding boundary,
the stored rows differ by a whole binary16 step (2^-11 relative) instead of
an f32 one, and the model carries that like any other change of the cache.
Hence TOL16 sits above the f32 mode's 1e-3 (measured: 1.3e-3 worst over 64
tiny-model steps).

Bars: logits within TOL16 relative L2 of the f16-mode oracle per step, greedy
tokens identical to its picks; exported rows equal numpy's rounding of what was
imported, bit for bit.  Against the f32 oracle (the cost of the mode, reported
apart from the f32 parity mode: 2e-2 on the tiny model) the logits stay within
TOL16_VS_F32.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from inferox_amd import _native, synth
from oracle import binding as orc
from tests.conftest import rel_l2
from tests.gpu_util import GpuModel

pytestmark = pytest.mark.gpu

TOL16 = 4e-3          # vs the f16-mode oracle
TOL16_VS_F32 = 5e-2   # vs the f32 oracle


def f16(x):
    with np.errstate(over="ignore"):
        return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def last_argmax(lg):
    return len(lg) - 1 - int(np.argmax(lg[::-1]))


@pytest.fixture(scope="module")
def tiny(tiny_path):
    g = GpuModel(tiny_path)
    o = orc.Model(tiny_path)
    yield g, o
    g.close()
    o.close()


def test_kv_f16_import_export_rounding(tiny):
    """Import rounds to nearest even (ties, subnormals, overflow to inf),
    export widens exactly."""
    g, o = tiny
    c = o.cfg
    L = 37
    kvd = c.n_kv_heads * c.head_dim
    n = c.n_layers * L * kvd
    rng = np.random.default_rng(5)
    k = (rng.standard_normal(n) * 10.0 ** rng.uniform(-9, 5, n)).astype(np.float32)
    v = synth.normal_f32(n, seed=6)
    # ties between neighbouring halves (1 + (2j+1) 2^-11), values near the top
    # of the range, the smallest subnormals and their halves
    special = np.array([1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 65504.0, 65519.0, 65520.0, 1e6, -7e4,
                        2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -15 + 2.0 ** -26, 0.0, -0.0],
                       np.float32)
    k[:special.size] = special
    s = g.session(64, kv_f16=True)
    assert s.kv_import(k, v, L) == 0
    ke, ve = s.kv_export(L)
    np.testing.assert_array_equal(ke, f16(k))
    np.testing.assert_array_equal(ve, f16(v))
    assert np.isinf(ke[4]) and np.isinf(ke[5]) and ke[3] == 65504.0
    assert np.signbit(ke[13])


def test_kv_f16_decode_tiny(tiny, tiny_prompt):
    """The CLI path (every prompt token through decode_step, then greedy
    steps) on an f16 cache, against the rounded-cache oracle at every step."""
    g, o = tiny
    s, kv, kv32 = g.session(256, kv_f16=True), o.kv(256, f16=True), o.kv(256)
    worst, worst32, tok = 0.0, 0.0, None
    for i in range(16 + 48):
        t = int(tiny_prompt[i]) if i < 16 else tok
        rc, lg = s.decode_step(t)
        orc_rc, ref = o.decode_step(kv, t)
        _, ref32 = o.decode_step(kv32, t)
        assert rc == 0 and orc_rc == 0
        worst = max(worst, rel_l2(lg, ref))
        worst32 = max(worst32, rel_l2(lg, ref32))
        tok = orc.argmax(ref)[1]
        assert last_argmax(lg) == tok, f"step {i}: greedy pick differs"
    print(f"f16 KV decode: rel L2 {worst:.2e} vs the f16-mode oracle, {worst32:.2e} vs the f32 oracle")
    assert worst < TOL16, worst
    assert worst32 < TOL16_VS_F32, worst32
    # the stored rows are the rounded rows
    k, v = s.kv_export(64)
    kr, vr = kv.export(64)
    assert rel_l2(k, kr) < 1e-3 and rel_l2(v, vr) < 1e-3  # binary16 steps where roundings part
    np.testing.assert_array_equal(k, f16(k))


def test_kv_f16_generate_tiny(tiny, tiny_prompt):
    """ifx_generate (prompt replay, then the captured greedy step) on an f16
    cache: the f16-mode oracle's generate, 96 tokens."""
    g, o = tiny
    s, kv = g.session(256, kv_f16=True), o.kv(256, f16=True)
    rc, toks = s.generate(tiny_prompt, 96)
    orc_rc, ref = o.generate(kv, tiny_prompt, 96)
    assert rc == 0 and orc_rc == 0
    assert toks.tolist() == ref.tolist()


def test_kv_f16_batched_prefill_tiny(tiny, tiny_prompt):
    """Whole-chunk prefill (GEMMs + batched attention reading the f16 rows),
    a second chunk, then decode."""
    g, o = tiny
    assert g.batched_prefill()
    s, kv = g.session(256, kv_f16=True), o.kv(256, f16=True)
    s.set_prefill_batch(1)
    ids = synth.token_ids(100, synth.TINY.vocab, seed=77)
    rc, lg = s.prefill(ids)
    orc_rc, ref = o.prefill(kv, ids)
    assert rc == 0 and orc_rc == 0
    w1 = max(rel_l2(lg[t], ref[t]) for t in range(len(ids)))
    rc, lg2 = s.prefill(tiny_prompt)
    orc_rc, ref2 = o.prefill(kv, tiny_prompt)
    assert rc == 0 and orc_rc == 0
    w2 = max(rel_l2(lg2[t], ref2[t]) for t in range(len(tiny_prompt)))
    print(f"f16 KV batched prefill: rel L2 {w1:.2e}, second chunk {w2:.2e}")
    assert w1 < TOL16 and w2 < TOL16, (w1, w2)
    k, v = s.kv_export(116)
    kr, vr = kv.export(116)
    assert rel_l2(k, kr) < 1e-3 and rel_l2(v, vr) < 1e-3  # binary16 steps where roundings part
    tok = orc.argmax(ref2[-1])[1]
    for step in range(8):
        rc, lg = s.decode_step(tok)
        _, r = o.decode_step(kv, tok)
        assert rc == 0 and rel_l2(lg, r) < TOL16, step
        tok = orc.argmax(r)[1]
        assert last_argmax(lg) == tok


@pytest.mark.parametrize("shape,seed,L", [("8b", 8, 200), ("70b", 70, 300)])
def test_kv_f16_wide_shapes(tmpdir_session, shape, seed, L):
    """Llama-3-8B and -70B widths, two layers: decode from an imported
    context (group 4 and group 8 attention over f16 rows), then a batched chunk."""
    base = synth.LLAMA3_8B if shape == "8b" else synth.LLAMA3_70B
    spec = synth.reduced(base, n_layers=2, ctx=512)
    p = str(tmpdir_session / f"l{shape}_2l_kv16.gguf")
    synth.write_llama(p, spec, seed=seed)
    g, o = GpuModel(p), orc.Model(p)
    c = o.cfg
    kvd = c.n_kv_heads * c.head_dim
    k = synth.normal_f32(c.n_layers * L * kvd, seed=seed + 1)
    v = synth.normal_f32(c.n_layers * L * kvd, seed=seed + 2)
    s, kv = g.session(512, kv_f16=True), o.kv(512, f16=True)
    assert s.kv_import(k, v, L) == 0 and kv.import_(f16(k), f16(v), L) == 0
    tok = 1000 + seed
    for step in range(3):
        rc, lg = s.decode_step(tok)
        _, ref = o.decode_step(kv, tok)
        assert rc == 0
        assert rel_l2(lg, ref) < TOL16, step
        tok = orc.argmax(ref)[1]
        assert lg[tok] == lg.max()
    ids = synth.token_ids(64, spec.vocab, seed=seed + 3)
    rc, lg = s.prefill(ids)
    orc_rc, ref = o.prefill(kv, ids)
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg[t], ref[t]) for t in range(len(ids))) < TOL16
    last = C.c_uint32()
    assert _native.lib().ifx_session_last_token(s.h, C.byref(last)) == 0
    assert last.value == orc.argmax(ref[-1])[1]
    g.close()


def test_kv_f16_bad_type(tiny):
    g, _ = tiny
    h = C.c_void_p()
    assert _native.lib().ifx_session_create_kv(g.h, 64, 2, C.byref(h)) == 20  # IFX_E_INVALID_ARG
    assert not h.value


def test_kv_f16_needs_head_dim_multiple_of_8(tmp_path):
    """head_dim 4 (the reference's forward-test model): an f32 cache is fine,
    an f16 one is refused with IFX_E_INVALID_ARG; decode on the f32 one runs."""
    from tests import fixtures_gguf as fx
    p = str(tmp_path / "hd4.gguf")
    fx.builder_llama_gguf(p, 1.0, hidden=8, heads=2)
    g = GpuModel(p)
    h = C.c_void_p()
    assert _native.lib().ifx_session_create_kv(g.h, 16, 1, C.byref(h)) == 20
    assert not h.value
    s = g.session(16)
    rc, lg = s.decode_step(3)
    assert rc == 0 and np.all(np.isfinite(lg))
    s.close()
    g.close()
