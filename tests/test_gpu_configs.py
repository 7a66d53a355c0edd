"""Parity at the benchmark workloads' own sizes, against the oracle.

* 8B shape: decode over a 2048-row cache (two layers); batched prefill of 512
  and 2048 ids (two layers), causal and non-causal, f32 and f16 caches; and
  the full 32-layer model: a GPU prefill of 2048 ids, its cache exported into
  the oracle, then 64 decode steps compared step by step (logits within 1e-3
  relative L2, greedy picks identical) and the device's own 64-token greedy
  loop equal to the oracle's picks.
* 70B shape: decode over an 8192-row cache (two layers; 129 chunk records per
  kv head to merge).
* The attention merge in the O projection's prologue (the default up to 48
  chunk records) at a length in each of its chunk bounds (8 to 48 records),
  forced at 63 and 129 records, and the separate merge launch forced at 33.
* Long caches past one merge batch (256 chunks of 64 rows): 4200 and 20000
  rows at query-group sizes 1, 4 and 8, with the f32 and the f16 cache.
* Tiny model prefill chunks of 129, 300 and 512 ids (several 128-query
  blocks, causal key ranges over several key blocks).

The f32 cache is the reference's KvCache (src/model/cache.rs:8-24); the f16
cache is compared with the oracle's f16 mode at TOL16 (see test_gpu_kv_f16).
Decode attention follows src/model/forward.rs:383-414, prefill
src/model/forward.rs:215-337,496-538, generate src/model/forward.rs:592-622.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

from inferox_amd import _native, synth
from oracle import binding as orc
from tests.conftest import rel_l2
from tests.gpu_util import GpuModel

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL16 = 4e-3


def f16(x):
    with np.errstate(over="ignore"):
        return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def last_argmax(lg):
    return len(lg) - 1 - int(np.argmax(lg[::-1]))


def _model(tmpdir, name, spec, seed):
    p = str(tmpdir / name)
    if not os.path.exists(p):
        synth.write_llama(p, spec, seed=seed)
    return p


def _decode_from_import(g, o, rows, max_seq, steps, tok, seed, kv_f16=False):
    """Seeded K/V rows imported into both, then `steps` decode steps compared."""
    c = o.cfg
    kvd = c.n_kv_heads * c.head_dim
    k = synth.normal_f32(c.n_layers * rows * kvd, seed=seed)
    v = synth.normal_f32(c.n_layers * rows * kvd, seed=seed + 1)
    if kv_f16:
        k, v = f16(k), f16(v)
    s, kv = g.session(max_seq, kv_f16=kv_f16), o.kv(max_seq, f16=kv_f16)
    assert s.kv_import(k, v, rows) == 0 and kv.import_(k, v, rows) == 0
    tol = TOL16 if kv_f16 else TOL
    worst = 0.0
    for step in range(steps):
        rc, lg = s.decode_step(tok)
        orc_rc, ref = o.decode_step(kv, tok)
        assert rc == 0 and orc_rc == 0
        worst = max(worst, rel_l2(lg, ref))
        tok = orc.argmax(ref)[1]
        assert last_argmax(lg) == tok, step
    assert worst < tol, worst
    s.close()
    return worst


# ---------------------------------------------------------------- decode sizes

def test_8b_decode_over_2048_rows(tmpdir_session):
    """Two layers of the 8B shape decoding over a 2048-row cache (33 chunks per kv head)."""
    spec = synth.reduced(synth.LLAMA3_8B, n_layers=2, ctx=512)
    p = _model(tmpdir_session, "l8b_2l.gguf", spec, 8)
    g, o = GpuModel(p), orc.Model(p)
    _decode_from_import(g, o, 2048, 2304, 4, 1000, seed=41)
    _decode_from_import(g, o, 2048, 2304, 2, 77, seed=43, kv_f16=True)
    g.close()
    o.close()


def test_70b_decode_over_8192_rows(tmpdir_session):
    """Two layers of the 70B shape decoding over an 8192-row cache: 129 chunk
    records per kv head in one merge batch, query group 8, the 28672-column
    down projection."""
    spec = synth.reduced(synth.LLAMA3_70B, n_layers=2, ctx=512)
    p = _model(tmpdir_session, "l70b_2l.gguf", spec, 70)
    g, o = GpuModel(p), orc.Model(p)
    _decode_from_import(g, o, 8192, 8320, 4, 4242, seed=45)
    g.close()
    o.close()


@pytest.mark.parametrize("shape,rows", [("8b", 4000), ("70b", 8192)])
def test_merge_in_o_projection_long(tmpdir_session, monkeypatch, shape, rows):
    """The attention merge in the O projection's prologue (taken by default up
    to 48 chunk records) forced at 63 and 129 records per kv head: the chunks
    past its first batch, and past 64 for the maximum and the denominator, are
    read in its loops."""
    monkeypatch.setenv("IFX_MERGE_O", "1")
    base, name, seed = (synth.LLAMA3_8B, "l8b_2l.gguf", 8) if shape == "8b" else (synth.LLAMA3_70B, "l70b_2l.gguf", 70)
    spec = synth.reduced(base, n_layers=2, ctx=512)
    p = _model(tmpdir_session, name, spec, seed)
    g, o = GpuModel(p), orc.Model(p)
    _decode_from_import(g, o, rows, rows + 8, 2, 321, seed=rows + 7)
    g.close()
    o.close()


@pytest.mark.parametrize("shape,rows", [("8b", r) for r in (100, 900, 1400, 1900, 2400, 2900)]
                         + [("70b", 900), ("70b", 2900)])
def test_merge_in_o_projection_each_bound(tmpdir_session, shape, rows):
    """The merged O launch at every chunk bound it has an instance for: 2, 15,
    22, 30, 38 and 46 chunk records per kv head (the host's bounds 8, 16, 24,
    32, 40 and 48; the launch loads that many records per kv head)."""
    base, name, seed = (synth.LLAMA3_8B, "l8b_2l.gguf", 8) if shape == "8b" else (synth.LLAMA3_70B, "l70b_2l.gguf", 70)
    spec = synth.reduced(base, n_layers=2, ctx=512)
    p = _model(tmpdir_session, name, spec, seed)
    g, o = GpuModel(p), orc.Model(p)
    _decode_from_import(g, o, rows, rows + 8, 1, 555, seed=rows + 3)
    g.close()
    o.close()


def test_separate_merge_short_context(tmpdir_session, monkeypatch):
    """The separate merge launch forced where the fused one is the default (2048 rows)."""
    monkeypatch.setenv("IFX_MERGE_O", "0")
    spec = synth.reduced(synth.LLAMA3_8B, n_layers=2, ctx=512)
    p = _model(tmpdir_session, "l8b_2l.gguf", spec, 8)
    g, o = GpuModel(p), orc.Model(p)
    _decode_from_import(g, o, 2048, 2304, 2, 1000, seed=51)
    g.close()
    o.close()


NARROW = {
    # group 4 and group 8 at head dim 128 (the 8B / 70B attention kernels), small widths
    4: synth.reduced(synth.LLAMA3_8B, name="narrow-g4", dim=1024, ffn=1024, n_layers=2, n_heads=8, n_kv_heads=2,
                     vocab=2048, ctx=512),
    8: synth.reduced(synth.LLAMA3_8B, name="narrow-g8", dim=2048, ffn=1024, n_layers=2, n_heads=16, n_kv_heads=2,
                     vocab=2048, ctx=512),
}


@pytest.mark.parametrize("rows", [4200, 20000])
@pytest.mark.parametrize("group", [1, 4, 8])
@pytest.mark.parametrize("kv_f16", [False, True])
def test_long_cache_merge(tmpdir_session, tiny_path, rows, group, kv_f16):
    """Caches of 66 and 313 chunks per kv head: the merge's weights taken over
    more than one 256-chunk batch (20000 rows), past the former 16384-row cap."""
    if group == 1:
        p = tiny_path
    else:
        p = _model(tmpdir_session, f"narrow_g{group}.gguf", NARROW[group], 90 + group)
    g, o = GpuModel(p), orc.Model(p)
    assert g.cfg.n_heads // g.cfg.n_kv_heads == group
    _decode_from_import(g, o, rows, rows + 8, 2, 11, seed=rows + group, kv_f16=kv_f16)
    g.close()
    o.close()


def test_session_beyond_former_cap(tiny_path):
    """A 131072-row session (a common context_length) decodes: no 16384-row limit."""
    g, o = GpuModel(tiny_path), orc.Model(tiny_path)
    s, kv = g.session(131072), o.kv(64)
    for t in (5, 9, 13):
        rc, lg = s.decode_step(t)
        _, ref = o.decode_step(kv, t)
        assert rc == 0 and rel_l2(lg, ref) < TOL
    s.close()
    g.close()
    o.close()


# --------------------------------------------------------------- prefill sizes

@pytest.mark.parametrize("n", [129, 300, 512])
def test_tiny_prefill_chunk_sizes(tiny_path, n):
    """Several 128-query blocks and causal key ranges spanning several 64-key
    blocks; logits of every row and the cache rows."""
    g, o = GpuModel(tiny_path), orc.Model(tiny_path)
    ids = synth.token_ids(n, synth.TINY.vocab, seed=600 + n)
    s, kv = g.session(n + 16), o.kv(n + 16)
    rc, lg = s.prefill(ids)
    orc_rc, ref = o.prefill(kv, ids)
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg[t], ref[t]) for t in range(n)) < TOL
    k, v = s.kv_export(n)
    kr, vr = kv.export(n)
    assert rel_l2(k, kr) < 1e-4 and rel_l2(v, vr) < 1e-4
    rc, lg = g.forward(ids)
    orc_rc, ref = o.forward(ids)
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg[t], ref[t]) for t in range(n)) < TOL
    s.close()
    g.close()
    o.close()


def _sample_rows(n, seed):
    rng = np.random.default_rng(seed)
    return sorted(set(rng.choice(n, 64, replace=False).tolist()) | {0, n - 1})


@pytest.mark.parametrize("n", [512, 2048])
def test_8b_batched_prefill_sizes(tmpdir_session, n):
    """Two layers of the 8B shape, one prefill chunk of n ids through the
    Q4_K/Q6_K GEMMs and the causal attention: the last row and 64 seeded rows
    of logits, every K/V row, and the greedy pick of the last row."""
    spec = synth.reduced(synth.LLAMA3_8B, n_layers=2, ctx=512)
    p = _model(tmpdir_session, "l8b_2l.gguf", spec, 8)
    g, o = GpuModel(p), orc.Model(p)
    assert g.batched_prefill()
    ids = synth.token_ids(n, spec.vocab, seed=512 + n)
    rows = _sample_rows(n, n)
    s, kv = g.session(n + 16), o.kv(n + 16)
    rc, lg = s.prefill(ids)
    orc_rc, ref = o.prefill_rows(kv, ids, rows)
    assert rc == 0 and orc_rc == 0
    worst = max(rel_l2(lg[t], ref[i]) for i, t in enumerate(rows))
    assert worst < TOL, worst
    k, v = s.kv_export(n)
    kr, vr = kv.export(n)
    assert rel_l2(k, kr) < 1e-4 and rel_l2(v, vr) < 1e-4
    last = C.c_uint32()
    assert _native.lib().ifx_session_last_token(s.h, C.byref(last)) == 0
    assert last.value == orc.argmax(ref[-1])[1]
    s.close()
    g.close()
    o.close()


def test_8b_prefill_512_forward_and_f16(tmpdir_session):
    """The same 8B-shape model at 512 ids: non-causal Model::forward (no cache)
    and the causal prefill into an f16 cache."""
    spec = synth.reduced(synth.LLAMA3_8B, n_layers=2, ctx=512)
    p = _model(tmpdir_session, "l8b_2l.gguf", spec, 8)
    g, o = GpuModel(p), orc.Model(p)
    n = 512
    ids = synth.token_ids(n, spec.vocab, seed=1512)
    rows = _sample_rows(n, 7)
    rc, lg = g.forward(ids)
    orc_rc, ref = o.forward_rows(ids, rows)
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg[t], ref[i]) for i, t in enumerate(rows)) < TOL
    s, kv = g.session(n + 16, kv_f16=True), o.kv(n + 16, f16=True)
    rc, lg = s.prefill(ids)
    orc_rc, ref = o.prefill_rows(kv, ids, rows)
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg[t], ref[i]) for i, t in enumerate(rows)) < TOL16
    s.close()
    g.close()
    o.close()


# --------------------------------------------------------- the full 8B model

def test_8b_full_model_prefill_then_64_greedy_tokens(tmpdir_session):
    """The benchmark's 8B Q4_K_M workload end to end at full depth (32 layers):
    a GPU batched prefill of 2048 seeded ids, its cache exported into the
    oracle, then 64 decode steps from the prefill's greedy pick with logits
    within 1e-3 per step and identical greedy picks; the device's own greedy
    loop (ifx_decode_greedy) after the same prefill gives the same 64 tokens."""
    p = _model(tmpdir_session, "l8b_full.gguf", synth.LLAMA3_8B, 1234)
    g = GpuModel(p)
    c = g.cfg
    assert c.n_layers == 32 and g.batched_prefill()
    ctx, steps, max_seq = 2048, 64, 2048 + 64 + 8
    ids = synth.token_ids(ctx, c.vocab_size, seed=2048)
    s = g.session(max_seq)
    rc, _ = s.prefill(ids, want_logits=False)
    assert rc == 0
    last = C.c_uint32()
    assert _native.lib().ifx_session_last_token(s.h, C.byref(last)) == 0
    k, v = s.kv_export(ctx)
    o = orc.Model(p)
    kv = o.kv(max_seq)
    assert kv.import_(k, v, ctx) == 0
    del k, v
    tok, picks, worst = int(last.value), [], 0.0
    for step in range(steps):
        rc, lg = s.decode_step(tok)
        orc_rc, ref = o.decode_step(kv, tok)
        assert rc == 0 and orc_rc == 0
        worst = max(worst, rel_l2(lg, ref))
        tok = orc.argmax(ref)[1]
        assert last_argmax(lg) == tok, step
        picks.append(tok)
    assert worst < TOL, worst
    s.close()
    # the device greedy loop from the same prefilled state
    s2 = g.session(max_seq)
    rc, _ = s2.prefill(ids, want_logits=False)
    assert rc == 0
    rc, toks = s2.decode_greedy(int(last.value), steps)
    assert rc == 0
    assert toks.tolist() == picks
    s2.close()
    g.close()
    o.close()
