"""Model-level parity on the GPU against the oracle.

Bar (the token loop's correctness contract): logits within 1e-3 relative L2 of
the oracle per step, and greedy tokens identical for the whole run (>= 64
tokens) on the synthetic models; bit-exact KV export of imported state.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from inferox_amd import synth
from oracle import binding as orc
from tests import fixtures_gguf as fx
from tests.conftest import rel_l2
from tests.gpu_util import GpuModel

pytestmark = pytest.mark.gpu

TOL = 1e-3  # relative L2 of the logits per step


@pytest.fixture(scope="module")
def tiny(tiny_path):
    g = GpuModel(tiny_path)
    o = orc.Model(tiny_path)
    yield g, o
    g.close()
    o.close()


def test_tiny_config(tiny):
    g, o = tiny
    assert (g.cfg.vocab_size, g.cfg.hidden_size, g.cfg.n_layers, g.cfg.n_heads, g.cfg.head_dim) == \
        (32000, 288, 6, 6, 48)
    assert g.cfg.rope_base == o.cfg.rope_base and g.cfg.rope_dim == o.cfg.rope_dim


def test_tiny_decode_steps_cli_style(tiny, tiny_prompt):
    """The CLI path (src/main.rs:68-82): every prompt token through decode_step,
    then greedy decode_steps; logits compared at every step."""
    g, o = tiny
    s, kv = g.session(256), o.kv(256)
    worst = 0.0
    tok = None
    for i in range(16 + 48):
        t = int(tiny_prompt[i]) if i < 16 else tok
        rc, lg = s.decode_step(t)
        orc_rc, ref = o.decode_step(kv, t)
        assert rc == 0 and orc_rc == 0
        worst = max(worst, rel_l2(lg, ref))
        tok = orc.argmax(ref)[1]
        gpu_pick = len(lg) - 1 - int(np.argmax(lg[::-1]))  # last index of the maximum
        assert gpu_pick == tok, f"step {i}: greedy pick differs"
    assert worst < TOL, worst
    assert len(s) == 64


def test_tiny_generate_matches_oracle(tiny, tiny_prompt):
    """Model::generate (src/model/forward.rs:592-612): 16-token prompt, 128 greedy steps."""
    g, o = tiny
    s, kv = g.session(256), o.kv(256)
    rc, toks = s.generate(tiny_prompt, 128)
    orc_rc, ref = o.generate(kv, tiny_prompt, 128)
    assert rc == 0 and orc_rc == 0
    assert toks.tolist() == ref.tolist()
    assert len(s) == 16 + 128


def test_tiny_prefill_logits(tiny, tiny_prompt):
    g, o = tiny
    s, kv = g.session(64), o.kv(64)
    rc, lg = s.prefill(tiny_prompt)
    orc_rc, ref = o.prefill(kv, tiny_prompt)
    assert rc == 0 and orc_rc == 0
    for t in range(len(tiny_prompt)):
        assert rel_l2(lg[t], ref[t]) < TOL, t
    # a second chunk: positions restart, attention stays inside the chunk (Q2)
    rc, lg2 = s.prefill(tiny_prompt[:5])
    orc_rc, ref2 = o.prefill(kv, tiny_prompt[:5])
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg2[t], ref2[t]) for t in range(5)) < TOL
    assert len(s) == 21
    # KV state equals the oracle's
    k, v = s.kv_export(21)
    kr, vr = kv.export(21)
    assert rel_l2(k, kr) < TOL and rel_l2(v, vr) < TOL


def test_tiny_forward(tiny, tiny_prompt):
    g, o = tiny
    rc, lg = g.forward(tiny_prompt[:8])
    orc_rc, ref = o.forward(tiny_prompt[:8])
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg[t], ref[t]) for t in range(8)) < TOL


def test_tiny_kv_import_export_and_decode(tiny):
    g, o = tiny
    c = o.cfg
    L = 40
    kvd = c.n_kv_heads * c.head_dim
    k = synth.normal_f32(c.n_layers * L * kvd, seed=3)
    v = synth.normal_f32(c.n_layers * L * kvd, seed=4)
    s, kv = g.session(128), o.kv(128)
    assert s.kv_import(k, v, L) == 0 and kv.import_(k, v, L) == 0
    ke, ve = s.kv_export(L)
    np.testing.assert_array_equal(ke, k)
    np.testing.assert_array_equal(ve, v)
    worst = 0.0
    for t in [5, 900, 31999, 0]:
        rc, lg = s.decode_step(t)
        _, ref = o.decode_step(kv, t)
        assert rc == 0
        worst = max(worst, rel_l2(lg, ref))
    assert worst < TOL
    # greedy continuation on the device equals the oracle's picks
    rc, toks = s.decode_greedy(7, 24)
    assert rc == 0
    ref_toks, t = [], 7
    for _ in range(24):
        _, lg = o.decode_step(kv, t)
        t = orc.argmax(lg)[1]
        ref_toks.append(t)
    assert toks.tolist() == ref_toks


def test_tiny_rope_absolute(tiny, tiny_prompt):
    g, o = tiny
    s, kv = g.session(64), o.kv(64)
    s.set_rope_mode(1)
    for t in tiny_prompt[:10]:
        rc, lg = s.decode_step(int(t))
        _, ref = o.decode_step(kv, int(t), rope_mode=orc.ROPE_ABSOLUTE)
        assert rc == 0 and rel_l2(lg, ref) < TOL


def test_tiny_decode_to_the_last_row(tiny, tiny_prompt):
    """130 decode steps in a session of 130 rows (two 64-row chunks and a
    2-row one), every step against the oracle; the last attends every row of
    the cache, and a further step is refused."""
    g, o = tiny
    s, kv = g.session(130), o.kv(130)
    tok = int(tiny_prompt[0])
    for step in range(130):
        rc, lg = s.decode_step(tok)
        _, ref = o.decode_step(kv, tok)
        assert rc == 0 and rel_l2(lg, ref) < TOL, step
        tok = int(tiny_prompt[(step + 1) % len(tiny_prompt)])
    assert len(s) == 130 and s.decode_step(tok)[0] == 21


def test_errors(tiny):
    g, _ = tiny
    s = g.session(2)
    assert s.decode_step(32000)[0] == 10
    assert s.decode_step(1)[0] == 0 and s.decode_step(1)[0] == 0
    assert s.decode_step(1)[0] == 21
    s.clear()
    assert len(s) == 0 and s.decode_step(1)[0] == 0
    assert s.prefill([1, 32000])[0] == 10
    assert s.prefill([1, 2, 3])[0] == 21
    assert s.generate(np.zeros(0, np.uint32), 3)[0] == 20
    assert s.generate([1], 5)[0] == 21


def test_reference_generate_kat(tmp_path):
    """generate_with_kv_cache_runs (src/model/forward.rs:786-839) on the GPU: all-zero
    weights give zero logits, ties go to the last index: [99]*5 and len 8."""
    p = str(tmp_path / "z.gguf")
    fx.builder_llama_gguf(p, fill=0.0, ctx=32)
    g = GpuModel(p)
    s = g.session(32)
    rc, toks = s.generate([0, 1, 2], 5)
    assert rc == 0 and toks.tolist() == [99] * 5 and len(s) == 8
    rc, lg = g.forward([0])
    assert rc == 0 and lg.shape == (1, 100)
    g.close()


def test_layer_forward_runs(tmp_path):
    """layer_forward_runs_without_panic (src/model/forward.rs:729-784) on the GPU,
    with the oracle's logits as the check."""
    p = str(tmp_path / "f.gguf")
    fx.builder_llama_gguf(p, fill=1.0, ctx=128)
    g, o = GpuModel(p), orc.Model(p)
    rc, lg = g.forward([0])
    _, ref = o.forward([0])
    assert rc == 0 and lg.shape == (1, 100)
    np.testing.assert_allclose(lg, ref, atol=1e-6)
    g.close()


@pytest.mark.parametrize("max_seq", [512, 4096])
def test_8b_shape_two_layers(tmpdir_session, max_seq):
    """Full-width Llama-3-8B shape (Q4_K / Q6_K mix, GQA 32/8, vocab 128256), two
    layers so the oracle finishes in seconds: decode from a seeded KV context,
    in a 512-row and a 4096-row cache (64 chunk records per kv head to merge)."""
    spec = synth.reduced(synth.LLAMA3_8B, n_layers=2, ctx=512)
    p = str(tmpdir_session / "l8b_2l.gguf")
    if not os.path.exists(p):
        synth.write_llama(p, spec, seed=8)
    g, o = GpuModel(p), orc.Model(p)
    c = o.cfg
    L = 200
    kvd = c.n_kv_heads * c.head_dim
    k = synth.normal_f32(c.n_layers * L * kvd, seed=21)
    v = synth.normal_f32(c.n_layers * L * kvd, seed=22)
    s, kv = g.session(max_seq), o.kv(max_seq)
    assert s.kv_import(k, v, L) == 0 and kv.import_(k, v, L) == 0
    tok = 1000
    for step in range(4):
        rc, lg = s.decode_step(tok)
        _, ref = o.decode_step(kv, tok)
        assert rc == 0
        assert rel_l2(lg, ref) < TOL, step
        tok = orc.argmax(ref)[1]
        assert lg[tok] == lg.max()
    g.close()


@pytest.mark.parametrize("max_seq", [512, 2048])
def test_70b_shape_two_layers(tmpdir_session, max_seq):
    """Llama-3-70B widths (dim 8192, ffn 28672, GQA 64/8, vocab 128256), two
    layers: decode from a seeded KV context (group-8 attention, 28672-column
    down projection) and a batched prefill chunk, against the oracle."""
    spec = synth.reduced(synth.LLAMA3_70B, n_layers=2, ctx=512)
    p = str(tmpdir_session / "l70b_2l.gguf")
    if not os.path.exists(p):
        synth.write_llama(p, spec, seed=70)
    g, o = GpuModel(p), orc.Model(p)
    c = o.cfg
    L = 300
    kvd = c.n_kv_heads * c.head_dim
    k = synth.normal_f32(c.n_layers * L * kvd, seed=23)
    v = synth.normal_f32(c.n_layers * L * kvd, seed=24)
    s, kv = g.session(max_seq), o.kv(max_seq)
    assert s.kv_import(k, v, L) == 0 and kv.import_(k, v, L) == 0
    tok = 4242
    for step in range(3):
        rc, lg = s.decode_step(tok)
        _, ref = o.decode_step(kv, tok)
        assert rc == 0
        assert rel_l2(lg, ref) < TOL, step
        tok = orc.argmax(ref)[1]
        assert lg[tok] == lg.max()
    # a batched prefill chunk after the decoded rows (chunk-only attention)
    ids = synth.token_ids(64, spec.vocab, seed=71)
    rc, lg = s.prefill(ids)
    orc_rc, ref = o.prefill(kv, ids)
    assert rc == 0 and orc_rc == 0
    assert max(rel_l2(lg[t], ref[t]) for t in range(len(ids))) < TOL
    g.close()
