"""Model-level parity on centred synthetic models (zero-mean K-quant weights,
inferox_amd/synth.py), where the attention carries weight in the logits and
the greedy picks move from token to token.

Each test first checks on the oracle side that it can see what it is about:
replacing the imported V rows (decode) or dropping the causal mask (prefill)
moves the oracle's logits by at least 10 x TOL; the ABSOLUTE-RoPE test checks
that the rotation moves them.  Then the GPU runs the same steps: logits within
TOL relative L2 per step, identical greedy picks, and the K/V rows the steps
write (src/model/forward.rs:371-378) within 1e-4 of the oracle's.

* 8B shape (32/8 heads, 4096 wide; two layers): decode over 2048 imported
  rows, batched prefill of 512 and 2048 ids, ABSOLUTE RoPE (K-split q/k/v on
  the f32 cache, the tiled launch on the f16 cache and in the deterministic
  mode), the deterministic mode (bit-identical reruns, sampled generate), the
  launch variants behind the IFX_* switches, and per-layer types as real
  Q4_K_M files mix them.
* 70B shape (64/8 heads, 8192 wide; two layers): decode over 8192 rows.
* The full 32-layer 8B shape: GPU prefill of 2048 ids, then 64 greedy steps
  against the oracle (Model::generate, src/model/forward.rs:592-622).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np
import pytest

from inferox_amd import _native, synth
from inferox_amd.gguf_writer import Q4_K, Q6_K
from oracle import binding as orc
from tests.conftest import rel_l2
from tests.gpu_util import GpuModel

pytestmark = pytest.mark.gpu

TOL = 1e-3
TOL16 = 4e-3
KV_TOL = 1e-4
SEEN = 10.0  # the guards: what a test relies on moves the logits by >= SEEN x TOL

C8B = synth.reduced(synth.LLAMA3_8B, name="c8b", n_layers=2, ctx=512, centred=True)
C70B = synth.reduced(synth.LLAMA3_70B, name="c70b", n_layers=2, ctx=512, centred=True)
# layer 1 as other layers of a real Q4_K_M file: attn_v and ffn_down in Q4_K, and
# (beyond Q4_K_M) attn_output in Q6_K for the Q6_K merged-O launch
C8B_MIX = synth.reduced(C8B, name="c8b-mix", layer_types={1: {"v": Q4_K, "down": Q4_K, "o": Q6_K}})
C8B_FULL = synth.reduced(synth.LLAMA3_8B, name="c8b-full", centred=True)


def last_argmax(lg):
    return len(lg) - 1 - int(np.argmax(lg[::-1]))


def f16(x):
    with np.errstate(over="ignore"):
        return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def _model(tmpdir, name, spec, seed):
    p = str(tmpdir / name)
    if not os.path.exists(p):
        synth.write_llama(p, spec, seed=seed)
    return p


def _kv_rows(o, rows, seed, kv_f16=False):
    c = o.cfg
    n = c.n_layers * rows * c.n_kv_heads * c.head_dim
    k, v = synth.normal_f32(n, seed=seed), synth.normal_f32(n, seed=seed + 1)
    return (f16(k), f16(v)) if kv_f16 else (k, v)


def _rows_of(x, c, rows, r0, r1):
    """Rows r0..r1-1 of an export [layer][rows][kv_dim]."""
    return x.reshape(c.n_layers, rows, -1)[:, r0:r1]


def decode_parity(g, o, rows, steps, tok, seed, kv_f16=False, rope_mode=0, deterministic=False, guard=True,
                  spare=8):
    """Seeded rows imported into both, `steps` decode steps compared (logits,
    picks), then the rows the steps wrote; the session holds `spare` rows
    more.  Returns (worst rel L2, picks)."""
    c = o.cfg
    max_seq = rows + steps + spare
    k, v = _kv_rows(o, rows, seed, kv_f16)
    if guard:
        # the oracle's first step sees the imported V rows
        kv_a, kv_b = o.kv(max_seq, f16=kv_f16), o.kv(max_seq, f16=kv_f16)
        assert kv_a.import_(k, v, rows) == 0
        v2 = _kv_rows(o, rows, seed + 7, kv_f16)[1]
        assert kv_b.import_(k, v2, rows) == 0
        _, la = o.decode_step(kv_a, tok, rope_mode=rope_mode)
        _, lb = o.decode_step(kv_b, tok, rope_mode=rope_mode)
        assert rel_l2(lb, la) >= SEEN * TOL, rel_l2(lb, la)
    s, kv = g.session(max_seq, kv_f16=kv_f16), o.kv(max_seq, f16=kv_f16)
    if rope_mode:
        s.set_rope_mode(rope_mode)
    if deterministic:
        s.set_deterministic(True)
    assert s.kv_import(k, v, rows) == 0 and kv.import_(k, v, rows) == 0
    tol = TOL16 if kv_f16 else TOL
    worst, picks = 0.0, []
    for step in range(steps):
        rc, lg = s.decode_step(tok)
        orc_rc, ref = o.decode_step(kv, tok, rope_mode=rope_mode)
        assert rc == 0 and orc_rc == 0
        worst = max(worst, rel_l2(lg, ref))
        tok = orc.argmax(ref)[1]
        assert last_argmax(lg) == tok, step
        picks.append(tok)
    assert worst < tol, worst
    if spare == 0:  # the cache is full: the next step is refused (src/model/forward.rs:376)
        assert s.decode_step(tok)[0] == 21
    # the K/V rows the steps appended (src/model/forward.rs:374-378)
    kg, vg = s.kv_export(rows + steps)
    kr, vr = kv.export(rows + steps)
    for a, b in ((kg, kr), (vg, vr)):
        new_g, new_r = _rows_of(a, c, rows + steps, rows, rows + steps), _rows_of(b, c, rows + steps, rows, rows + steps)
        assert rel_l2(new_g, new_r) < (TOL16 if kv_f16 else KV_TOL), rel_l2(new_g, new_r)
        # and the imported rows are untouched
        assert np.array_equal(_rows_of(a, c, rows + steps, 0, rows), _rows_of(b, c, rows + steps, 0, rows))
    s.close()
    return worst, picks


def test_centred_8b_decode_over_2048_rows(tmpdir_session):
    p = _model(tmpdir_session, "c8b_2l.gguf", C8B, 88)
    g, o = GpuModel(p), orc.Model(p)
    decode_parity(g, o, 2048, 4, 1000, seed=41)
    decode_parity(g, o, 2048, 2, 77, seed=43, kv_f16=True)
    g.close()
    o.close()


@pytest.mark.parametrize("kv_f16", [False, True])
def test_centred_8b_decode_fills_the_cache(tmpdir_session, kv_f16):
    """A session of exactly 2048 rows, 2045 imported and 3 decoded: the last
    step writes row 2047 and attends all 32 chunks of the chunk grid, which
    ends there; a further step is refused."""
    p = _model(tmpdir_session, "c8b_2l.gguf", C8B, 88)
    g, o = GpuModel(p), orc.Model(p)
    decode_parity(g, o, 2045, 3, 321, seed=47, kv_f16=kv_f16, spare=0)
    g.close()
    o.close()


def test_centred_70b_decode_over_8192_rows(tmpdir_session):
    """Query group 8, 129 chunk records per kv head merged by their own launch."""
    p = _model(tmpdir_session, "c70b_2l.gguf", C70B, 77)
    g, o = GpuModel(p), orc.Model(p)
    decode_parity(g, o, 8192, 2, 4242, seed=45)
    g.close()
    o.close()


@pytest.mark.parametrize("kv_f16,deterministic", [(False, False), (True, False), (False, True)])
def test_centred_absolute_rope_decode(tmpdir_session, kv_f16, deterministic):
    """ABSOLUTE RoPE at positions 300.. on the K-quant path: the K-split q/k/v
    launch rotating its partial sums (f32 cache), the tiled launch's epilogue
    (f16 cache, and the deterministic mode on the f32 cache)."""
    p = _model(tmpdir_session, "c8b_2l.gguf", C8B, 88)
    g, o = GpuModel(p), orc.Model(p)
    rows = 300
    # the guard: ABSOLUTE and REFERENCE positions give different logits
    k, v = _kv_rows(o, rows, 61)
    kv_a, kv_b = o.kv(rows + 8), o.kv(rows + 8)
    kv_a.import_(k, v, rows)
    kv_b.import_(k, v, rows)
    _, la = o.decode_step(kv_a, 5, rope_mode=orc.ROPE_ABSOLUTE)
    _, lb = o.decode_step(kv_b, 5, rope_mode=orc.ROPE_REFERENCE)
    assert rel_l2(la, lb) >= SEEN * TOL
    decode_parity(g, o, rows, 3, 5, seed=61, kv_f16=kv_f16, rope_mode=orc.ROPE_ABSOLUTE,
                  deterministic=deterministic)
    g.close()
    o.close()


@pytest.mark.parametrize("n", [512, 2048])
def test_centred_8b_batched_prefill(tmpdir_session, n):
    """One prefill chunk of n ids through the GEMMs and the causal attention:
    sampled rows' logits, every K/V row and the last row's pick."""
    p = _model(tmpdir_session, "c8b_2l.gguf", C8B, 88)
    g, o = GpuModel(p), orc.Model(p)
    assert g.batched_prefill()
    ids = synth.token_ids(n, C8B.vocab, seed=900 + n)
    rng = np.random.default_rng(n)
    rows = sorted(set(rng.choice(n - 1, 24, replace=False).tolist()) | {0, n // 2, n - 1})
    kv = o.kv(n + 8)
    orc_rc, ref = o.prefill_rows(kv, ids, rows)
    assert orc_rc == 0
    # the guard: without the causal mask the sampled rows' logits move
    _, full = o.forward_rows(ids, rows)
    moved = [rel_l2(full[i], ref[i]) for i in range(len(rows) - 1)]
    assert np.median(moved) >= SEEN * TOL, moved
    s = g.session(n + 8)
    rc, lg = s.prefill(ids)
    assert rc == 0
    worst = max(rel_l2(lg[t], ref[i]) for i, t in enumerate(rows))
    assert worst < TOL, worst
    kg, vg = s.kv_export(n)
    kr, vr = kv.export(n)
    assert rel_l2(kg, kr) < KV_TOL and rel_l2(vg, vr) < KV_TOL
    last = C.c_uint32()
    assert _native.lib().ifx_session_last_token(s.h, C.byref(last)) == 0
    assert last.value == orc.argmax(ref[-1])[1]
    s.close()
    g.close()
    o.close()


def test_centred_8b_two_prefill_chunks_then_decode(tmpdir_session):
    """Two batched prefill chunks, 300 ids and then 200 at cache row 300
    (RoPE positions relative to the chunk, attention within it:
    src/model/forward.rs:496-538), neither a whole number of 128-row query
    blocks; then 3 decode steps over all 500 rows.  Sampled rows' logits,
    every K/V row, and the decode logits and picks against the oracle."""
    p = _model(tmpdir_session, "c8b_2l.gguf", C8B, 88)
    g, o = GpuModel(p), orc.Model(p)
    assert g.batched_prefill()
    # the guard: the second chunk at absolute positions 300.. stores other K
    # rows (its own logits hardly move: a common shift of q and k positions
    # leaves q . k as it is)
    ids1, ids2 = synth.token_ids(300, C8B.vocab, seed=1300), synth.token_ids(200, C8B.vocab, seed=1301)
    kv_a, kv_b = o.kv(512), o.kv(512)
    for kv_x, mode in ((kv_a, orc.ROPE_REFERENCE), (kv_b, orc.ROPE_ABSOLUTE)):
        assert o.prefill_rows(kv_x, ids1, [299])[0] == 0
        assert o.prefill_rows(kv_x, ids2, [199], rope_mode=mode)[0] == 0
    ka, kb = kv_a.export(500)[0], kv_b.export(500)[0]
    assert rel_l2(_rows_of(kb, o.cfg, 500, 300, 500), _rows_of(ka, o.cfg, 500, 300, 500)) >= SEEN * KV_TOL
    kv, s = o.kv(512), g.session(512)
    for n, seed in ((300, 1300), (200, 1301)):
        ids = synth.token_ids(n, C8B.vocab, seed=seed)
        rows = sorted({0, 1, n // 3, n // 2, n - 2, n - 1})
        orc_rc, ref = o.prefill_rows(kv, ids, rows)
        rc, lg = s.prefill(ids)
        assert rc == 0 and orc_rc == 0
        worst = max(rel_l2(lg[t], ref[i]) for i, t in enumerate(rows))
        assert worst < TOL, (n, worst)
    kg, vg = s.kv_export(500)
    kr, vr = kv.export(500)
    assert rel_l2(kg, kr) < KV_TOL and rel_l2(vg, vr) < KV_TOL
    tok = 77
    for step in range(3):
        rc, lg = s.decode_step(tok)
        orc_rc, ref = o.decode_step(kv, tok)
        assert rc == 0 and orc_rc == 0
        assert rel_l2(lg, ref) < TOL, step
        tok = orc.argmax(ref)[1]
        assert last_argmax(lg) == tok, step
    s.close()
    g.close()
    o.close()


def test_deterministic_mode_reruns_bit_identical(tmpdir_session):
    """ifx_session_set_deterministic: two sessions decoding the same steps give
    bit-identical logits; two sampled generates with one seed give the same
    tokens; and the mode keeps parity."""
    p = _model(tmpdir_session, "c8b_2l.gguf", C8B, 88)
    g, o = GpuModel(p), orc.Model(p)
    rows, steps = 2048, 6
    k, v = _kv_rows(o, rows, 71)
    runs = []
    for _ in range(2):
        s = g.session(rows + steps + 4)
        s.set_deterministic(True)
        assert s.kv_import(k, v, rows) == 0
        tok, out = 321, []
        for _ in range(steps):
            rc, lg = s.decode_step(tok)
            assert rc == 0
            out.append(lg.copy())
            tok = last_argmax(lg)
        runs.append(np.stack(out))
        s.close()
    assert np.array_equal(runs[0].view(np.uint32), runs[1].view(np.uint32))
    decode_parity(g, o, rows, 3, 321, seed=71, deterministic=True, guard=False)
    prompt = synth.token_ids(80, C8B.vocab, seed=5)
    toks = []
    for _ in range(2):
        s = g.session(160)
        s.set_deterministic(True)
        s.set_sampler(0.8, 40, 0.95, 1234)
        rc, t = s.generate_sampled(prompt, 48)
        assert rc == 0
        toks.append(t.tolist())
        s.close()
    assert toks[0] == toks[1]
    assert len(set(toks[0])) > 8  # the draws move
    g.close()
    o.close()


@pytest.mark.parametrize("env", [{"IFX_KS_LOCK": "0"}, {"IFX_QKV_KS": "0"}, {"IFX_QKV_KS": "0", "IFX_QKV_PLACE": "0"},
                                 {"IFX_ATTN_HKF": "0"}, {"IFX_ATTN_HKF": "1"}, {"IFX_MERGE_O": "0"},
                                 {"IFX_MERGE_O": "1"}, {"IFX_GEMV_HALVES": "0"}])
def test_centred_launch_variants(tmpdir_session, monkeypatch, env):
    """The launch variants the IFX_* switches select: each wave of the K-split
    residual launch on its own, the tiled q/k/v launch on the f32 cache (with
    and without its placement of the Q6_K tiles), both attention grid orders,
    each merge form forced, and the gate/up and head launches on whole tiles
    only (no half tiles in their last round)."""
    for key, val in env.items():
        monkeypatch.setenv(key, val)
    p = _model(tmpdir_session, "c8b_2l.gguf", C8B, 88)
    g, o = GpuModel(p), orc.Model(p)
    decode_parity(g, o, 1500, 2, 99, seed=81, guard=False)
    g.close()
    o.close()


def test_centred_mixed_layer_types(tmpdir_session):
    """Per-layer types as in real Q4_K_M files: layer 1's q/k/v launch all
    Q4_K, its ffn_down a Q4_K K-split launch at 14336 columns, and a Q6_K
    attn_output under the merged-O launch; decode and a prefill chunk."""
    p = _model(tmpdir_session, "c8b_mix.gguf", C8B_MIX, 89)
    g, o = GpuModel(p), orc.Model(p)
    decode_parity(g, o, 2048, 3, 17, seed=91)
    ids = synth.token_ids(256, C8B_MIX.vocab, seed=92)
    rows = [0, 100, 200, 255]
    kv = o.kv(300)
    _, ref = o.prefill_rows(kv, ids, rows)
    s = g.session(300)
    rc, lg = s.prefill(ids)
    assert rc == 0
    assert max(rel_l2(lg[t], ref[i]) for i, t in enumerate(rows)) < TOL
    s.close()
    g.close()
    o.close()


def test_centred_8b_full_model_prefill_then_64_greedy_tokens(tmpdir_session):
    """The 8B shape at full depth (32 layers, centred): a GPU batched prefill
    of 2048 seeded ids, its cache exported into the oracle, then 64 decode
    steps with logits within 1e-3 per step and identical greedy picks (which
    move); the top-2 margin of each step is printed.  The device's own greedy
    loop after the same prefill gives the same 64 tokens."""
    p = _model(tmpdir_session, "c8b_full.gguf", C8B_FULL, 1234)
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
    tok, picks, worst, margins = int(last.value), [], 0.0, []
    for step in range(steps):
        rc, lg = s.decode_step(tok)
        orc_rc, ref = o.decode_step(kv, tok)
        assert rc == 0 and orc_rc == 0
        worst = max(worst, rel_l2(lg, ref))
        top2 = np.sort(ref)[-2:]
        margins.append(float(top2[1] - top2[0]))
        tok = orc.argmax(ref)[1]
        assert last_argmax(lg) == tok, step
        picks.append(tok)
        if step % 16 == 15:
            print(f"step {step + 1}: worst rel L2 {worst:.2e}", flush=True)
    assert worst < TOL, worst
    assert len(set(picks)) > 32, picks  # the stream moves
    print("top-2 margins: min %.3g median %.3g" % (min(margins), float(np.median(margins))))
    s.close()
    s2 = g.session(max_seq)
    rc, _ = s2.prefill(ids, want_logits=False)
    assert rc == 0
    rc, toks = s2.decode_greedy(int(last.value), steps)
    assert rc == 0
    assert toks.tolist() == picks
    s2.close()
    g.close()
    o.close()
