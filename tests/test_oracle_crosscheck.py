"""Pins for what the reference KATs leave open (see the oracle header):

* dequant: the C oracle and an independent numpy restatement agree bit for bit
  on random and edge blocks (Q4_K high scale bits and dmin, Q6_K u8 scales and
  ql/qh order, Q8_K scales, f16 specials);
* matmul_t: the 8-lane FMA + hsum tree order (a case where order changes the
  sum), the scalar tail, and agreement with float64;
* rms_norm / softmax / swiglu / rope against float64 closed forms, rope at
  position 0 is the identity;
* the model code against a float64 brute-force forward, and invariants
  (prefill([t]) == decode_step(t) on an empty cache, FAITHFUL == FAST,
  decode invariance under a permutation of cached rows).
"""
from __future__ import annotations

import numpy as np
import pytest

from inferox_amd import synth
from inferox_amd.gguf_writer import F16, F32, Q4_0, Q4_K, Q6_K, Q8_0, Q8_K, GGUFWriter
from oracle import binding as orc
from oracle import numpy_ref
from tests.conftest import rel_l2

BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292)}


def _same(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    both_nan = np.isnan(a) & np.isnan(b)
    eq = (a.view(np.uint32) == b.view(np.uint32)) | both_nan
    return bool(np.all(eq))


def _random_raw(t, nblocks, rng, special_d=False):
    be, bb = BLOCK[t]
    raw = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    if not special_d:  # keep d/dmin finite and positive as a real file would
        nd = 2 if t in (Q4_K, Q8_K) else 1
        d = rng.uniform(1e-4, 1e-1, size=(nblocks, nd)).astype("<f2")
        raw[:, : 2 * nd] = d.view(np.uint8).reshape(nblocks, 2 * nd)
    return raw.reshape(-1), be * nblocks


@pytest.mark.parametrize("t", [Q4_0, Q8_0, Q4_K, Q6_K, Q8_K])
def test_dequant_c_vs_numpy_random(t):
    rng = np.random.default_rng(t)
    for special in (False, True):  # True: every bit pattern of d/dmin, incl. inf/NaN/subnormal
        raw, n = _random_raw(t, 4096, rng, special_d=special)
        rc, c = orc.dequantize(t, raw, n)
        assert rc == 0
        assert _same(c, numpy_ref.dequant(t, raw))


def test_dequant_f16_f32_all_values():
    raw = np.arange(65536, dtype=np.uint16).view(np.uint8)
    rc, c = orc.dequantize(F16, raw, 65536)
    assert rc == 0
    assert _same(c, numpy_ref.dequant(F16, raw))
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2**32, size=10000, dtype=np.uint64).astype(np.uint32)
    rc, c = orc.dequantize(F32, bits.view(np.uint8), 10000)
    assert rc == 0 and np.array_equal(c.view(np.uint32), bits)


def test_q4k_scale_bits_every_value():
    """All 64 values of each 6-bit scale and min, in all 8 groups, against a
    direct per-element evaluation of src/gguf/dequant.rs:141-158."""
    blocks = []
    for v in range(64):
        s = np.zeros(12, np.uint8)
        for g in range(4):
            s[g] = (v & 63) | ((v >> 4) << 6)          # sc low 6 bits (g<4), top bits feed g+4
            s[g + 4] = ((63 - v) & 63) | (((63 - v) >> 4) << 6)
            s[g + 8] = (v & 15) | (((63 - v) & 15) << 4)
        qs = np.arange(128, dtype=np.uint8) * 37
        blocks.append(np.concatenate([np.frombuffer(np.array([0.5, 0.25], "<f2").tobytes(), np.uint8), s, qs]))
    raw = np.concatenate(blocks)
    rc, c = orc.dequantize(Q4_K, raw, 256 * 64)
    assert rc == 0
    exp = np.empty(256 * 64, np.float32)
    for b in range(64):
        blk = raw[b * 144:(b + 1) * 144]
        s = blk[4:16].astype(np.uint32)
        for g in range(8):
            if g < 4:
                sc, mn = s[g] & 63, s[g + 4] & 63
            else:
                sc = (s[g + 4] & 15) | ((s[g - 4] >> 6) << 4)
                mn = (s[g + 4] >> 4) | ((s[g] >> 6) << 4)
            dall = np.float32(0.5) * np.float32(sc)
            dm = np.float32(0.25) * np.float32(mn)
            for l in range(32):
                byte = int(blk[16 + 16 * g + l // 2])
                q = (byte >> 4) if l & 1 else (byte & 15)
                exp[b * 256 + 32 * g + l] = dall * np.float32(q) - dm
    assert _same(c, exp)


def test_q6k_scales_are_unsigned():
    """A scale byte of 0xF0 (-16 as i8) acts as 240 (src/gguf/dequant.rs:195 reads u8)."""
    raw = bytearray(np.array([1.0], "<f2").tobytes()) + bytes([0xF0] * 16) + bytes([0x11] * 128) + bytes(64)
    rc, c = orc.dequantize(Q6_K, np.frombuffer(bytes(raw), np.uint8), 256)
    assert rc == 0
    np.testing.assert_array_equal(c, np.full(256, 240.0 * (1 - 32), np.float32))


def test_matmul_t_lane_order():
    """k=16: lane r accumulates products l=r and l=r+8; the tree is
    ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)).  Values chosen so that a sequential
    sum gives a different float32 result."""
    a = np.zeros(16, np.float32)
    a[0] = 2.0**24                   # sequential: the three 1.0 below are lost against 2^24
    a[1] = a[2] = a[3] = 1.0
    a[15] = -2.0**24                 # lane 7; the tree keeps two of the 1.0 -> 2.0
    b = np.ones(16, np.float32)
    c = orc.matmul_t(a, b, 1, 1, 16)[0]
    lanes = np.zeros(8, np.float32)
    for l in range(16):
        lanes[l % 8] = np.float32(lanes[l % 8] + a[l] * b[l])
    s = [np.float32(lanes[r] + lanes[r + 4]) for r in range(4)]
    tree = np.float32(np.float32(s[0] + s[1]) + np.float32(s[2] + s[3]))
    seq = np.float32(0)
    for l in range(16):
        seq = np.float32(seq + a[l] * b[l])
    assert c == tree and tree != seq


def test_matmul_t_vs_float64_and_tail():
    rng = np.random.default_rng(1)
    for (m, n, k) in [(1, 37, 29), (3, 17, 64), (2, 5, 7), (1, 64, 4096)]:
        a = rng.standard_normal(m * k).astype(np.float32)
        b = rng.standard_normal(n * k).astype(np.float32)
        c = orc.matmul_t(a, b, m, n, k)
        ref = a.reshape(m, k).astype(np.float64) @ b.reshape(n, k).astype(np.float64).T
        assert rel_l2(c, ref.reshape(-1)) < 1e-6
        # small integers: every partial sum is exact, all orders agree
        ai = rng.integers(-8, 8, m * k).astype(np.float32)
        bi = rng.integers(-8, 8, n * k).astype(np.float32)
        exact = (ai.reshape(m, k).astype(np.int64) @ bi.reshape(n, k).astype(np.int64).T).reshape(-1)
        np.testing.assert_array_equal(orc.matmul_t(ai, bi, m, n, k), exact.astype(np.float32))
        np.testing.assert_array_equal(orc.matmul_t(ai, bi, m, n, k, scalar=True), exact.astype(np.float32))


def test_small_ops_vs_float64():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 96)).astype(np.float32) * 30
    w = (1 + 0.02 * rng.standard_normal(96)).astype(np.float32)
    got = orc.rms_norm_rows(x.reshape(-1), w, 1e-5, rows=5).reshape(5, 96)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-5) * w
    assert rel_l2(got, ref) < 1e-6
    s = orc.softmax_rows(x.reshape(-1), 5, 96).reshape(5, 96)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    assert rel_l2(s, e / e.sum(axis=1, keepdims=True)) < 1e-5
    g, u = x[0], x[1]
    g64 = g.astype(np.float64)
    ref = g64 / (1 + np.exp(-np.clip(g64, -80, 80))) * u
    assert rel_l2(orc.swiglu(g, u), ref) < 1e-6


def test_rope_identity_at_zero_and_rotation():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(3 * 4 * 16).astype(np.float32)
    # position 0: cos=1, sin=0 exactly -> bit-identical (decode's rope, Q1)
    y = orc.rope(x[: 4 * 16], 1, 4, 16, 16, 10000.0)
    np.testing.assert_array_equal(y, x[: 4 * 16])
    # positions 0..2 against a float64 rotation; pair norms are preserved
    y = orc.rope(x, 3, 4, 16, 12, 500000.0).reshape(3, 4, 16)
    xr = x.reshape(3, 4, 16).astype(np.float64)
    i = np.arange(0, 12, 2)
    ang = np.arange(3)[:, None] * (1.0 / 500000.0 ** (i / 12))[None, :]
    a, b = xr[:, :, i], xr[:, :, i + 1]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    np.testing.assert_allclose(y[:, :, i], a * c - b * s, atol=1e-5)
    np.testing.assert_allclose(y[:, :, i + 1], a * s + b * c, atol=1e-5)
    np.testing.assert_array_equal(y[:, :, 12:], x.reshape(3, 4, 16)[:, :, 12:])


def _small_f32_model(path, seed=7, dim=64, ffn=96, layers=2, heads=4, kv_heads=2, vocab=50, scale=0.15):
    rng = np.random.default_rng(seed)
    hd = dim // heads
    w = GGUFWriter()
    w.add_string("general.architecture", "llama")
    for k, v in [("vocab_size", vocab), ("embedding_length", dim), ("block_count", layers),
                 ("attention.head_count", heads), ("attention.head_count_kv", kv_heads),
                 ("feed_forward_length", ffn), ("context_length", 64)]:
        w.add_u32("llama." + k, v)
    w.add_f32("llama.rope.freq_base", 10000.0)
    tensors = {}

    def add(name, rows, cols, norm=False):
        if norm:
            arr = (1 + 0.05 * rng.standard_normal(cols)).astype(np.float32)
            w.tensor_f32(name, [cols], arr)
        else:
            arr = (scale * rng.standard_normal((rows, cols))).astype(np.float32)
            w.tensor_f32(name, [cols, rows], arr.reshape(-1))
        tensors[name] = arr.astype(np.float64)

    add("token_embd.weight", vocab, dim)
    add("output_norm.weight", 1, dim, norm=True)
    add("output.weight", vocab, dim)
    for l in range(layers):
        p = f"blk.{l}."
        add(p + "attn_norm.weight", 1, dim, norm=True)
        add(p + "attn_q.weight", dim, dim)
        add(p + "attn_k.weight", kv_heads * hd, dim)
        add(p + "attn_v.weight", kv_heads * hd, dim)
        add(p + "attn_output.weight", dim, dim)
        add(p + "ffn_norm.weight", 1, dim, norm=True)
        add(p + "ffn_gate.weight", ffn, dim)
        add(p + "ffn_up.weight", ffn, dim)
        add(p + "ffn_down.weight", dim, ffn)
    w.write(path)
    cfg = dict(dim=dim, n_heads=heads, n_kv_heads=kv_heads, head_dim=hd, rope_dim=hd, rope_base=10000.0,
               eps=1e-5, n_layers=layers)
    return tensors, cfg


def test_model_vs_float64_bruteforce(tmp_path):
    p = str(tmp_path / "s.gguf")
    weights, cfg = _small_f32_model(p)
    m = orc.Model(p)
    ids = [3, 17, 42, 8, 0, 49, 21]
    rc, pre = m.prefill(m.kv(64), ids, mode=orc.MODE_FAITHFUL)
    assert rc == 0
    ref = numpy_ref.forward64(weights, cfg, ids, causal=True)
    assert rel_l2(pre, ref) < 1e-5
    rc, fwd = m.forward(ids, mode=orc.MODE_FAITHFUL)
    assert rc == 0
    assert rel_l2(fwd, numpy_ref.forward64(weights, cfg, ids, causal=False)) < 1e-5
    # decode: q and k rotated at position 0 (Q1) over the whole cache
    kv = m.kv(64)
    rows = []
    for t in ids:
        rc, lg = m.decode_step(kv, t, mode=orc.MODE_FAITHFUL)
        assert rc == 0
        rows.append(lg)
    ref = numpy_ref.forward64(weights, cfg, ids, causal=True, positions=[0] * len(ids))
    assert rel_l2(np.stack(rows), ref) < 1e-5


def test_model_invariants(tiny_path, tiny_prompt):
    m = orc.Model(tiny_path)
    tok = int(tiny_prompt[0])
    # prefill([t]) is decode_step(t) on an empty cache: same ops, m=1, position 0
    rc, pre = m.prefill(m.kv(8), [tok], mode=orc.MODE_FAST)
    rc2, dec = m.decode_step(m.kv(8), tok, mode=orc.MODE_FAST)
    assert rc == rc2 == 0
    np.testing.assert_array_equal(pre[0], dec)
    # FAITHFUL (per-step full dequant) and FAST (row-fused, threaded) agree bit for bit
    kv_a, kv_b = m.kv(32), m.kv(32)
    for t in tiny_prompt[:4]:
        ra, la = m.decode_step(kv_a, int(t), mode=orc.MODE_FAITHFUL)
        rb, lb = m.decode_step(kv_b, int(t), mode=orc.MODE_FAST)
        assert ra == rb == 0
        np.testing.assert_array_equal(la, lb)
    # decode attention carries no position (Q1): permuting cached rows changes
    # only the summation order
    c = m.cfg
    kvd = c.n_kv_heads * c.head_dim
    k, v = kv_b.export(4)
    perm = [2, 0, 3, 1]
    kp = k.reshape(c.n_layers, 4, kvd)[:, perm].reshape(-1)
    vp = v.reshape(c.n_layers, 4, kvd)[:, perm].reshape(-1)
    kv_p = m.kv(32)
    assert kv_p.import_(kp, vp, 4) == 0
    kv_c = m.kv(32)
    assert kv_c.import_(k, v, 4) == 0
    _, l1 = m.decode_step(kv_c, 5, mode=orc.MODE_FAST)
    _, l2 = m.decode_step(kv_p, 5, mode=orc.MODE_FAST)
    assert rel_l2(l2, l1) < 1e-5


def test_model_error_paths(tiny_path):
    m = orc.Model(tiny_path)
    kv = m.kv(2)
    assert m.decode_step(kv, m.vocab)[0] == 10          # InvalidTensorIndex
    assert m.decode_step(kv, 1)[0] == 0
    assert m.decode_step(kv, 1)[0] == 0
    assert m.decode_step(kv, 1)[0] == 21                # KV full (the reference panics)
    assert m.prefill(m.kv(4), [1, m.vocab])[0] == 10
    assert m.prefill(m.kv(4), [1, 2, 3, 4, 5])[0] == 21


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q6_K])
def test_fast_dequant_equals_restatement(t):
    """The FAST mode's vectorised dequantization (used only by FAST linear
    layers) gives the restatement's bits on random blocks, every bit pattern
    of d/dmin included."""
    rng = np.random.default_rng(100 + t)
    for special in (False, True):
        raw, n = _random_raw(t, 8192, rng, special_d=special)
        rc, ref = orc.dequantize(t, raw, n)
        rc2, fast = orc.dequantize_fast(t, raw, n)
        assert rc == rc2 == 0
        assert _same(fast, ref)


@pytest.fixture(scope="module")
def kquant_small(tmp_path_factory):
    """A Q4_K/Q6_K GQA model small enough for FAITHFUL prefill (head_dim 64,
    vocab not a multiple of the 64-row weight blocks)."""
    p = str(tmp_path_factory.mktemp("kq") / "kq.gguf")
    spec = synth.reduced(synth.LLAMA3_8B, dim=512, ffn=768, n_layers=2, n_heads=8, n_kv_heads=2, vocab=1003,
                         ctx=64)
    synth.write_llama(p, spec, seed=77)
    return p


@pytest.mark.parametrize("n", [1, 5, 13])
def test_fast_prefill_equals_faithful(tiny_path, tiny_prompt, kquant_small, n):
    """FAST prefill/forward (register-tiled matmul_t, head-parallel attention
    with 8-key score lanes) equal FAITHFUL (the reference's loops) bit for bit:
    row counts off the 3-row tiles, head dims 48 (off the 8-lane p.V) and 64,
    causal and full attention, and the cache rows written."""
    ids = np.concatenate([tiny_prompt, tiny_prompt])[:n]
    for path in (tiny_path, kquant_small):
        m = orc.Model(path)
        ids_m = ids % m.vocab
        kv_a, kv_b = m.kv(32), m.kv(32)
        ra, la = m.prefill(kv_a, ids_m, mode=orc.MODE_FAITHFUL)
        rb, lb = m.prefill(kv_b, ids_m, mode=orc.MODE_FAST)
        assert ra == rb == 0
        np.testing.assert_array_equal(la, lb)
        ka, va = kv_a.export(n)
        kb, vb = kv_b.export(n)
        np.testing.assert_array_equal(ka, kb)
        np.testing.assert_array_equal(va, vb)
        ra, fa = m.forward(ids_m, mode=orc.MODE_FAITHFUL)
        rb, fb = m.forward(ids_m, mode=orc.MODE_FAST)
        assert ra == rb == 0
        np.testing.assert_array_equal(fa, fb)
        # decode after the chunk: the head-parallel decode attention too
        ra, da = m.decode_step(kv_a, 7, mode=orc.MODE_FAITHFUL)
        rb, db = m.decode_step(kv_b, 7, mode=orc.MODE_FAST)
        assert ra == rb == 0
        np.testing.assert_array_equal(da, db)
        # prefill_rows: the listed rows of prefill's logits, in order
        rows = [n - 1, 0] if n > 1 else [0]
        rc, lr = m.prefill_rows(m.kv(32), ids_m, rows)
        assert rc == 0
        np.testing.assert_array_equal(lr, lb[rows])
        m.close()
