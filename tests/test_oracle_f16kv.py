"""The oracle's f16-KV mode (no reference counterpart; the checker of
ifx_session_create_kv(..., IFX_KV_F16)), pinned on the CPU:

* orc_round_f16 equals numpy's float32 -> float16 -> float32 conversion (an
  independent implementation that rounds to nearest even) on every binary16
  value, on every midpoint between neighbouring binary16 values (the ties),
  around the overflow threshold and the subnormal range, and on random floats;
* a decode with the mode on stores layer 0's rows as exactly the rounding of
  the f32 cache's layer-0 rows (layer 0 does not depend on the cache), every
  stored row is a binary16 value, and the logits stay near the f32 run's.
"""
from __future__ import annotations

import numpy as np

from inferox_amd import synth
from oracle import binding as orc
from tests.conftest import rel_l2


def np_f16(x):
    with np.errstate(over="ignore"):
        return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def test_round_f16_every_half_and_midpoint():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    fin = h[np.isfinite(h)].astype(np.float32)
    np.testing.assert_array_equal(orc.round_f16(fin), fin)
    # midpoints between neighbouring non-negative finite halves, both signs
    pos = np.sort(fin[fin >= 0].astype(np.float64))
    pos = np.unique(pos)
    mid = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)  # exact in float32 (one more bit)
    assert np.all(mid.astype(np.float64) == (pos[:-1] + pos[1:]) / 2)
    for m in (mid, -mid):
        np.testing.assert_array_equal(orc.round_f16(m), np_f16(m))


def test_round_f16_edges_and_random():
    edges = np.array([65504.0, 65519.99, 65520.0, 65536.0, 1e30, -65520.0, 2.0 ** -24, 2.0 ** -25,
                      np.nextafter(np.float32(2.0 ** -25), np.float32(1)), 3 * 2.0 ** -26, 2.0 ** -14,
                      np.nextafter(np.float32(2.0 ** -14), np.float32(0)), 1e-30, 0.0, -0.0, np.inf, -np.inf],
                     np.float32)
    r = orc.round_f16(edges)
    np.testing.assert_array_equal(r, np_f16(edges))
    assert np.signbit(r[14])
    assert np.isnan(orc.round_f16(np.array([np.nan], np.float32))[0])
    rng = np.random.default_rng(16)
    x = (rng.standard_normal(40000) * 10.0 ** rng.uniform(-10, 6, 40000)).astype(np.float32)
    np.testing.assert_array_equal(orc.round_f16(x), np_f16(x))


def test_f16_cache_mode_rows(tmp_path):
    spec = synth.reduced(synth.TINY, n_layers=2, ctx=64)
    p = str(tmp_path / "t2.gguf")
    synth.write_llama(p, spec, seed=9)
    o = orc.Model(p)
    c = o.cfg
    ids = synth.token_ids(12, spec.vocab, seed=10)
    kv16, kv32 = o.kv(64, f16=True), o.kv(64)
    worst = 0.0
    for t in ids:
        rc16, lg16 = o.decode_step(kv16, int(t))
        rc32, lg32 = o.decode_step(kv32, int(t))
        assert rc16 == 0 and rc32 == 0
        worst = max(worst, rel_l2(lg16, lg32))
    assert 0.0 < worst < 2e-2
    n, kvd = len(ids), c.n_kv_heads * c.head_dim
    k16, v16 = kv16.export(n)
    k32, v32 = kv32.export(n)
    np.testing.assert_array_equal(k16, np_f16(k16))
    np.testing.assert_array_equal(v16, np_f16(v16))
    np.testing.assert_array_equal(k16[: n * kvd], np_f16(k32[: n * kvd]))   # layer 0
    np.testing.assert_array_equal(v16[: n * kvd], np_f16(v32[: n * kvd]))
    assert not np.array_equal(k16[n * kvd:], np_f16(k32[n * kvd:]))         # layer 1 saw rounded rows
    # a prefill chunk: the same rows as the token path's rounding of layer 0
    kvp = o.kv(64, f16=True)
    rc, _ = o.prefill(kvp, ids)
    assert rc == 0
    kp, vp = kvp.export(n)
    np.testing.assert_array_equal(kp, np_f16(kp))
    o.close()
