"""The decode step's and the batched prefill's attention kernels against the
oracle's attention loops, through ifx_ops_attention_decode /
ifx_ops_attention_decode_o / ifx_ops_attention_prefill.

Decode (src/model/forward.rs:383-414): every head dim, query-group size and
cache type the kernels are instantiated for, lengths on both sides of the
64-row chunk boundaries and past one 256-chunk merge batch, and every merge
path (the separate merge, the merge inside the O projection at each of its
record bounds, with records past the bound read in its loop).  Prefill
(src/model/forward.rs:255-303, forward's non-causal :104-156): chunks of 1 to
2048 rows at a cache offset, causal and not.

Bar: per head (and per prefill row), |o - o_oracle|_2 <= TOL * sum_t p_t
|v_t|_2 (p: the float64 softmax weights) — the size the rounding of any f32
evaluation is measured against; the oracle itself is within 7e-7 of float64
at every case here (tests/test_oracle_attention.py).  Each case first checks
on the oracle side that the test can see what it guards: removing one 64-row
chunk (decode) or dropping the causal mask (prefill) moves the float64
output by at least 100 x TOL (tests/attn_cases.py: every chunk for `flat`
inputs, the median chunk for `spread`, the aligned rows' chunks for `onehot`
and `tie`).  Cache rows past the attended ones hold NaN, so a read of them
shows.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from inferox_amd import _native, synth
from inferox_amd.gguf_writer import Q4_K, Q6_K
from oracle import binding as orc
from tests import attn_cases as ac
from tests.gpu_util import Dev, Tensor

pytestmark = pytest.mark.gpu

TOL = 5e-6      # decode attention, per head
TOL_O = 2e-5    # attention + O projection, per row (the GEMV's own 1e-5 plus the attention's)
TOL_PRE = 1e-5  # prefill attention (fp16 hi/lo operand pairs), per row and head
GUARD = 100.0

LENGTHS = (1, 63, 64, 65, 2048, 3072, 3073, 8193, 16385, 20000)
KV_F32, KV_F16 = 0, 1


def head_major(x, n, n_kv, hd, max_seq, f16):
    """Reference rows [n][n_kv*hd] as the device cache [n_kv][max_seq][hd];
    rows n.. hold NaN."""
    c = np.full((n_kv, max_seq, hd), np.nan, np.float32)
    c[:, :n] = np.asarray(x, np.float32).reshape(n, n_kv, hd).transpose(1, 0, 2)
    return c.astype(np.float16) if f16 else c


def run_decode(q, k, v, n, nh, nkv, hd, f16, slack=37):
    max_seq = n + slack
    dq = Dev.of(np.asarray(q, np.float32))
    dk = Dev.of(head_major(k, n, nkv, hd, max_seq, f16))
    dv = Dev.of(head_major(v, n, nkv, hd, max_seq, f16))
    do = Dev(nh * hd * 4)
    rc = _native.lib().ifx_ops_attention_decode(dq.ptr, dk.ptr, dv.ptr, KV_F16 if f16 else KV_F32, max_seq, n, nh,
                                                nkv, hd, do.ptr, None)
    assert rc == 0, _native.lib().ifx_last_error()
    return do.get(np.float32, nh * hd).reshape(nh, hd)


def check_decode(n, nh, nkv, hd, kind, f16, seed):
    print(f"decode attention n={n} heads={nh}/{nkv} hd={hd} {kind} f16={f16} seed={seed}", flush=True)
    q, k, v, _ = ac.decode_case(n, nh, nkv, hd, kind, seed, f16=f16)
    o64, scale, _ = ac.eval64(q, k, v, nh, nkv, hd)
    g = ac.guard_decode(kind, ac.chunk_removal(q, k, v, nh, nkv, hd))
    assert g >= GUARD * TOL, (n, kind, g)
    ref = orc.attention_decode(q, k, v, n, nh, nkv, hd).reshape(nh, hd)
    got = run_decode(q, k, v, n, nh, nkv, hd, f16)
    err = np.linalg.norm(got.astype(np.float64) - ref, axis=1) / scale
    assert np.isfinite(got).all()
    assert err.max() <= TOL, (n, kind, float(err.max()))
    return float(err.max())


@pytest.mark.parametrize("hd,group", [(48, 1), (48, 4), (48, 8), (128, 1), (128, 4), (128, 8), (64, 4), (64, 1)])
@pytest.mark.parametrize("kv_f16", [False, True])
@pytest.mark.parametrize("kind", ["flat", "spread", "onehot", "tie"])
def test_decode_attention(hd, group, kv_f16, kind):
    """Two kv heads of `group` query heads; the decode kernels of each head
    dim and group (templated for 128 x {1, 4, 8} and 64 x {1, 4}, generic
    otherwise)."""
    lengths = LENGTHS if kind in ("flat", "spread") else (1, 65, 3073, 20000)
    if hd == 64:
        lengths = (1, 65, 3073, 16385)
    worst = 0.0
    for n in lengths:
        worst = max(worst, check_decode(n, 2 * group, 2, hd, kind, kv_f16, seed=n * 31 + hd + group))
    print(f"worst {worst:.2e} of {TOL:.0e}")


@pytest.mark.parametrize("group,n", [(4, 2048), (4, 2049), (4, 4097), (8, 8192), (8, 8193), (8, 20000)])
def test_decode_attention_model_shapes(group, n):
    """The 8B (32/8 heads) and 70B (64/8) attention at their decode lengths:
    the chunk grid ordered kv head fastest (at most two workgroups per CU) and
    chunk fastest (larger grids)."""
    for kind in ("flat", "spread"):
        for f16 in (False, True):
            check_decode(n, 8 * group, 8, 128, kind, f16, seed=n + group)


def _centred_matrix(t, rows, cols, seed):
    raw = synth.random_centred_blocks(t, rows * cols, cols, "o", seed)
    rc, w = orc.dequantize(t, raw, rows * cols)
    assert rc == 0
    return raw, w.reshape(rows, cols)


def identity_blocks(t, dim):
    """The [dim x dim] identity as Q4_K or Q6_K blocks, built from the
    reference's element formulas (src/gguf/dequant.rs:133-197): Q4_K d = 1,
    dmin = 0, every 6-bit scale 1, nibble 1 on the diagonal and 0 elsewhere;
    Q6_K d = 1, u8 scales 1, q = 33 on the diagonal and 32 elsewhere."""
    nb = dim // 256
    if t == Q4_K:
        blk = np.zeros((dim, nb, 144), np.uint8)
        blk[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        blk[:, :, 4:8] = 1
        blk[:, :, 12:16] = 1
        for i in range(dim):
            e = i % 256
            g, l = e // 32, e % 32
            blk[i, i // 256, 16 + 16 * g + l // 2] = 1 << (4 * (l & 1))
    else:
        blk = np.zeros((dim, nb, 210), np.uint8)
        blk[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        blk[:, :, 2:18] = 1
        blk[:, :, 146:210] = 0xAA  # every 2-bit high field 2: q = 32 + low nibble
        for i in range(dim):
            j = i % 256
            blk[i, i // 256, 18 + j // 2] = 1 << (4 * (j & 1))
    raw = blk.reshape(-1)
    rc, w = orc.dequantize(t, raw, dim * dim)
    assert rc == 0 and np.array_equal(w.reshape(dim, dim), np.eye(dim, dtype=np.float32))
    return raw


def merged_o_lengths(bound):
    if bound == 0:
        return (65, 2048, 3073, 20000)
    return (1, 64, bound * 64 - 37, bound * 64 + 100, 20000)


def run_decode_o(q, k, v, n, nh, nkv, hd, wt, h0, bound):
    max_seq = n + 29
    dq = Dev.of(q)
    dk = Dev.of(head_major(k, n, nkv, hd, max_seq, False))
    dv = Dev.of(head_major(v, n, nkv, hd, max_seq, False))
    dh = Dev.of(h0)
    rc = _native.lib().ifx_ops_attention_decode_o(dq.ptr, dk.ptr, dv.ptr, KV_F32, max_seq, n, nh, nkv, hd, wt.h,
                                                  dh.ptr, bound, None, None)
    assert rc == 0, _native.lib().ifx_last_error()
    return dh.get(np.float32, h0.size).astype(np.float64)


@pytest.mark.parametrize("group", [4, 8])
def test_attention_merged_o_exact(group):
    """Attention + O projection + residual (src/model/forward.rs:383-419) as
    the decode step runs it: the records merged in the O launch's prologue at
    each bound (8..48 records loaded up front, the rest in its loop; 20000 rows
    is 313 records), and the separate merge followed by the K-split O launch
    (bound 0).  W_o is the identity as Q4_K blocks and h starts at 0, so the
    launch's output is the merged attention itself (the O launch carries x as
    22-bit fixed point: 2^-22 of its 32-element group's largest magnitude),
    held to the decode attention's bar with the chunk guard.  (A Q6_K identity
    would not do: that kernel forms (q - 32) . x as q . x - 32 sum(x), whose
    fixed-point rounding the identity's all-32 rows multiply by 32.  The merge
    is the same code for both weight types; the dense test below covers Q6_K.)"""
    nkv, hd = 8, 128
    nh, dim = nkv * group, nkv * group * hd
    eye = Tensor(Q4_K, identity_blocks(Q4_K, dim), dim, dim)
    for bound in (0, 8, 16, 24, 32, 40, 48):
        for n in merged_o_lengths(bound):
            print(f"attention+O identity group={group} bound={bound} n={n}", flush=True)
            q, k, v, _ = ac.decode_case(n, nh, nkv, hd, "flat", seed=n + 17 * bound + group)
            _, scale, _ = ac.eval64(q, k, v, nh, nkv, hd)
            assert ac.guard_decode("flat", ac.chunk_removal(q, k, v, nh, nkv, hd)) >= GUARD * TOL
            ra = orc.attention_decode(q, k, v, n, nh, nkv, hd).astype(np.float64).reshape(nh, hd)
            got = run_decode_o(q, k, v, n, nh, nkv, hd, eye, np.zeros(dim, np.float32), bound).reshape(nh, hd)
            gmax = np.abs(ra).reshape(nh, hd // 32, 32).max(2)
            qerr = np.linalg.norm(np.repeat(gmax, 32, axis=1), axis=1) * 2.0 ** -21
            err = np.linalg.norm(got - ra, axis=1)
            assert (err <= TOL * scale + qerr).all(), (bound, n, float((err / (TOL * scale + qerr)).max()))


@pytest.mark.parametrize("group,wtype", [(4, Q4_K), (8, Q4_K), (4, Q6_K), (8, Q6_K)])
def test_attention_merged_o_dense(group, wtype):
    """The same launches with a dense centred W_o and a random residual, at
    one length per merge bound: every row within the GEMV's bar,
    TOL_O * sum_j |W_ij| sum_t p_t |v_tj|."""
    nkv, hd = 8, 128
    nh, dim = nkv * group, nkv * group * hd
    raw, w = _centred_matrix(wtype, dim, dim, seed=700 + group + wtype)
    dense = Tensor(wtype, raw, dim, dim)
    w64 = w.astype(np.float64)
    wabs = np.abs(w64)
    rng = np.random.default_rng(group)
    for bound in (0, 8, 16, 24, 32, 40, 48):
        n = merged_o_lengths(bound)[-2]
        print(f"attention+O dense group={group} type={wtype} bound={bound} n={n}", flush=True)
        q, k, v, _ = ac.decode_case(n, nh, nkv, hd, "flat", seed=n + 5 * bound)
        _, _, amag = ac.eval64(q, k, v, nh, nkv, hd)
        h0 = rng.standard_normal(dim).astype(np.float32)
        ref = h0.astype(np.float64) + w64 @ orc.attention_decode(q, k, v, n, nh, nkv, hd).astype(np.float64)
        tol = TOL_O * (wabs @ amag.reshape(-1)) + 2.0 ** -23 * (np.abs(h0) + np.abs(ref))
        got = run_decode_o(q, k, v, n, nh, nkv, hd, dense, h0, bound)
        bad = np.abs(got - ref) > tol
        assert not bad.any(), (bound, n, int(bad.sum()), float((np.abs(got - ref) / tol).max()))


def test_attention_merged_o_refuses_other_shapes():
    """The fused form needs the 8-kv-head, head-dim-128 shapes; others are refused."""
    raw, _ = _centred_matrix(Q4_K, 1024, 1024, seed=3)
    wt = Tensor(Q4_K, raw, 1024, 1024)
    q, k, v, _ = ac.decode_case(100, 8, 2, 128, "flat", seed=1)
    dq, dk, dv = Dev.of(q), Dev.of(head_major(k, 100, 2, 128, 128, False)), Dev.of(head_major(v, 100, 2, 128, 128, False))
    dh = Dev(1024 * 4)
    rc = _native.lib().ifx_ops_attention_decode_o(dq.ptr, dk.ptr, dv.ptr, KV_F32, 128, 100, 8, 2, 128, wt.h,
                                                  dh.ptr, 8, None, None)
    assert rc == 20  # IFX_E_INVALID_ARG
    rc = _native.lib().ifx_ops_attention_decode(dq.ptr, dk.ptr, dv.ptr, KV_F32, 128, 129, 8, 2, 128, dh.ptr, None)
    assert rc == 20  # more rows than the cache holds


# ------------------------------------------------------------------ prefill

def prefill_case(n, nh, nkv, hd, seed, f16):
    rng = np.random.default_rng(seed)
    q = (0.5 * rng.standard_normal((n, nh * hd))).astype(np.float32)
    k = rng.standard_normal((n, nkv * hd)).astype(np.float32)
    off = rng.standard_normal(((n + 63) // 64, nkv * hd)).astype(np.float32)
    v = (rng.standard_normal((n, nkv * hd)) + 3.0 * np.repeat(off, 64, axis=0)[:n]).astype(np.float32)
    if f16:
        k, v = ac.round_f16(k), ac.round_f16(v)
    return q, k, v


def prefill64(q, k, v, rows, nh, nkv, hd, causal):
    """float64 outputs [len(rows)][nh][hd] and scales [len(rows)][nh] of the given query rows."""
    n = k.shape[0]
    group = nh // nkv
    q3 = q.astype(np.float64).reshape(n, nh, hd)
    k3 = k.astype(np.float64).reshape(n, nkv, hd)
    v3 = v.astype(np.float64).reshape(n, nkv, hd)
    out = np.empty((len(rows), nh, hd))
    scale = np.empty((len(rows), nh))
    for i, p in enumerate(rows):
        end = p + 1 if causal else n
        for h in range(nh):
            s = k3[:end, h // group] @ q3[p, h] / np.sqrt(hd)
            e = np.exp(s - s.max())
            pr = e / e.sum()
            out[i, h] = pr @ v3[:end, h // group]
            scale[i, h] = pr @ np.linalg.norm(v3[:end, h // group], axis=1)
    return out, scale


PREFILL_SIZES = ((1, 0), (63, 5), (64, 0), (65, 37), (129, 0), (300, 11), (512, 0))


@pytest.mark.parametrize("hd,group", [(48, 1), (64, 4), (96, 2), (128, 4), (128, 8)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("kv_f16", [False, True])
def test_prefill_attention(hd, group, causal, kv_f16):
    nkv = 2
    nh = nkv * group
    sizes = PREFILL_SIZES + (((2048, 0),) if (hd, group) == (128, 4) and causal else ())
    for n, row0 in sizes:
        print(f"prefill attention n={n} row0={row0} heads={nh}/{nkv} hd={hd} causal={causal} f16={kv_f16}",
              flush=True)
        q, k, v = prefill_case(n, nh, nkv, hd, seed=n + hd + group, f16=kv_f16)
        rows = sorted(set(np.random.default_rng(n).choice(n, min(n, 24), replace=False).tolist()) | {0, n - 1})
        o64, scale = prefill64(q, k, v, rows, nh, nkv, hd, causal)
        if n > 1:
            # the guard: the other masking moves the median sampled row by >= 100 x TOL_PRE
            other, _ = prefill64(q, k, v, rows[:-1], nh, nkv, hd, not causal)
            moved = np.linalg.norm(other - o64[:-1], axis=2) / scale[:-1]
            assert np.median(moved.max(1)) >= GUARD * TOL_PRE, (n, float(np.median(moved.max(1))))
            # and every 64-key block matters to the last row of a full chunk
            last = q[n - 1]
            rem = ac.chunk_removal(last, k, v, nh, nkv, hd)
            assert rem.min() >= GUARD * TOL_PRE, (n, float(rem.min()))
        ref = orc.attention_batch(q, k, v, n, nh, nkv, hd, causal=causal).reshape(n, nh, hd)
        max_seq = row0 + n + 19
        ck = np.full((max_seq, nkv * hd), np.nan, np.float32)
        cv = np.full((max_seq, nkv * hd), np.nan, np.float32)
        ck[row0:row0 + n], cv[row0:row0 + n] = k, v
        hm = lambda x: np.ascontiguousarray(x.reshape(max_seq, nkv, hd).transpose(1, 0, 2))  # noqa: E731
        dk = Dev.of(hm(ck).astype(np.float16) if kv_f16 else hm(ck))
        dv = Dev.of(hm(cv).astype(np.float16) if kv_f16 else hm(cv))
        dq, do = Dev.of(q), Dev(n * nh * hd * 4)
        rc = _native.lib().ifx_ops_attention_prefill(dq.ptr, dk.ptr, dv.ptr, KV_F16 if kv_f16 else KV_F32, max_seq,
                                                     row0, n, nh, nkv, hd, int(causal), do.ptr, None)
        assert rc == 0, _native.lib().ifx_last_error()
        got = do.get(np.float32, n * nh * hd).reshape(n, nh, hd)
        assert np.isfinite(got).all()
        err = np.linalg.norm(got[rows].astype(np.float64) - ref[rows], axis=2) / scale
        assert err.max() <= TOL_PRE, (n, float(err.max()))
        # every row (not only the sampled ones) against the oracle, at the scale of the row's |v|
        vmag = np.linalg.norm(v.reshape(n, nkv, hd), axis=2).max()
        assert np.abs(got - ref).max() <= 10 * TOL_PRE * vmag
