"""Sessions on several host threads, one model shared: the contract of
include/inferox.h (an ifx_model is immutable after open and shared by threads;
each ifx_session, with its own stream, is used by one thread at a time), the
reference's `&Model` shared and `&mut KvCache` per caller
(src/model/forward.rs:543-548,592-622).

Each thread runs its own prompt through its own session; its tokens and
logits must equal, bit for bit, those of the same calls made one after the
other on one thread. ctypes releases the GIL around every library call, so
the sessions' launches overlap on the device.
"""
from __future__ import annotations

import os
import threading

import numpy as np
import pytest

from inferox_amd import synth
from tests.gpu_util import GpuModel

pytestmark = pytest.mark.gpu

C8B = synth.reduced(synth.LLAMA3_8B, name="c8b", n_layers=2, ctx=512, centred=True)


def _run_threads(fn, n):
    out, errs = [None] * n, []

    def body(i):
        try:
            out[i] = fn(i)
        except Exception as e:  # re-raised on the main thread
            errs.append(e)

    ts = [threading.Thread(target=body, args=(i,)) for i in range(n)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=300)
    assert not any(t.is_alive() for t in ts), "a session thread did not finish"
    if errs:
        raise errs[0]
    return out


def test_tiny_sessions_on_four_threads(tiny_path):
    """Four sessions of the tiny Q8_0 model, four prompts, each thread three
    generate calls of 64 greedy tokens and 8 decode steps with logits, against
    the same calls made sequentially."""
    g = GpuModel(tiny_path)
    prompts = [synth.token_ids(12 + 3 * i, synth.TINY.vocab, seed=900 + i) for i in range(4)]

    def work(i):
        s = g.session(256)
        toks = []
        for _ in range(3):
            rc, t = s.generate(prompts[i], 64)
            assert rc == 0
            toks.append(t.copy())
        assert all(np.array_equal(toks[0], t) for t in toks)
        s.clear()
        rc, _ = s.prefill(prompts[i], want_logits=False)
        assert rc == 0
        tok, lgs = int(toks[0][0]), []
        for _ in range(8):
            rc, lg = s.decode_step(tok)
            assert rc == 0
            lgs.append(lg.copy())
            tok = len(lg) - 1 - int(np.argmax(lg[::-1]))
        s.close()
        return toks[0], np.stack(lgs)

    ref = [work(i) for i in range(4)]
    got = _run_threads(work, 4)
    for i in range(4):
        assert np.array_equal(got[i][0], ref[i][0]), i
        assert np.array_equal(got[i][1].view(np.uint32), ref[i][1].view(np.uint32)), i
    g.close()


def test_8b_shape_sessions_on_two_threads_deterministic(tmpdir_session):
    """The 8B shape (two centred layers) in deterministic mode: two threads,
    each a batched prefill of its own 300 ids and 16 decode steps with
    logits, against the same sessions run one after the other."""
    p = str(tmpdir_session / "c8b_threads.gguf")
    if not os.path.exists(p):
        synth.write_llama(p, C8B, seed=88)
    g = GpuModel(p)
    prompts = [synth.token_ids(300, C8B.vocab, seed=950 + i) for i in range(2)]

    def work(i):
        s = g.session(400)
        s.set_deterministic(True)
        rc, _ = s.prefill(prompts[i], want_logits=False)
        assert rc == 0
        tok, lgs, picks = int(prompts[i][-1]), [], []
        for _ in range(16):
            rc, lg = s.decode_step(tok)
            assert rc == 0
            lgs.append(lg.copy())
            tok = len(lg) - 1 - int(np.argmax(lg[::-1]))
            picks.append(tok)
        s.close()
        return picks, np.stack(lgs)

    ref = [work(i) for i in range(2)]
    got = _run_threads(work, 2)
    for i in range(2):
        assert got[i][0] == ref[i][0], i
        assert np.array_equal(got[i][1].view(np.uint32), ref[i][1].view(np.uint32)), i
    assert ref[0][0] != ref[1][0]  # the two streams differ, so a swap would show
    g.close()
