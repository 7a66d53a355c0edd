"""The 70B shape at full depth (80 layers, centred weights), the long-context
workload of Model::generate (src/model/forward.rs:592-622): a GPU batched
prefill of 8192 seeded ids, its KV cache exported into the oracle, then 8
decode steps compared with the oracle (logits within 1e-3 relative L2, the
greedy picks identical), and the device's own greedy loop after the same
prefill giving the same 8 tokens.

The model file is 45 GB: the test needs that much free scratch space (it is
skipped, with the reason, otherwise) and removes the file when it ends.
Progress lines go to the terminal as each phase ends.
"""
from __future__ import annotations

import ctypes as C
import os
import shutil
import time

import numpy as np
import pytest

from inferox_amd import _native, synth
from oracle import binding as orc
from tests.conftest import rel_l2
from tests.gpu_util import GpuModel

pytestmark = pytest.mark.gpu

TOL = 1e-3
C70B_FULL = synth.reduced(synth.LLAMA3_70B, name="c70b-full", centred=True)


def last_argmax(lg):
    return len(lg) - 1 - int(np.argmax(lg[::-1]))


def test_centred_70b_full_depth_8192_context(tmp_path, capsys):
    need = C70B_FULL.gguf_bytes() + (8 << 30)
    free = shutil.disk_usage(str(tmp_path)).free
    if free < need:
        pytest.skip(f"needs {need / 1e9:.0f} GB of scratch space, {free / 1e9:.0f} GB free")
    t0 = time.time()

    def say(msg):
        with capsys.disabled():
            print(f"\n[70b full] {msg} ({time.time() - t0:.0f} s)", flush=True)

    p = str(tmp_path / "c70b_full.gguf")
    try:
        synth.write_llama(p, C70B_FULL, seed=7070)
        say("model written")
        g = GpuModel(p)
        c = g.cfg
        assert c.n_layers == 80 and c.hidden_size == 8192 and g.batched_prefill()
        ctx, steps = 8192, 8
        max_seq = ctx + steps + 8
        ids = synth.token_ids(ctx, c.vocab_size, seed=8192)
        s = g.session(max_seq)
        rc, _ = s.prefill(ids, want_logits=False)
        assert rc == 0
        last = C.c_uint32()
        assert _native.lib().ifx_session_last_token(s.h, C.byref(last)) == 0
        say("GPU prefill of 8192 ids done")
        k, v = s.kv_export(ctx)
        o = orc.Model(p)
        kv = o.kv(max_seq)
        assert kv.import_(k, v, ctx) == 0
        del k, v
        say("cache exported into the oracle")
        tok, picks, worst = int(last.value), [], 0.0
        for step in range(steps):
            rc, lg = s.decode_step(tok)
            orc_rc, ref = o.decode_step(kv, tok)
            assert rc == 0 and orc_rc == 0
            err = rel_l2(lg, ref)
            worst = max(worst, err)
            tok = orc.argmax(ref)[1]
            assert last_argmax(lg) == tok, step
            picks.append(tok)
            say(f"step {step + 1}: rel L2 {err:.2e}, pick {tok}")
        assert worst < TOL, worst
        s.close()
        o.close()
        s2 = g.session(max_seq)
        rc, _ = s2.prefill(ids, want_logits=False)
        assert rc == 0
        rc, toks = s2.decode_greedy(int(last.value), steps)
        assert rc == 0
        assert toks.tolist() == picks
        s2.close()
        g.close()
        say(f"greedy loop equal; worst rel L2 {worst:.2e}")
    finally:
        if os.path.exists(p):
            os.remove(p)
