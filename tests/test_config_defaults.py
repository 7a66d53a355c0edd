"""Config::from_gguf defaults (src/model/config.rs:47-68) on both sides.

GGUF files that omit llama.attention.head_count_kv (-> head_count),
llama.attention.key_length (-> embedding_length / head_count),
llama.rope.dimension_count (-> head_dim), llama.context_length (-> 4096) and
llama.vocab_size (-> 0), or that set key_length / rope.dimension_count
explicitly.  The closed-form defaults are asserted on the oracle here (CPU)
and on the product's ifx_model_config on the GPU, with vocab_size 0 making
every token an InvalidTensorIndex (src/model/forward.rs:552-554: the token
is checked against vocab_size before anything else).
"""
from __future__ import annotations

import numpy as np
import pytest

from inferox_amd.gguf_writer import GGUFWriter
from oracle import binding as orc
from tests.conftest import rel_l2

DIM, HEADS, FFN, LAYERS, NV = 64, 4, 128, 2, 100

OPTIONAL = ("head_count_kv", "key_length", "rope_dim", "context_length", "vocab_size")


def write_model(path, omit=(), kv_heads=2, key_length=None, rope_dim=None, seed=5):
    """A small F32 llama whose optional metadata keys are written or omitted."""
    rng = np.random.default_rng(seed)
    kvh = HEADS if "head_count_kv" in omit else kv_heads
    hd = DIM // HEADS
    w = GGUFWriter()
    w.add_string("general.architecture", "llama")
    if "vocab_size" not in omit:
        w.add_u32("llama.vocab_size", NV)
    w.add_u32("llama.embedding_length", DIM).add_u32("llama.block_count", LAYERS)
    w.add_u32("llama.attention.head_count", HEADS)
    if "head_count_kv" not in omit:
        w.add_u32("llama.attention.head_count_kv", kv_heads)
    if key_length is not None:
        w.add_u32("llama.attention.key_length", key_length)
    if rope_dim is not None:
        w.add_u32("llama.rope.dimension_count", rope_dim)
    if "context_length" not in omit:
        w.add_u32("llama.context_length", 256)
    w.add_u32("llama.feed_forward_length", FFN)
    w.add_f32("llama.rope.freq_base", 10000.0)

    def mat(name, rows, cols, scale=0.15):
        w.tensor_f32(name, [cols, rows], (rng.standard_normal(rows * cols) * scale).astype(np.float32))

    mat("token_embd.weight", NV, DIM, 1.0)
    w.tensor_f32("output_norm.weight", [DIM], (1 + 0.02 * rng.standard_normal(DIM)).astype(np.float32))
    mat("output.weight", NV, DIM)
    for i in range(LAYERS):
        p = f"blk.{i}."
        w.tensor_f32(p + "attn_norm.weight", [DIM], (1 + 0.02 * rng.standard_normal(DIM)).astype(np.float32))
        mat(p + "attn_q.weight", DIM, DIM)
        mat(p + "attn_k.weight", kvh * hd, DIM)
        mat(p + "attn_v.weight", kvh * hd, DIM)
        mat(p + "attn_output.weight", DIM, DIM)
        w.tensor_f32(p + "ffn_norm.weight", [DIM], (1 + 0.02 * rng.standard_normal(DIM)).astype(np.float32))
        mat(p + "ffn_gate.weight", FFN, DIM)
        mat(p + "ffn_up.weight", FFN, DIM)
        mat(p + "ffn_down.weight", DIM, FFN)
    w.write(path)


def expected_config(omit=(), kv_heads=2, key_length=None, rope_dim=None):
    hd = key_length if key_length is not None else DIM // HEADS
    return dict(n_kv_heads=HEADS if "head_count_kv" in omit else kv_heads, head_dim=hd,
                rope_dim=rope_dim if rope_dim is not None else hd,
                context_length=4096 if "context_length" in omit else 256,
                vocab_size=0 if "vocab_size" in omit else NV)


CASES = [((), None, None), (("head_count_kv",), None, None), (("context_length",), None, None),
         (("vocab_size",), None, None), (OPTIONAL, None, None), ((), DIM // HEADS, None), ((), None, 8)]


def _cfg_dict(c):
    return dict(n_kv_heads=c.n_kv_heads, head_dim=c.head_dim, rope_dim=c.rope_dim,
                context_length=c.context_length, vocab_size=c.vocab_size)


@pytest.mark.parametrize("omit,key_length,rope_dim", CASES)
def test_oracle_defaults(tmp_path, omit, key_length, rope_dim):
    p = str(tmp_path / "m.gguf")
    write_model(p, omit, key_length=key_length, rope_dim=rope_dim)
    o = orc.Model(p)
    assert _cfg_dict(o.cfg) == expected_config(omit, key_length=key_length, rope_dim=rope_dim)
    assert o.cfg.n_heads == HEADS and o.cfg.hidden_size == DIM and o.cfg.n_layers == LAYERS
    kv = o.kv(16)
    if "vocab_size" in omit:
        for t in (0, 1, NV - 1):
            assert o.decode_step(kv, t)[0] == 10
        assert o.prefill(kv, [0, 1])[0] == 10
        assert o.generate(kv, [0], 2)[0] == 10
    else:
        assert o.decode_step(kv, 3)[0] == 0
    o.close()


@pytest.mark.gpu
@pytest.mark.parametrize("omit,key_length,rope_dim", CASES)
def test_product_defaults(tmp_path, omit, key_length, rope_dim):
    from tests.gpu_util import GpuModel
    p = str(tmp_path / "m.gguf")
    write_model(p, omit, key_length=key_length, rope_dim=rope_dim)
    g, o = GpuModel(p), orc.Model(p)
    assert _cfg_dict(g.cfg) == expected_config(omit, key_length=key_length, rope_dim=rope_dim)
    assert _cfg_dict(g.cfg) == _cfg_dict(o.cfg)
    s, kv = g.session(16), o.kv(16)
    if "vocab_size" in omit:
        for t in (0, 1, NV - 1):
            assert s.decode_step(t)[0] == 10
        assert s.prefill([0, 1])[0] == 10
        assert s.generate([0], 2)[0] == 10
    else:
        # the defaulted (or explicit) shape runs and matches the oracle, with
        # absolute RoPE so that a partial rope_dim rotates something
        s.set_rope_mode(1)
        for t in (3, 7, 11):
            rc, lg = s.decode_step(t)
            _, ref = o.decode_step(kv, t, rope_mode=orc.ROPE_ABSOLUTE)
            assert rc == 0 and rel_l2(lg, ref) < 1e-3
    s.close()
    g.close()
    o.close()
