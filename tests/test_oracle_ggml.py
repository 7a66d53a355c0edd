"""The numpy restatements of ggml's Q4_K / Q6_K dequantizers (the checker of
the ggml-layout mode; llama.cpp ggml-quants.c dequantize_row_q4_K / _q6_K),
pinned on the CPU:

* on blocks both layouts can hold (every Q4_K block; Q6_K blocks whose scales
  are below 128) a reference block rewritten in ggml's layout dequantizes,
  through the ggml restatement, to exactly the reference restatement's values;
* hand-built ggml blocks give the values the published formulas give for
  chosen elements (nibble halves, the qh bit pairs, a negative scale).
"""
from __future__ import annotations

import numpy as np

from inferox_amd import synth
from oracle import numpy_ref as nr
from tests.ggml_layout import q4k_ref_to_ggml, q6k_ref_to_ggml

Q4_K, Q6_K = 12, 14


def f16b(v):
    return np.array([v], np.float16).view(np.uint8)


def test_q4k_layouts_agree():
    ref = synth.random_blocks(Q4_K, 256 * 64, seed=3)
    a = nr.dequant_q4_k(ref)
    b = nr.dequant_q4_k_ggml(q4k_ref_to_ggml(ref))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q6k_layouts_agree_on_small_scales():
    ref = synth.random_blocks(Q6_K, 256 * 64, seed=4).reshape(-1, 210).copy()
    ref[:, 2:18] &= 127                       # scales both layouts read alike
    sc = ref[:, 2:18].astype(np.int8)
    a = nr.dequant_q6_k(ref.reshape(-1))
    b = nr.dequant_q6_k_ggml(q6k_ref_to_ggml(ref.reshape(-1), sc))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q4k_ggml_hand_block():
    blk = np.zeros(144, np.uint8)
    blk[0:2] = f16b(0.5)       # d
    blk[2:4] = f16b(0.25)      # dmin
    blk[4:16] = [1, 2, 3, 4, 1, 1, 1, 1, 0, 0, 0, 0]  # sc = 1,2,3,4 for sub-blocks 0..3, mins 1
    blk[16] = 0x7A             # qs[0]: low 0xA -> element 0 (sub-block 0), high 7 -> element 32 (sub-block 1)
    blk[16 + 32] = 0x3C        # qs[32]: low 0xC -> element 64 (sub-block 2), high 3 -> element 96 (sub-block 3)
    y = nr.dequant_q4_k_ggml(blk)
    assert y[0] == np.float32(0.5 * 1 * 10 - 0.25)
    assert y[32] == np.float32(0.5 * 2 * 7 - 0.25)
    assert y[64] == np.float32(0.5 * 3 * 12 - 0.25)
    assert y[96] == np.float32(0.5 * 4 * 3 - 0.25)
    assert y[1] == np.float32(-0.25)


def test_q6k_ggml_hand_block():
    blk = np.zeros(210, np.uint8)
    blk[0] = 0x5A              # ql[0]: low 0xA -> element 0, high 5 -> element 64
    blk[32] = 0x31             # ql[32]: low 1 -> element 32, high 3 -> element 96
    blk[128] = 0b10_01_11_00   # qh[0]: bits 0-1 -> e0, 2-3 -> e32, 4-5 -> e64, 6-7 -> e96
    blk[64 + 5] = 0x0F         # ql[64 + 5]: low 0xF -> element 128 + 5 (second half)
    blk[128 + 32 + 5] = 0b11   # qh[32 + 5]: element 133's high bits
    sc = np.zeros(16, np.int8)
    sc[0], sc[2], sc[4], sc[6], sc[8] = -3, 7, -128, 127, -1
    blk[192:208] = sc.view(np.uint8)
    blk[208:210] = f16b(0.5)
    y = nr.dequant_q6_k_ggml(blk)
    assert y[0] == np.float32((0.5 * -3) * ((0xA | 0 << 4) - 32))
    assert y[32] == np.float32((0.5 * 7) * ((1 | 3 << 4) - 32))
    assert y[64] == np.float32((0.5 * -128) * ((5 | 1 << 4) - 32))
    assert y[96] == np.float32((0.5 * 127) * ((3 | 2 << 4) - 32))
    assert y[133] == np.float32((0.5 * -1) * ((0xF | 3 << 4) - 32))
    assert y[1] == np.float32((0.5 * -3) * -32)
