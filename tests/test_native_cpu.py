"""CPU-side checks of the product library: it loads, exports every entry point
declared in include/inferox.h, and its GGUF parser returns the same status as
the oracle (and the reference's gguf::Error variant) for malformed files.
No kernels are launched here."""
from __future__ import annotations

import ctypes as C
import os
import re
import struct

import numpy as np
import pytest

from inferox_amd import _native, synth
from inferox_amd.gguf_writer import GGUFWriter, _gguf_string
from oracle import binding as orc
from tests import fixtures_gguf as fx

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

pytestmark = pytest.mark.skipif(not os.path.exists(_native.PRODUCT_LIB),
                                reason="libinferox.so not built (run __graft_entry__.build())")


def _declared_symbols():
    names = set()
    inc = os.path.join(ROOT, "include")
    for fn in os.listdir(inc):
        if fn.endswith(".h"):
            text = open(os.path.join(inc, fn)).read()
            names |= set(re.findall(r"\b(ifx_[a-z0-9_]+)\s*\(", text))
    return names


def test_exports_every_declared_symbol():
    lib = C.CDLL(_native.PRODUCT_LIB)
    declared = _declared_symbols()
    assert len(declared) >= 40
    missing = [n for n in sorted(declared) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(declared) == set(_native.SIGNATURES)


def test_status_strings():
    L = _native.lib()
    for code in list(_native.STATUS_NAMES):
        assert L.ifx_status_string(code)
    assert L.ifx_status_string(9999) == b"unknown status"


def _open_product(path):
    h = C.c_void_p()
    rc = _native.lib().ifx_model_open(path.encode(), C.byref(h))
    if rc == 0:
        _native.lib().ifx_model_close(h)
    return rc


def _header(version=3, n_tensors=0, n_kv=0, magic=b"GGUF"):
    return magic + struct.pack("<IQQ", version, n_tensors, n_kv)


def _malformed(tmp_path):
    """(name, bytes, expected status) — the reference error each one raises."""
    cases = []
    cases.append(("bad_magic", _header(magic=b"GGML"), 2))
    cases.append(("version_1", _header(version=1), 3))
    cases.append(("version_4", _header(version=4), 3))
    cases.append(("truncated", b"GGUF\x03\x00", 1))
    kv = _gguf_string("k") + struct.pack("<I", 13)
    cases.append(("value_type_13", _header(n_kv=1) + kv, 4))
    kv = _gguf_string("k") + struct.pack("<IIQ", 9, 99, 1)
    cases.append(("array_item_type_99", _header(n_kv=1) + kv, 4))
    kv = struct.pack("<Q", 2) + b"\xff\xfe" + struct.pack("<IB", 0, 1)
    cases.append(("utf8_key", _header(n_kv=1) + kv, 6))
    ti = _gguf_string("t") + struct.pack("<I", 5) + struct.pack("<5Q", 1, 1, 1, 1, 1) + struct.pack("<IQ", 0, 0)
    cases.append(("n_dims_5", _header(n_tensors=1) + ti, 7))
    for bad in (4, 9, 31):
        ti = _gguf_string("t") + struct.pack("<I", 1) + struct.pack("<Q", 32) + struct.pack("<IQ", bad, 0)
        cases.append((f"tensor_type_{bad}", _header(n_tensors=1) + ti, 5))
    cases.append(("no_architecture", _header(), 9))
    w = GGUFWriter()
    w.add_string("general.architecture", "gpt2")
    cases.append(("arch_gpt2", w.header_bytes(), 12))
    return cases


def test_parser_errors_match_oracle(tmp_path):
    for name, data, expected in _malformed(tmp_path):
        p = str(tmp_path / f"{name}.gguf")
        with open(p, "wb") as f:
            f.write(data)
        assert orc.Model.open_status(p) == expected, name
        assert _open_product(p) == expected, name


def test_missing_tensor_and_metadata(tmp_path):
    p = str(tmp_path / "m.gguf")
    fx.llama_wiring_gguf(p)
    # drop blk.1.ffn_down.weight: TensorNotFound("blk.1.*")
    w = GGUFWriter()
    fx._llama_meta(w, 100, 64, 2, 4, 2, 128, 512)
    for n in ["token_embd.weight", "output_norm.weight"] + [
            f"blk.{i}.{r}.weight" for i in range(2) for r in
            ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm", "ffn_gate", "ffn_up",
             "ffn_down")][:-1]:
        w.tensor_f32(n, [1, 1], [0.0])
    q = str(tmp_path / "missing.gguf")
    w.write(q)
    assert orc.Model.open_status(q) == 9
    assert _open_product(q) == 9
    # required metadata missing: embedding_length
    w = GGUFWriter()
    w.add_string("general.architecture", "llama")
    r = str(tmp_path / "nometa.gguf")
    w.write(r)
    assert orc.Model.open_status(r) == 9
    assert _open_product(r) == 9


def test_device_required_after_parse(tmp_path):
    """A well-formed model parses on the host; with no gfx950 device present the
    product refuses loudly (no CPU fallback exists)."""
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU driver is present")
    p = str(tmp_path / "ok.gguf")
    fx.builder_llama_gguf(p, fill=0.0)
    assert _open_product(p) == 25
    h = C.c_void_p()
    assert _native.lib().ifx_malloc(C.byref(h), 16) == 25
    # the sampler entry point checks its arguments, then the device
    logits = (C.c_float * 8)(*range(8))
    out = (C.c_uint32 * 2)()
    assert _native.lib().ifx_sample_logits(logits, 8, 1.0, 0, 1.0, 1, 2, out) == 25
    assert _native.lib().ifx_sample_logits(logits, 0, 1.0, 0, 1.0, 1, 2, out) == 20


def test_synth_is_deterministic(tmp_path):
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    spec = synth.reduced(synth.TINY, n_layers=1, vocab=512)
    size = synth.write_llama(a, spec, seed=9)
    synth.write_llama(b, spec, seed=9)
    assert open(a, "rb").read() == open(b, "rb").read()
    m = orc.Model(a)
    assert m.cfg.vocab_size == 512 and m.cfg.n_layers == 1 and m.cfg.head_dim == 48
    assert size >= spec.gguf_bytes()
    # payload distribution of the Q8_0 blocks: delta in [1e-3, 1e-2], quants in [-127, 127]
    infos = m.tensor_infos()
    idx = [i for i, t in enumerate(infos) if t[0] == "blk.0.attn_q.weight"][0]
    raw = m.tensor_bytes(idx).reshape(-1, 34)
    d = raw[:, :2].copy().view("<f2").astype(np.float32)
    assert d.min() >= 9.9e-4 and d.max() <= 1.001e-2
    q = raw[:, 2:].view(np.int8)
    assert q.min() >= -127 and q.max() <= 127


def test_synth_8b_layout_bytes():
    """Stored bytes of the 8B-shape Q4_K_M model (the decode roofline numerator)."""
    s = synth.LLAMA3_8B
    per_layer = sum(synth.byte_size(t, r * c) for (n, _, t, r, c) in s.shapes() if n.startswith("blk.0."))
    assert per_layer == 138_936_320  # includes the two f32 norms
    head = synth.byte_size(synth.Q6_K, 128256 * 4096)
    assert head == 430_940_160


def test_huge_block_count_is_tensor_not_found(tmp_path):
    """llama.block_count is a u64 from the file: a count whose 9x product wraps
    to 2 (2049638230412172402) must meet blk.1.* missing and report
    TensorNotFound (src/model/mod.rs:69-72), not size a buffer from it."""
    w = GGUFWriter()
    w.add_string("general.architecture", "llama")
    w.add_u32("llama.vocab_size", 100).add_u32("llama.embedding_length", 64)
    w.add_u64("llama.block_count", 2049638230412172402)
    assert (9 * 2049638230412172402) % (1 << 64) == 2
    w.add_u32("llama.attention.head_count", 4).add_u32("llama.feed_forward_length", 128)
    names = ["token_embd.weight", "output_norm.weight"] + [
        f"blk.0.{r}.weight" for r in ("attn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_norm",
                                      "ffn_gate", "ffn_up", "ffn_down")]
    for n in names:
        w.tensor_f32(n, [1, 1], [0.0])
    p = str(tmp_path / "huge_blocks.gguf")
    w.write(p)
    assert orc.Model.open_status(p) == 9
    assert _open_product(p) == 9


def test_huge_counts_are_io_errors(tmp_path):
    """Metadata, array and tensor counts larger than the file can back end in an
    io error as the reference's reads would (src/gguf/file.rs:93-110,
    src/gguf/value.rs:55-66), with no allocation sized by the count."""
    # an array claiming 2^40 items of u8 in a tiny file
    kv = _gguf_string("k") + struct.pack("<IIQ", 9, 0, 1 << 40)
    p = str(tmp_path / "arr.gguf")
    with open(p, "wb") as f:
        f.write(_header(n_kv=1) + kv + b"\x00" * 64)
    assert orc.Model.open_status(p) == 1
    assert _open_product(p) == 1
    # metadata and tensor counts just under the file size: entries run out first
    for n_kv, n_t in ((200, 0), (0, 200)):
        q = str(tmp_path / f"counts_{n_kv}_{n_t}.gguf")
        with open(q, "wb") as f:
            f.write(_header(n_tensors=n_t, n_kv=n_kv) + b"\x01" * 220)
        assert orc.Model.open_status(q) == _open_product(q)
        assert _open_product(q) in (1, 4, 5, 6, 7)
