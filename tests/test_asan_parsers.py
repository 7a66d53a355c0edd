"""AddressSanitizer (+ UndefinedBehaviorSanitizer) run of the product's
untrusted-input parsers on the CPU: the GGUF reader (host_gguf.cpp, with the
type tables of host_types.cpp; counterpart of src/gguf/file.rs:57-116), the
model loader's host half (host_config.cpp: Config::from_gguf,
src/model/config.rs:34-84, and the weight resolution of Model::open,
src/model/mod.rs:34-92) and the tokenizer.json reader + BPE
(host_tokenizer.cpp; src/tokenizer/mod.rs:61-226).

tests/asan/parse_driver.cpp is compiled with g++ -fsanitize=address,undefined
together with those three sources and fed: the malformed GGUF files of the
parser-status test, counts larger than the file, seeded truncations and byte
flips of a valid file, and valid / malformed / truncated tokenizer JSON.  Any
sanitizer report fails the run; the statuses must equal the regular build's.
"""
from __future__ import annotations

import json
import os
import random
import shutil
import struct
import subprocess

import numpy as np
import pytest

from inferox_amd import _native
from inferox_amd.gguf_writer import _gguf_string
from inferox_amd.tokenizer import BpeTokenizer, TokenizerError
from tests import fixtures_gguf as fx
from tests.test_native_cpu import _header, _malformed
from tests.test_tokenizer import tiny_json

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "inferox_amd", "csrc")
PARSE_ERRORS = {1, 2, 3, 4, 5, 6, 7, 8}


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    gxx = shutil.which("g++")
    if not gxx:
        pytest.skip("g++ not available")
    out = str(tmp_path_factory.mktemp("asan") / "parse_driver")
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=undefined", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           os.path.join(ROOT, "tests", "asan", "parse_driver.cpp"), os.path.join(CSRC, "host_gguf.cpp"),
           os.path.join(CSRC, "host_config.cpp"),
           os.path.join(CSRC, "host_types.cpp"), os.path.join(CSRC, "host_tokenizer.cpp"), "-o", out]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        if "asan" in r.stdout.lower() and "cannot find" in r.stdout.lower():
            pytest.skip("libasan not installed")
        raise AssertionError(r.stdout)
    return out


def _run(driver, args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=86",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1:exitcode=87")
    r = subprocess.run([driver, *args], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, env=env,
                       timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "Sanitizer" not in r.stderr, r.stderr[-4000:]
    return [int(x) for x in r.stdout.split()]


def _gguf_cases(tmp_path):
    """(path, expected status or None for 'any status')"""
    cases = []
    for name, data, expected in _malformed(tmp_path):
        p = str(tmp_path / f"m_{name}.gguf")
        open(p, "wb").write(data)
        cases.append((p, expected if expected in PARSE_ERRORS else 0))
    kv = _gguf_string("k") + struct.pack("<IIQ", 9, 0, 1 << 40)
    p = str(tmp_path / "huge_array.gguf")
    open(p, "wb").write(_header(n_kv=1) + kv + b"\x00" * 64)
    cases.append((p, 1))
    # nested arrays claiming more items than bytes remain
    kv = _gguf_string("k") + struct.pack("<IIQ", 9, 9, 3) + struct.pack("<IQ", 8, 1 << 33)
    p = str(tmp_path / "nested_array.gguf")
    open(p, "wb").write(_header(n_kv=1) + kv + b"\x00" * 32)
    cases.append((p, 1))
    good = str(tmp_path / "wiring.gguf")
    fx.llama_wiring_gguf(good)
    cases.append((good, 0))
    tiny = str(tmp_path / "builder.gguf")
    fx.builder_llama_gguf(tiny, fill=1.0)
    cases.append((tiny, 0))
    raw = open(good, "rb").read()
    rng = random.Random(1234)
    for i, cut in enumerate(sorted(rng.sample(range(1, len(raw)), 60))):
        p = str(tmp_path / f"cut_{i}.gguf")
        open(p, "wb").write(raw[:cut])
        cases.append((p, None))
    for i in range(120):
        b = bytearray(raw)
        for _ in range(rng.randint(1, 6)):
            b[rng.randrange(len(b))] = rng.randrange(256)
        p = str(tmp_path / f"flip_{i}.gguf")
        open(p, "wb").write(bytes(b))
        cases.append((p, None))
    return cases


def test_gguf_parser_under_asan(driver, tmp_path):
    cases = _gguf_cases(tmp_path)
    got = _run(driver, ["g:" + p for p, _ in cases])
    assert len(got) == len(cases)
    for (p, want), st in zip(cases, got):
        if want is None:
            assert st == 0 or st in PARSE_ERRORS or st in (9, 10, 11), (p, st)
        else:
            assert st == want, (os.path.basename(p), st, want)


def _tok_cases():
    good = tiny_json(extra_vocab=["ab", "bc", "hello"], merges=["a b", "b c", "h e"])
    cases = [good, tiny_json(unk=None), "", "{", "[]", "null", '{"model": 3}', '{"model": {"type": "WordPiece"}}',
             '{"model": {"type": "BPE", "vocab": {"a": -1}, "merges": []}}',
             '{"model": {"type": "BPE", "vocab": {"a": 1e400}, "merges": []}}',
             '{"model": {"type": "BPE", "vocab": {"\\ud800": 1}, "merges": ["\\u0000 a"]}}',
             '{"added_tokens": [{"content": ""}], "model": {"type": "BPE", "vocab": {}, "merges": ["a"]}}',
             "[" * 5000 + "]" * 5000, '"' + "\\u" * 100]
    rng = random.Random(99)
    for _ in range(80):
        cut = rng.randrange(1, len(good))
        cases.append(good[:cut])
    for _ in range(80):
        b = bytearray(good.encode())
        for _ in range(rng.randint(1, 4)):
            b[rng.randrange(len(b))] = rng.randrange(32, 127)
        cases.append(b.decode("latin-1"))
    return cases


def _python_status(text: str) -> int:
    try:
        BpeTokenizer.from_json(text)
        return 0
    except TokenizerError as e:
        return e.status


def test_tokenizer_reader_under_asan(driver, tmp_path):
    cases = _tok_cases()
    paths = []
    for i, text in enumerate(cases):
        p = str(tmp_path / f"tok_{i}.json")
        open(p, "w", encoding="latin-1").write(text)
        paths.append(p)
    got = _run(driver, ["t:" + p for p in paths])
    assert len(got) == len(cases)
    want = [_python_status(t) for t in cases]
    assert got == want
    assert got[0] == 0 and got[1] == 0


def _llama(path, *, block_count=1, dim=64, heads=4, kv_heads=None, ffn=128, key_length=None, skip=(),
           shapes=None):
    """A small llama GGUF with one block's tensors (F32 zeros) and chosen metadata."""
    from inferox_amd.gguf_writer import GGUFWriter
    w = GGUFWriter()
    w.add_string("general.architecture", "llama")
    w.add_u32("llama.vocab_size", 16).add_u64("llama.embedding_length", dim)
    w.add_u64("llama.block_count", block_count).add_u64("llama.attention.head_count", heads)
    if kv_heads is not None:
        w.add_u32("llama.attention.head_count_kv", kv_heads)
    if key_length is not None:
        w.add_u32("llama.attention.key_length", key_length)
    w.add_u64("llama.feed_forward_length", ffn)
    d, f, kv = min(dim, 64), min(ffn, 128), min(dim, 64)  # the tensors stay small whatever the metadata says
    base = {"token_embd.weight": [d, 16], "output_norm.weight": [d], "blk.0.attn_norm.weight": [d],
            "blk.0.attn_q.weight": [d, d], "blk.0.attn_k.weight": [d, kv], "blk.0.attn_v.weight": [d, kv],
            "blk.0.attn_output.weight": [d, d], "blk.0.ffn_norm.weight": [d],
            "blk.0.ffn_gate.weight": [d, f], "blk.0.ffn_up.weight": [d, f], "blk.0.ffn_down.weight": [f, d]}
    base.update(shapes or {})
    for name, shape in base.items():
        if name in skip:
            continue
        n = int(np.prod(shape))
        w.tensor_f32(name, shape, [0.0] * n)
    w.write(path)
    return path


def test_asan_model_loader(driver, tmp_path):
    """The loader's host half on valid and hostile metadata: wrapping and huge
    block counts end at the first missing blk.N tensor (TensorNotFound),
    dimensions whose products overflow or do not match the tensors are
    InvalidArg, missing tensors TensorNotFound; nothing is sized from a count."""
    T = str(tmp_path)
    cases = [
        (_llama(T + "/ok.gguf"), 0),
        (_llama(T + "/wrap.gguf", block_count=2049638230412172402), 9),
        (_llama(T + "/huge_blocks.gguf", block_count=(1 << 64) - 1), 9),
        (_llama(T + "/two_blocks.gguf", block_count=2), 9),
        (_llama(T + "/heads0.gguf", heads=0), 20),
        (_llama(T + "/huge_dim.gguf", dim=1 << 62), 20),
        (_llama(T + "/huge_ffn.gguf", ffn=(1 << 63) + 64), 20),
        (_llama(T + "/huge_kv.gguf", kv_heads=0xFFFFFFFF, key_length=0xFFFFFFFF), 20),
        (_llama(T + "/no_v.gguf", skip=("blk.0.attn_v.weight",)), 9),
        (_llama(T + "/no_onorm.gguf", skip=("output_norm.weight",)), 9),
        (_llama(T + "/no_embd.gguf", skip=("token_embd.weight",)), 9),
        (_llama(T + "/untied.gguf", shapes={"output.weight": [64, 16]}), 0),
        (_llama(T + "/bad_output.gguf", shapes={"output.weight": [63, 16]}), 20),
        (_llama(T + "/bad_q.gguf", shapes={"blk.0.attn_q.weight": [64, 63]}), 20),
        (_llama(T + "/bad_embd.gguf", shapes={"token_embd.weight": [63, 16]}), 20),
        (_llama(T + "/bad_norm.gguf", shapes={"blk.0.ffn_norm.weight": [65]}), 20),
        (_llama(T + "/bad_down.gguf", shapes={"blk.0.ffn_down.weight": [128, 63]}), 20),
    ]
    got = _run(driver, ["m:" + p for p, _ in cases])
    assert got == [e for _, e in cases], list(zip([os.path.basename(p) for p, _ in cases], got))
    # the regular build reports the same statuses for what it decides before any device work
    for (p, e), g in zip(cases, got):
        if e == 9:
            assert _native_open_status(p) == 9, p


def _native_open_status(path):
    import ctypes as C
    h = C.c_void_p()
    rc = _native.lib().ifx_model_open(path.encode(), C.byref(h))
    if rc == 0:
        _native.lib().ifx_model_close(h)
    return rc
