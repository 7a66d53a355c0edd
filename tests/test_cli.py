"""The `inferox` command (src/main.rs): the inspect report on the CPU and the
generate text path on the GPU.

Inspect: a GGUF holding every metadata value type (arrays short, long, nested
and of strings; floats whose Rust Display differs from C's) against the
report's format strings (src/main.rs:109-182) with the values formatted by
numpy's shortest-round-trip positional formatter (Rust's float Display rule).
Generate: the tiny model with a tokenizer covering its vocabulary; the printed
text is the tokenizer's decoding of the oracle's CLI-path tokens (each prompt
token through decode_step, then greedy picks fed back).
"""
from __future__ import annotations

import json
import os
import subprocess

import numpy as np
import pytest

from inferox_amd import gguf_writer as gw
from inferox_amd.gguf_writer import GGUFWriter
from inferox_amd.tokenizer import BpeTokenizer, byte_encoder

CLI = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "inferox_amd", "lib", "inferox")
RULE = "-" * 72
VT_NAMES = ["uint8", "int8", "uint16", "int16", "uint32", "int32", "float32", "bool", "string", "array",
            "uint64", "int64", "float64"]


def run(*args, env=None):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([CLI, *args], capture_output=True, timeout=300, env=e)


def rust_display(vt, v):
    if vt == gw.VT_F32:
        x = np.float32(v)
        if np.isnan(x):
            return "NaN"
        if np.isinf(x):
            return "inf" if x > 0 else "-inf"
        return np.format_float_positional(x, unique=True, trim="-")
    if vt == gw.VT_F64:
        return np.format_float_positional(np.float64(v), unique=True, trim="-")
    if vt == gw.VT_BOOL:
        return "true" if v else "false"
    if vt == gw.VT_ARR:
        it, items = v
        parts = []
        for i, x in enumerate(items):
            if i >= 8 and len(items) > 9:
                parts.append("...")
                break
            parts.append(rust_display(it, x))
        return f"{VT_NAMES[it]}[{len(items)}] [" + ", ".join(parts) + "]"
    return str(v)


META = [
    ("general.architecture", gw.VT_STR, "llama"),
    ("a.u8", gw.VT_U8, 200), ("a.i8", gw.VT_I8, -7), ("a.u16", gw.VT_U16, 65535), ("a.i16", gw.VT_I16, -300),
    ("a.u32", gw.VT_U32, 4000000000), ("a.i32", gw.VT_I32, -2000000000), ("a.u64", gw.VT_U64, 2 ** 63 + 5),
    ("a.i64", gw.VT_I64, -(2 ** 62)), ("a.bool", gw.VT_BOOL, 1), ("a.bool0", gw.VT_BOOL, 0),
    ("f.eps", gw.VT_F32, 1e-5), ("f.big", gw.VT_F32, 1e30), ("f.tenth", gw.VT_F32, 0.1), ("f.negz", gw.VT_F32, -0.0),
    ("f.base", gw.VT_F32, 500000.0), ("f.nan", gw.VT_F32, float("nan")), ("f.inf", gw.VT_F32, float("-inf")),
    ("f.tiny", gw.VT_F32, 1e-45), ("d.tenth", gw.VT_F64, 0.1), ("d.third", gw.VT_F64, 1 / 3),
    ("arr.short", gw.VT_ARR, (gw.VT_U32, [1, 2, 3])),
    ("arr.nine", gw.VT_ARR, (gw.VT_I32, list(range(-4, 5)))),
    ("arr.long", gw.VT_ARR, (gw.VT_F32, [0.5 * i for i in range(20)])),
    ("arr.str", gw.VT_ARR, (gw.VT_STR, ["a", "b c", ""])),
    ("arr.nested", gw.VT_ARR, (gw.VT_ARR, [(gw.VT_U8, [1, 2]), (gw.VT_U8, [])])),
    ("arr.empty", gw.VT_ARR, (gw.VT_U64, [])),
]


def test_inspect_report(tmp_path):
    p = str(tmp_path / "m.gguf")
    w = GGUFWriter()
    for k, vt, v in META:
        w.add(k, vt, v)
    w.tensor_f32("t.one", [2], [1.5, 2.5])
    w.add_tensor("t.q4k", [256, 2], 12)
    w.add_tensor("t.q5k", [512], 13)
    for i in range(4):
        w.tensor_f32(f"t.extra{i}", [1], [float(i)])
    w.write(p)
    r = run(p)
    assert r.returncode == 0, r.stderr
    lines = r.stdout.decode().splitlines()
    assert lines[:6] == [RULE, "Header", RULE, "  version:     3", "  n_tensors:   7", f"  n_kv:        {len(META)}"]
    assert lines[6:9] == [RULE, f"Metadata ({len(META)} entries)", RULE]
    for i, (k, vt, v) in enumerate(META):
        assert lines[9 + i] == f"  [{i:3}] {k:50} ({VT_NAMES[vt]}) => {rust_display(vt, v)}", k
    rest = lines[9 + len(META):]
    assert rest[:3] == [RULE, "Tensors (7 tensors)", RULE]
    assert rest[3:9] == ["  [  0] t.one", "        type:    F32 (id=0)", "        shape:   [2]",
                         "        elems:   2", "        offset:  0 bytes", "        size:    8 bytes"]
    assert rest[9:15] == ["  [  1] t.q4k", "        type:    Q4_K (id=12)", "        shape:   [256 x 2]",
                          "        elems:   512", "        offset:  32 bytes", "        size:    288 bytes"]
    assert rest[16] == "        type:    Q5_K (id=13)" and rest[20] == "        size:    352 bytes"
    tail = rest[3 + 6 * 7:]
    assert tail[:3] == [RULE, "Layout", RULE]
    assert tail[3] == f"  file:                 {p}"
    assert tail[5] == "  total tensor bytes:   " + str(8 + 288 + 352 + 4 * 4) + " bytes"
    assert tail[6:9] == [RULE, "Raw tensor bytes (mmap)", RULE]
    assert tail[9] == f"  {'t.one':40} -> 8 bytes"
    assert tail[14] == "  ... and 2 more tensor(s)"


def test_usage_and_open_errors(tmp_path):
    r = run()
    assert r.returncode == 1 and b"usage:" in r.stderr
    r = run(str(tmp_path / "nope.gguf"))
    assert r.returncode == 1 and b"error: failed to open" in r.stderr
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGUX" + bytes(20))
    r = run(str(bad))
    assert r.returncode == 1 and b"error: failed to open" in r.stderr


def tiny_tokenizer(path: str, vocab_size: int):
    """Ids 1..256 the byte characters, then distinct two-character tokens up to vocab_size."""
    enc = byte_encoder()
    vocab = {"<|endoftext|>": 0}
    for b in range(256):
        vocab[enc[b]] = b + 1
    i = 257
    for a in range(32, 127):
        for c in range(32, 127):
            if i >= vocab_size:
                break
            vocab[enc[a] + enc[c]] = i
            i += 1
    with open(path, "w") as f:
        json.dump({"added_tokens": [{"content": "<|endoftext|>"}],
                   "model": {"type": "BPE", "vocab": vocab, "merges": [], "unk_token": "<|endoftext|>"}}, f)


@pytest.mark.gpu
def test_generate_text_greedy(tiny_path, tmp_path):
    from oracle import binding as orc
    o = orc.Model(tiny_path)
    tok_path = str(tmp_path / "tok.json")
    tiny_tokenizer(tok_path, o.vocab)
    tok = BpeTokenizer.from_file(tok_path)
    prompt = "The quick brown fox"
    ids = tok.encode(prompt)
    # src/main.rs:68-82 on the oracle
    kv = o.kv(o.cfg.context_length)
    lg = None
    for t in ids:
        rc, lg = o.decode_step(kv, t)
        assert rc == 0
    gen = []
    for _ in range(24):
        nxt = orc.argmax(lg)[1]
        gen.append(nxt)
        rc, lg = o.decode_step(kv, nxt)
        assert rc == 0
    r = run(tiny_path, tok_path, prompt, "24")
    assert r.returncode == 0, r.stderr
    assert r.stdout.decode() == tok.decode(gen)
    # empty prompt: the first pick is the argmax of the zeroed logits (the last index)
    kv = o.kv(o.cfg.context_length)
    gen, nxt = [], o.vocab - 1
    for _ in range(5):
        gen.append(nxt)
        _, lg = o.decode_step(kv, nxt)
        nxt = orc.argmax(lg)[1]
    r = run(tiny_path, tok_path, "", "5", "0")
    assert r.returncode == 0 and r.stdout.decode() == tok.decode(gen)
    o.close()


@pytest.mark.gpu
def test_generate_text_sampled(tiny_path, tmp_path):
    tok_path = str(tmp_path / "tok.json")
    tiny_tokenizer(tok_path, 32000)
    a = run(tiny_path, tok_path, "hello", "12", "0.8", env={"IFX_SEED": "42"})
    b = run(tiny_path, tok_path, "hello", "12", "0.8", env={"IFX_SEED": "42"})
    assert a.returncode == 0 and b.returncode == 0, a.stderr
    assert a.stdout == b.stdout and len(a.stdout) > 0
    # a context overflow is the reference's panic, here an error exit
    r = run(tiny_path, tok_path, "x" * 250, "32")
    assert r.returncode == 1 and b"error: decode failed" in r.stderr
