"""The text path's BPE tokenizer (src/tokenizer/mod.rs) through the C ABI, on
the CPU (host code; no device).

Pins: the reference's own tests (src/tokenizer/mod.rs:268-318: ASCII round
trip, special-token split) on the same synthetic tokenizer.json; hand-worked
merge orders (lowest rank first, leftmost on equal ranks, merged pieces
missing from the vocab becoming unk); decode's byte table and non-byte
characters; String::from_utf8_lossy against CPython's UTF-8 decoder with
errors="replace" (the same maximal-subpart rule) on random byte strings;
round trips through byte-complete vocabularies; the JSON reader against
Python's json on escapes and surrogate pairs; and the error statuses of
TokenizerError::{Io, Json, UnsupportedModel}.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

from inferox_amd.tokenizer import (IFX_E_IO, IFX_E_JSON, IFX_E_UNSUPPORTED_TOKENIZER, BpeTokenizer,
                                   TokenizerError, byte_encoder)

ENC = byte_encoder()


def tiny_json(extra_vocab=(), merges=(), added=("<|endoftext|>",), unk="<|endoftext|>"):
    """The reference's test tokenizer (src/tokenizer/mod.rs:272-300): id 0 the
    end-of-text token, ids 1..256 the byte characters, one space+space merge."""
    vocab = {"<|endoftext|>": 0}
    for b in range(256):
        vocab[ENC[b]] = b + 1
    for i, tok in enumerate(extra_vocab):
        vocab[tok] = 257 + i
    ms = [f"{ENC[32]} {ENC[32]}"] + list(merges)
    model = {"type": "BPE", "vocab": vocab, "merges": ms}
    if unk is not None:
        model["unk_token"] = unk
    return json.dumps({"version": "1.0", "added_tokens": [{"content": a} for a in added], "model": model})


def test_encode_decode_ascii_roundtrip():
    t = BpeTokenizer.from_json(tiny_json())
    ids = t.encode("hello world")
    assert ids
    assert t.decode(ids) == "hello world"
    assert ids == [ord(c) + 1 for c in "hello world"]


def test_special_token_is_split():
    t = BpeTokenizer.from_json(tiny_json())
    ids = t.encode("hi<|endoftext|>lo")
    assert 0 in ids
    assert ids == [ord("h") + 1, ord("i") + 1, 0, ord("l") + 1, ord("o") + 1]


def test_merge_order_and_unk():
    a, b, c = "a", "b", "c"
    # (b, c) ranks before (a, b): "abc" -> a + bc
    t = BpeTokenizer.from_json(tiny_json(extra_vocab=["ab", "bc"], merges=[f"{b} {c}", f"{a} {b}"]))
    assert t.encode("abc") == [ord("a") + 1, 258]
    # leftmost pair on equal ranks: aaaa -> aa a a -> aa aa (no (aa, aa) merge)
    t = BpeTokenizer.from_json(tiny_json(extra_vocab=["aa"], merges=["a a"]))
    assert t.encode("aaaa") == [257, 257]
    assert t.encode("aaa") == [257, ord("a") + 1]
    # the space+space merge has no vocab entry: unk (id 0)
    t = BpeTokenizer.from_json(tiny_json())
    assert t.encode("a  b") == [ord("a") + 1, 0, ord("b") + 1]
    # unk_token absent from the model, or not in the vocab: id 0
    t = BpeTokenizer.from_json(tiny_json(unk=None, extra_vocab=["zz"]))
    assert t.encode("  ") == [0]
    # a duplicate merge line keeps its later rank (HashMap insert)
    t = BpeTokenizer.from_json(tiny_json(extra_vocab=["ab", "bc"], merges=["a b", "b c", "a b"]))
    assert t.encode("abc") == [ord("a") + 1, 258]


def test_special_tokens_edges():
    t = BpeTokenizer.from_json(tiny_json(added=("<|endoftext|>", "<s>", "<s>x", ""), extra_vocab=["<s>"]))
    assert t.encode("") == []
    assert t.encode("<s><|endoftext|>") == [257, 0]
    # two specials at the same position: the longer one ("<s>x" is not in the vocab: unk)
    assert t.encode("q<s>xq") == [ord("q") + 1, 0, ord("q") + 1]
    assert t.encode("<s>") == [257]
    assert t.encode("<s") == [ord("<") + 1, ord("s") + 1]


def test_decode_bytes_and_other_characters():
    t = BpeTokenizer.from_json(tiny_json(extra_vocab=["中", "xĠy"]))
    assert t.decode([257]) == "中"                 # not in the byte table: its UTF-8 bytes
    assert t.decode([258]) == "x y"                 # U+0120 is byte 0x20
    assert t.decode([99999, ord("a") + 1]) == "a"   # unknown ids are skipped
    assert t.decode([]) == ""
    # bytes that do not form UTF-8: replacement characters
    assert t.decode([0xE2 + 1, 0x82 + 1, ord("a") + 1]) == "�a"
    assert t.decode([0xC0 + 1, 0x80 + 1]) == "��"


def test_lossy_decode_matches_cpython():
    t = BpeTokenizer.from_json(tiny_json())
    rng = np.random.default_rng(7)
    specials = [0x80, 0xBF, 0xC0, 0xC2, 0xDF, 0xE0, 0xA0, 0xED, 0x9F, 0xEF, 0xF0, 0x90, 0xF4, 0x8F, 0xF5, 0xFF]
    for trial in range(400):
        n = int(rng.integers(1, 12))
        pool = np.array(specials + list(range(0x20, 0x7F)), np.int64)
        bs = bytes(int(x) for x in (rng.choice(pool, n) if trial % 2 else rng.integers(0, 256, n)))
        got = t.decode([b + 1 for b in bs])
        assert got == bs.decode("utf-8", errors="replace"), bs


def test_roundtrip_byte_complete_vocab():
    rng = np.random.default_rng(11)
    text = "".join(rng.choice(list("ab cdé中😀\n"), 400))
    data = text.encode()
    # merges learned greedily from the data's byte pairs; every merge result is in the vocab
    pieces = [ENC[b] for b in data]
    extra, merges = [], []
    for _ in range(40):
        counts = {}
        for x, y in zip(pieces, pieces[1:]):
            counts[(x, y)] = counts.get((x, y), 0) + 1
        if not counts:
            break
        (x, y), _ = max(counts.items(), key=lambda kv: kv[1])
        merges.append(f"{x} {y}")
        extra.append(x + y)
        out, i = [], 0
        while i < len(pieces):
            if i + 1 < len(pieces) and pieces[i] == x and pieces[i + 1] == y:
                out.append(x + y)
                i += 2
            else:
                out.append(pieces[i])
                i += 1
        pieces = out
    # (tiny_json's rank-0 space+space merge needs its vocab entry too)
    extra = list(dict.fromkeys(e for e in [ENC[32] * 2] + extra if e not in ENC))
    t = BpeTokenizer.from_json(tiny_json(extra_vocab=extra, merges=merges))
    for k in range(20):
        s = "".join(rng.choice(list("ab cdé中😀\n"), int(rng.integers(0, 60))))
        ids = t.encode(s)
        assert t.decode(ids) == s
        assert 0 not in ids
    assert len(t.encode(text)) < len(data)


def test_json_escapes_match_python():
    keys = ["\\u0120a", "\\ud83d\\ude00", "tab\\t", "q\\\"", "sl\\/", "\\u00e9"]
    body = ", ".join(f'"{k}": {i + 300}' for i, k in enumerate(keys))
    raw = '{"model": {"type": "BPE", "vocab": {' + body + '}, "merges": []}, "extra": [1, 2.5e3, null, true]}'
    t = BpeTokenizer.from_json(raw)
    parsed = json.loads(raw)["model"]["vocab"]
    for k, v in parsed.items():
        got = t.decode([v]).encode()
        want = bytes(b for ch in k for b in ([ENC.index(ch)] if ch in ENC else list(ch.encode())))
        assert got == want.decode("utf-8", errors="replace").encode(), k
    assert t.vocab_size() == len(parsed)


@pytest.mark.parametrize("raw,status", [
    ('{"model": {"type": "WordPiece", "vocab": {}, "merges": []}}', IFX_E_UNSUPPORTED_TOKENIZER),
    ('{"model": {"type": "BPE", "vocab": {}, "merges": []}', IFX_E_JSON),          # unterminated
    ('{"model": {"type": "BPE", "vocab": {}, "merges": []}} x', IFX_E_JSON),       # trailing characters
    ('{"added_tokens": []}', IFX_E_JSON),                                          # missing model
    ('{"model": {"type": "BPE", "vocab": {"a": -1}, "merges": []}}', IFX_E_JSON),  # not a u32
    ('{"model": {"type": "BPE", "vocab": {"a": 1.0}, "merges": []}}', IFX_E_JSON),
    ('{"model": {"type": "BPE", "vocab": {"a": 4294967296}, "merges": []}}', IFX_E_JSON),
    ('{"model": {"type": "BPE", "vocab": {}, "merges": [["a", "b"]]}}', IFX_E_JSON),  # array merges
    ('{"model": {"type": "BPE", "vocab": {}}}', IFX_E_JSON),                       # missing merges
    ('{"model": {"type": "BPE", "type": "BPE", "vocab": {}, "merges": []}}', IFX_E_JSON),  # duplicate field
    ('{"model": {"type": "BPE", "vocab": {"\\ud800": 1}, "merges": []}}', IFX_E_JSON),    # lone surrogate
    ('{"model": {"type": "BPE", "vocab": {}, "merges": []}, "added_tokens": [{"id": 3}]}', IFX_E_JSON),
])
def test_json_errors(raw, status):
    with pytest.raises(TokenizerError) as e:
        BpeTokenizer.from_json(raw)
    assert e.value.status == status


def test_file_errors(tmp_path):
    with pytest.raises(TokenizerError) as e:
        BpeTokenizer.from_file(str(tmp_path / "missing.json"))
    assert e.value.status == IFX_E_IO
    bad = tmp_path / "bad.json"
    bad.write_bytes(b'{"model": {"type": "BPE", "vocab": {"\xff": 1}, "merges": []}}')
    with pytest.raises(TokenizerError) as e:
        BpeTokenizer.from_file(str(bad))
    assert e.value.status == IFX_E_IO
    good = tmp_path / "tok.json"
    good.write_text(tiny_json())
    assert BpeTokenizer.from_file(str(good)).encode("ok") == [ord("o") + 1, ord("k") + 1]
