"""The text front-end (include/rpg_text.h, the code rpg_engine_generate runs
around the GPU token loop) against what the reference itself produced for the
same inputs (tests/golden/text.npz, written by tests/golden/make_text_golden.py
from the reference compiled here): the Unicode classes of every code point,
the BBPE tokenizer on a synthetic Qwen-style vocabulary (encode with and
without special tokens, pre-tokenizer pieces, decode with and without
specials), ChatML rendering, reply parsing and JSON writing -- all byte for
byte. CPU only."""

import json
import os
import struct

import numpy as np
import pytest

from rpgbarengine_amd import synth
from rpgbarengine_amd import text

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "text.npz")


@pytest.fixture(scope="module")
def g():
    return np.load(GOLDEN)


def records(buf):
    b, out, i = bytes(buf), [], 0
    while i + 4 <= len(b):
        (n,) = struct.unpack_from("<I", b, i)
        out.append(b[i + 4:i + 4 + n])
        i += 4 + n
    assert i == len(b)
    return out


def text_results(buf, n_texts):
    """Per text: three id records (u32 count + int32 ids) then two byte
    records (u32 length + bytes)."""
    b, out, i = bytes(buf), [], 0
    for _ in range(n_texts):
        one = []
        for kind in ("ids", "ids", "ids", "bytes", "bytes"):
            (n,) = struct.unpack_from("<I", b, i)
            size = 4 * n if kind == "ids" else n
            chunk = b[i + 4:i + 4 + size]
            one.append(np.frombuffer(chunk, dtype=np.int32) if kind == "ids" else chunk)
            i += 4 + size
        out.append(one)
    assert i == len(b)
    return out


@pytest.fixture(scope="module")
def tok(g, tmp_path_factory):
    spec = json.loads(str(g["gguf_spec"][0]))
    s = synth.PRESETS[spec["preset"]].with_(mix=synth.MIXES[spec["mix"]], seed=spec["seed"],
                                            tokenizer=spec["tokenizer"])
    path = synth.write_gguf(str(tmp_path_factory.mktemp("bbpe") / "tiny_bbpe.gguf"), s)
    t = text.Tokenizer(path)
    yield t
    t.close()


def test_unicode_classes_of_every_code_point(g):
    """Letter / number / space of U+0000..U+10FFFF as the reference classifies
    them (Unicode 15.1)."""
    want = g["unicode_classes"]
    got = text.char_classes(0, 0x110000)
    diff = np.nonzero(got != want)[0]
    assert diff.size == 0, [hex(int(c)) for c in diff[:20]]
    # a plausible slip would move whole classes: these must hold
    assert want[ord("a")] == 1 and want[ord("7")] == 2 and want[ord(" ")] == 4 and want[0x3000] == 4
    assert want[0x4E2D] == 1 and want[0x2167] == 2 and want[0x0301] == 0 and want[0x200B] == 0


def test_tokenizer_matches_reference(g, tok):
    """Per text: special-aware ids, plain ids, pre-tokenizer pieces, decode
    with and without specials -- identical to the reference's."""
    ins = records(g["text_in"])
    for k, (t, (ids, plain, pieces, dec, dec_skip)) in enumerate(zip(ins, text_results(g["text_out"], len(ins)))):
        got = tok.encode(t, parse_special=True)
        assert np.array_equal(got, ids), (k, t[:60])
        assert np.array_equal(tok.encode(t, parse_special=False), plain), (k, t[:60])
        assert [len(p) for p in tok.split(t)] == pieces.tolist(), (k, t[:60])
        assert tok.decode(got) == dec, (k, t[:60])
        assert tok.decode(got, skip_special=True) == dec_skip, (k, t[:60])


def test_tokenizer_round_trip_and_specials(tok):
    """Decode inverts encode on any bytes (byte-level BPE); a special token
    string is one id only when special tokens are parsed."""
    rng = np.random.default_rng(3)
    for _ in range(50):
        b = bytes(rng.integers(0, 256, size=int(rng.integers(1, 200)), dtype=np.uint8))
        assert tok.decode(tok.encode(b)) == b
    one = tok.encode("<|im_end|>")
    assert one.size == 1
    assert tok.encode("<|im_end|>", parse_special=False).size > 1


def test_chatml_matches_reference(g):
    ins = records(g["chatml_in"])
    outs = records(g["chatml_out"])
    assert len(ins) == len(outs)
    for k, (req, want) in enumerate(zip(ins, outs)):
        assert text.render_chatml(req) == want, (k, req[:80])


def test_reply_parse_matches_reference(g):
    ins = records(g["reply_in"])
    outs = records(g["reply_out"])
    assert len(ins) == len(outs)
    for k, (r, want) in enumerate(zip(ins, outs)):
        assert text.parse_reply(r) == want, (k, r[:80])


def test_json_writing_matches_reference(g):
    """Compact and json.dumps-style writing of parsed documents (number forms,
    key order, duplicate keys, escapes, surrogates); documents the reference
    rejects are rejected."""
    ins = records(g["json_in"])
    outs = records(g["json_out"])
    assert len(outs) == 2 * len(ins)
    for k, doc in enumerate(ins):
        compact, python = outs[2 * k], outs[2 * k + 1]
        if compact.startswith(b"\x01"):
            with pytest.raises(text.EngineError):
                text.json_redump(doc, False)
            continue
        assert text.json_redump(doc, False) == compact, (k, doc)
        assert text.json_redump(doc, True) == python, (k, doc)
