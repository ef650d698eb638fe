"""Model-load failures through the chat ABI: rpg_engine_load_model returns -1
with rpg_engine_last_error set, as the reference does (reference
src/engine.cc:201-240), for the GGUF files the reference rejects
(src/gguf.cc:69-160: a file too small, a wrong magic, an unsupported
version, a tensor past the end of the file; src/model.cc:73-97: a missing
tensor, a matrix of the wrong shape). Each broken file is derived from a
valid synthetic GGUF by tests/gguf_edit.py; the reference compiled here
rejects every one of them (its messages are in Chinese, so only the failure
and a nonempty message are compared). After each failure a valid load works.

One deliberate difference: the reference accepts a one-dimensional norm gain
of the wrong length and then reads past its buffer; the GPU engine refuses
it at load."""

import ctypes
import json
import os
import struct

import pytest

import rpgbarengine_amd as eng
from gguf_edit import Gguf

pytestmark = pytest.mark.gpu


def _broken(raw):
    g = lambda: Gguf(raw)  # noqa: E731
    out = {
        "file too small": raw[:16],
        "bad magic": b"GGUX" + raw[4:],
        "unsupported version": raw[:4] + struct.pack("<I", 7) + raw[8:],
        "truncated data": raw[: len(raw) // 2],
        "tensor past the end": raw[:-1],
    }
    a = g()
    a.drop("blk.1.ffn_down.weight")
    out["missing matrix"] = a.dump()
    a = g()
    a.drop("output_norm.weight")
    out["missing norm"] = a.dump()
    a = g()
    a.reshape("blk.0.attn_q.weight", [256, 256])
    out["matrix of the wrong shape"] = a.dump()
    a = g()
    a.reshape("blk.0.attn_norm.weight", [128])
    out["norm of the wrong length"] = a.dump()
    return out


def test_broken_gguf_files_fail_cleanly(gguf_factory, tmp_path):
    L = eng.abi()
    path = gguf_factory("tiny", "q4_k_m", seed=5)
    raw = open(path, "rb").read()
    assert Gguf(raw).dump() == raw  # the rewriter reproduces a valid file
    for what, data in _broken(raw).items():
        p = str(tmp_path / "broken.gguf")
        with open(p, "wb") as f:
            f.write(data)
        h = L.rpg_engine_load_model(p.encode(), b"")
        if h >= 1:
            L.rpg_engine_unload_model(h)
        assert h == -1, f"{what}: the load succeeded"
        assert L.rpg_engine_last_error().decode(), f"{what}: no error message"
        ok = L.rpg_engine_load_model(path.encode(), b'{"max_seq": 64}')
        assert ok >= 1, f"after {what}: {L.rpg_engine_last_error().decode()}"
        s = L.rpg_engine_session_create(ok, b"")
        assert s >= 1, L.rpg_engine_last_error()
        r = L.rpg_engine_generate(s, json.dumps({"input_ids": [1, 2, 3], "max_tokens": 2}).encode())
        assert r, L.rpg_engine_last_error()
        assert len(json.loads(ctypes.string_at(r).decode())["output_ids"]) == 2
        L.rpg_engine_free(r)
        L.rpg_engine_unload_model(ok)
    assert L.rpg_engine_load_model(str(tmp_path / "absent.gguf").encode(), b"") == -1
    assert L.rpg_engine_last_error().decode()
