"""rpg_engine_generate with chat messages, end to end on the GPU: two scripted
conversations (tools, multi-turn prefix reuse, a repeated request, reset,
sampled and greedy replies, stop strings, temperature clamp, capacity and
request errors) against the responses the reference's own C ABI gave for the
same script on the same synthetic model (tests/golden/text.npz, written by
tests/golden/make_text_golden.py). Responses must be byte-identical; a call the
reference failed must fail (the messages differ in language)."""

import ctypes
import json
import os
import struct

import numpy as np
import pytest

import rpgbarengine_amd as eng
from rpgbarengine_amd import synth

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "text.npz")


def records(buf):
    b, out, i = bytes(buf), [], 0
    while i + 4 <= len(b):
        (n,) = struct.unpack_from("<I", b, i)
        out.append(b[i + 4:i + 4 + n])
        i += 4 + n
    return out


@pytest.fixture(scope="module")
def abi():
    L = ctypes.CDLL(eng.LIB_PATH)
    L.rpg_engine_load_model.argtypes = [ctypes.c_char_p, ctypes.c_char_p]
    L.rpg_engine_load_model.restype = ctypes.c_int32
    L.rpg_engine_session_create.argtypes = [ctypes.c_int32, ctypes.c_char_p]
    L.rpg_engine_session_create.restype = ctypes.c_int32
    L.rpg_engine_session_reset.argtypes = [ctypes.c_int32]
    L.rpg_engine_session_reset.restype = ctypes.c_int32
    L.rpg_engine_session_destroy.argtypes = [ctypes.c_int32]
    L.rpg_engine_unload_model.argtypes = [ctypes.c_int32]
    L.rpg_engine_generate.argtypes = [ctypes.c_int32, ctypes.c_char_p]
    L.rpg_engine_generate.restype = ctypes.c_void_p
    L.rpg_engine_free.argtypes = [ctypes.c_void_p]
    L.rpg_engine_last_error.restype = ctypes.c_char_p
    return L


@pytest.fixture(scope="module")
def model_path(tmp_path_factory):
    g = np.load(GOLDEN)
    spec = json.loads(str(g["gguf_spec"][0]))
    s = synth.PRESETS[spec["preset"]].with_(mix=synth.MIXES[spec["mix"]], seed=spec["seed"],
                                            tokenizer=spec["tokenizer"])
    return synth.write_gguf(str(tmp_path_factory.mktemp("bbpe") / "tiny_bbpe.gguf"), s)


def run_script(L, path, script):
    config, session_json, requests = script[0], script[1], script[2:]
    m = L.rpg_engine_load_model(path.encode(), config)
    assert m >= 0, L.rpg_engine_last_error()
    s = L.rpg_engine_session_create(m, session_json)
    assert s >= 0, L.rpg_engine_last_error()
    out = []
    try:
        for r in requests:
            if r == b"!reset":
                out.append(b"ok" if L.rpg_engine_session_reset(s) == 0 else b"\x01" + L.rpg_engine_last_error())
                continue
            p = L.rpg_engine_generate(s, r)
            if not p:
                out.append(b"\x01" + L.rpg_engine_last_error())
            else:
                out.append(ctypes.string_at(p))
                L.rpg_engine_free(p)
    finally:
        L.rpg_engine_session_destroy(s)
        L.rpg_engine_unload_model(m)
    return out


@pytest.mark.parametrize("name", ["engine_a", "engine_b"])
def test_chat_conversation_matches_reference_engine(abi, model_path, name):
    g = np.load(GOLDEN)
    script = records(g[f"{name}_script"])
    want = records(g[f"{name}_out"])
    got = run_script(abi, model_path, script)
    assert len(got) == len(want)
    for k, (a, b) in enumerate(zip(got, want)):
        if b.startswith(b"\x01"):
            assert a.startswith(b"\x01"), (k, a[:200])
        else:
            assert a == b, (k, script[2 + k][:120], a[:300], b[:300])
    print(f"{name}: {len(got)} calls identical to the reference engine")
