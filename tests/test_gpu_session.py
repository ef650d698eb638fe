"""Session semantics of the chat ABI against the reference engine
(tests/golden/session.npz, tests/golden/make_session_golden.py): one session
answers a scripted conversation -- cached prefix reuse, a full hit that
recomputes one position, an unrelated prompt, a request that fails inside the
prefill and resets the session, and an explicit rpg_engine_session_reset --
and every answer must equal the reference's cold run of the request's whole
id list (reference src/engine.cc:383-448: reuse never changes the tokens)."""

import ctypes
import json
import os

import numpy as np
import pytest

import rpgbarengine_amd as eng
from rpgbarengine_amd import synth

pytestmark = pytest.mark.gpu

G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "session.npz"))


def _take(ptr):
    assert ptr, eng.lib().rpg_engine_last_error()
    s = ctypes.string_at(ptr).decode()
    eng.lib().rpg_engine_free(ptr)
    return json.loads(s)


def test_conversation_matches_reference_cold_runs(gguf_factory):
    T, _, _, seed, max_tokens, eos = G["params"]
    L = eng.lib()
    path = gguf_factory("tiny", "q8_0", seed=11)
    h = L.rpg_engine_load_model(path.encode(), b'{"max_seq": 256}')
    assert h >= 1, L.rpg_engine_last_error()
    s = L.rpg_engine_session_create(h, json.dumps({"max_tokens": int(max_tokens)}).encode())
    assert s >= 1, L.rpg_engine_last_error()

    def ask(i):
        ids = [int(v) for v in G[f"req{i}"]]
        req = {"input_ids": ids, "max_tokens": int(max_tokens), "temperature": float(T), "seed": int(seed)}
        r = _take(L.rpg_engine_generate(s, json.dumps(req).encode()))
        want = [int(v) for v in G[f"out{i}"]]
        assert r["output_ids"] == want, (i, r["output_ids"], want)
        assert r["usage"] == {"prompt_tokens": len(ids), "completion_tokens": len(want)}
        stopped = bool(want) and want[-1] == int(eos)
        assert r["finish_reason"] == ("stop" if stopped or len(want) < max_tokens else "length")

    for i in range(4):  # cold, prefix reuse, full hit, unrelated prompt
        ask(i)
    # a request that fails inside the prefill: the session is reset, not left
    # with a cache that disagrees with its ids
    bad = [int(v) for v in G["req0"]] + [int(v) for v in G["out0"]] + [synth.PRESETS["tiny"].vocab]
    ask(0)
    assert L.rpg_engine_generate(s, json.dumps({"input_ids": bad, "max_tokens": 4}).encode()) is None
    assert L.rpg_engine_last_error()
    ask(4)
    assert L.rpg_engine_session_reset(s) == 0
    ask(5)
    L.rpg_engine_session_destroy(s)
    L.rpg_engine_unload_model(h)
