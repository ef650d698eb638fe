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
    assert ptr, eng.abi().rpg_engine_last_error()
    s = ctypes.string_at(ptr).decode()
    eng.abi().rpg_engine_free(ptr)
    return json.loads(s)


def test_conversation_matches_reference_cold_runs(gguf_factory):
    T, _, _, seed, max_tokens, eos = G["params"]
    L = eng.abi()
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


INFO = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "info.npz"))


@pytest.mark.parametrize("case", sorted(int(k[4:]) for k in INFO.files if k.startswith("info")))
def test_model_info_matches_reference(tmp_path, case):
    """rpg_engine_model_info gives the reference's bytes (reference
    src/engine.cc:519-547: keys in its order, rope_theta as the shortest
    round-trip double, weight bytes of every tensor of the file) for the same
    model and load config, with one session open (tests/golden/info.npz,
    written by tests/golden/make_info_golden.py through the reference's own
    C ABI)."""
    preset, mix, seed, tok, cfg = json.loads(str(INFO[f"case{case}"][0]))
    spec = synth.PRESETS[preset].with_(mix=synth.MIXES[mix], seed=seed, tokenizer=tok)
    path = synth.write_gguf(str(tmp_path / f"m{case}.gguf"), spec)
    L = eng.abi()
    h = L.rpg_engine_load_model(path.encode(), cfg.encode())
    assert h >= 1, L.rpg_engine_last_error()
    try:
        s = L.rpg_engine_session_create(h, b"")
        assert s >= 1, L.rpg_engine_last_error()
        p = L.rpg_engine_model_info(h)
        assert p, L.rpg_engine_last_error()
        got = ctypes.string_at(p).decode()
        L.rpg_engine_free(p)
        want = str(INFO[f"info{case}"][0]).replace('"@PATH@"', json.dumps(path))
        assert got == want
        L.rpg_engine_session_destroy(s)
    finally:
        L.rpg_engine_unload_model(h)


def test_two_threads_two_sessions_one_model(gguf_factory):
    """The reference's threading contract (reference include/rpg_engine.h:9-14,
    src/engine.cc:87,107-112): one weight set, several sessions, one generate
    per session at a time from any host thread. Two threads run the scripted
    conversation on two sessions of one model at the same time, three times
    over with a reset between rounds; every answer equals the reference's
    cold run."""
    import threading

    T, _, _, seed, max_tokens, eos = G["params"]
    L = eng.abi()
    path = gguf_factory("tiny", "q8_0", seed=11)
    h = L.rpg_engine_load_model(path.encode(), b'{"max_seq": 256}')
    assert h >= 1, L.rpg_engine_last_error()
    errors = []
    start = threading.Barrier(2)

    def worker(tag):
        try:
            s = L.rpg_engine_session_create(h, json.dumps({"max_tokens": int(max_tokens)}).encode())
            assert s >= 1, L.rpg_engine_last_error()
            start.wait(timeout=60)
            for rnd in range(3):
                for i in (0, 1, 2, 3, 4):
                    ids = [int(v) for v in G[f"req{i}"]]
                    req = {"input_ids": ids, "max_tokens": int(max_tokens), "temperature": float(T), "seed": int(seed)}
                    p = L.rpg_engine_generate(s, json.dumps(req).encode())
                    assert p, L.rpg_engine_last_error()
                    r = json.loads(ctypes.string_at(p).decode())
                    L.rpg_engine_free(p)
                    assert r["output_ids"] == [int(v) for v in G[f"out{i}"]], (tag, rnd, i)
                assert L.rpg_engine_session_reset(s) == 0
            L.rpg_engine_session_destroy(s)
        except BaseException as e:  # reported by the main thread
            errors.append((tag, repr(e)))

    threads = [threading.Thread(target=worker, args=(t,)) for t in ("a", "b")]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    L.rpg_engine_unload_model(h)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    assert not errors, errors
