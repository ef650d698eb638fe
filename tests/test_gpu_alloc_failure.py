"""Out-of-memory contract of the chat ABI (reference src/engine.cc:175-191,
442-448): a device allocation that fails inside a call makes the call return
-1 / NULL with rpg_engine_last_error set; a failed prefill resets the session;
and the next request answers exactly as the reference's cold run of its ids
(tests/golden/session.npz, tests/golden/make_session_golden.py).

Failures are injected on the host with rpg_hip_fail_alloc_after(k): the
allocation after k successful ones fails as an out-of-memory hipMalloc would,
without calling it, so every allocation of a model load, a session creation
and a scratch regrowth is made to fail in turn. No kernel ever runs on a
missing buffer: the session refuses to enqueue work without its scratch."""

import ctypes
import json
import os

import numpy as np
import pytest

import rpgbarengine_amd as eng

pytestmark = pytest.mark.gpu

G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "session.npz"))
T, _, _, SEED, MAX_TOKENS, EOS = G["params"]


def _take(L, ptr):
    assert ptr, L.rpg_engine_last_error()
    s = ctypes.string_at(ptr).decode()
    L.rpg_engine_free(ptr)
    return json.loads(s)


def _request(i=None, ids=None):
    ids = [int(v) for v in (G[f"req{i}"] if ids is None else ids)]
    return json.dumps({"input_ids": ids, "max_tokens": int(MAX_TOKENS), "temperature": float(T),
                       "seed": int(SEED)}).encode()


def _ask(L, s, i):
    r = _take(L, L.rpg_engine_generate(s, _request(i)))
    assert r["output_ids"] == [int(v) for v in G[f"out{i}"]], (i, r["output_ids"])


@pytest.fixture(scope="module")
def model(gguf_factory):
    L = eng.lib()
    path = gguf_factory("tiny", "q8_0", seed=11)
    h = L.rpg_engine_load_model(path.encode(), b'{"max_seq": 256}')
    assert h >= 1, L.rpg_engine_last_error()
    yield L, h, path
    eng.fail_alloc_after(-1)
    L.rpg_engine_unload_model(h)


def test_failed_scratch_growth_leaves_a_usable_session(model):
    """A request whose prefill must grow the session's scratch (39 tokens
    after 20 and 15) meets a failed allocation at each of its buffers in
    turn. The call fails cleanly and resets the session; the next request --
    whose 20 tokens fit the capacity the session held before -- and a
    prefix-reusing one after it give the reference's ids."""
    L, h, _ = model
    failed = 0
    for k in range(14):
        s = L.rpg_engine_session_create(h, json.dumps({"max_tokens": int(MAX_TOKENS)}).encode())
        assert s >= 1, L.rpg_engine_last_error()
        try:
            _ask(L, s, 0)  # A: 20 tokens
            _ask(L, s, 3)  # C: 15 tokens, nothing reused
            eng.fail_alloc_after(k)
            r = L.rpg_engine_generate(s, _request(1))  # A + out0 + B: 39 tokens, cold after C
            eng.fail_alloc_after(-1)
            if r:
                got = json.loads(ctypes.string_at(r).decode())
                L.rpg_engine_free(r)
                assert got["output_ids"] == [int(v) for v in G["out1"]]
            else:
                failed += 1
                err = L.rpg_engine_last_error().decode()
                assert "OutOfMemory" in err, err
            _ask(L, s, 0)
            _ask(L, s, 1)
        finally:
            eng.fail_alloc_after(-1)
            L.rpg_engine_session_destroy(s)
    assert failed >= 8, f"only {failed} of the allocations were reached"


def test_failed_session_creation_and_model_load(model):
    """Session creation and model load fail cleanly at each of their
    allocations, and the handles created afterwards work."""
    L, h, path = model
    failed = 0
    for k in range(24):
        eng.fail_alloc_after(k)
        s = L.rpg_engine_session_create(h, json.dumps({"max_tokens": int(MAX_TOKENS)}).encode())
        eng.fail_alloc_after(-1)
        if s < 0:
            failed += 1
            assert "OutOfMemory" in L.rpg_engine_last_error().decode()
        else:
            L.rpg_engine_session_destroy(s)
    assert failed >= 10
    for k in range(4):
        eng.fail_alloc_after(k)
        h2 = L.rpg_engine_load_model(path.encode(), b'{"max_seq": 256}')
        eng.fail_alloc_after(-1)
        if h2 >= 1:
            L.rpg_engine_unload_model(h2)
        else:
            assert "OutOfMemory" in L.rpg_engine_last_error().decode()
    s = L.rpg_engine_session_create(h, json.dumps({"max_tokens": int(MAX_TOKENS)}).encode())
    assert s >= 1, L.rpg_engine_last_error()
    try:
        _ask(L, s, 0)
        _ask(L, s, 1)
    finally:
        L.rpg_engine_session_destroy(s)
