"""Token-loop parity on synthetic GGUF models: GPU engine (C ABI) vs the CPU
oracle (the reference's own arithmetic), on identical files and prompts.

Bars: logits max|d| <= 1e-3 * max|logit|; greedy ids identical;
sampled ids identical for equal logits and seed."""

import json

import numpy as np
import pytest

import oracle
import rpgbarengine_amd as eng
from rpgbarengine_amd import synth

pytestmark = pytest.mark.gpu


def _logit_ok(got, want):
    return float(np.max(np.abs(got - want))) <= 1e-3 * float(np.max(np.abs(want)))


@pytest.mark.parametrize("mix", ["q8_0", "q4_k_m", "f32", "q6_k", "other"])
def test_prefill_logits_and_kv(gguf_factory, mix):
    path = gguf_factory("small", mix)
    ids = synth.token_ids(3, 24, synth.PRESETS["small"].vocab)
    om = oracle.Model(path, threads=8)
    okv = om.kv(64)
    want = om.forward(ids, okv)
    m = eng.Model(path)
    s = m.session(64)
    got = s.prefill(ids, all_logits=True)
    assert s.len == ids.size
    for t in range(ids.size):
        assert _logit_ok(got[t], want[t]), t
    # the cache holds the same K/V (fp32, tolerance of the fused matvec)
    for layer in (0, m.n_layers - 1):
        for head in range(m.n_kv_heads):
            for which in (0, 1):
                g = s.kv(which, layer, head, ids.size)
                w = okv.read(which, layer, head, ids.size)
                assert np.max(np.abs(g - w)) <= 1e-4 * max(1.0, float(np.max(np.abs(w))))


@pytest.mark.parametrize("mix", ["q4_k_m", "q8_0", "other"])
def test_engine_matches_reference_golden(mix):
    """Against the vectors the reference engine itself wrote
    (tests/golden/make_golden.py): last-token logits within the bar, greedy
    and sampled ids identical."""
    import os
    g = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz"))
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        spec = synth.PRESETS["tiny"].with_(mix=synth.MIXES[mix], seed=11)
        path = synth.write_gguf(os.path.join(d, f"tiny_{mix}.gguf"), spec)
        m = eng.Model(path)
        ids = g[f"model_{mix}_ids"]
        s = m.session(64)
        last = s.prefill(ids)
        assert _logit_ok(last, g[f"model_{mix}_last_logits"])
        assert list(s.generate(len(g[f"model_{mix}_greedy"]))) == list(g[f"model_{mix}_greedy"])
        s2 = m.session(64)
        s2.prefill(ids)
        got = s2.generate(len(g[f"model_{mix}_sampled"]), temperature=0.8, top_k=40, top_p=0.95, seed=77)
        assert list(got) == list(g[f"model_{mix}_sampled"])


def test_prefill_chunked_equals_whole(gguf_factory):
    """Prefill in two segments == prefill at once (prefix reuse path)."""
    path = gguf_factory("tiny", "q4_k_m")
    ids = synth.token_ids(4, 20, synth.PRESETS["tiny"].vocab)
    m = eng.Model(path)
    a = m.session(64)
    whole = a.prefill(ids)
    b = m.session(64)
    b.prefill(ids[:13])
    part = b.prefill(ids[13:])
    assert b.len == 20
    assert np.max(np.abs(whole - part)) <= 1e-5 * float(np.max(np.abs(whole)))


@pytest.mark.parametrize("mix", ["q8_0", "q4_k_m", "other"])
def test_greedy_ids_identical(gguf_factory, mix):
    path = gguf_factory("small", mix)
    ids = synth.token_ids(8, 32, synth.PRESETS["small"].vocab)
    om = oracle.Model(path, threads=8)
    okv = om.kv(256)
    lg = om.forward(ids, okv)
    want = om.generate(okv, lg[-1], 64)
    m = eng.Model(path)
    s = m.session(256)
    s.prefill(ids)
    got = s.generate(64)
    assert list(got) == list(want)
    assert s.len == ids.size + 64  # every returned token was forwarded


@pytest.mark.parametrize("temperature,top_k,top_p", [(0.8, 40, 0.95), (0.7, 0, 0.95)])
def test_sampled_ids_identical(gguf_factory, temperature, top_k, top_p):
    path = gguf_factory("small", "q4_k_m")
    ids = synth.token_ids(9, 40, synth.PRESETS["small"].vocab)
    om = oracle.Model(path, threads=8)
    okv = om.kv(256)
    lg = om.forward(ids, okv)
    want = om.generate(okv, lg[-1], 64, temperature, top_k, top_p, seed=2024)
    m = eng.Model(path)
    s = m.session(256)
    s.prefill(ids)
    got = s.generate(64, temperature, top_k, top_p, seed=2024)
    assert list(got) == list(want)


def test_step_logits_track_oracle(gguf_factory):
    path = gguf_factory("small", "q8_0")
    ids = synth.token_ids(12, 16, synth.PRESETS["small"].vocab)
    om = oracle.Model(path, threads=8)
    okv = om.kv(128)
    lg = om.forward(ids, okv)
    want_ids, want_steps = om.generate(okv, lg[-1], 24, step_logits=True)
    m = eng.Model(path)
    s = m.session(128)
    s.prefill(ids)
    got_ids, got_steps = s.generate(24, step_logits=True)
    assert list(got_ids) == list(want_ids)
    for i in range(len(want_ids)):
        assert _logit_ok(got_steps[i], want_steps[i]), i


def test_prefill_in_passes_tracks_oracle(gguf_factory):
    """A prompt longer than one prefill pass (4500 tokens: passes of 4096 and
    404, the second attending over the first's cache), then greedy decode:
    the last position's logits and every step's within 1e-3 of max|logit|,
    the ids identical; and every position's logits of a 700-token prompt
    (passes of 512 and 188 while all rows are returned)."""
    path = gguf_factory("tiny", "q4_k_m", context_length=8192)
    vocab = synth.PRESETS["tiny"].vocab
    ids = synth.token_ids(23, 4500, vocab)
    om = oracle.Model(path, threads=8, max_pos=8192)
    okv = om.kv(4520)
    lg = om.forward(ids, okv)
    want_ids, want_steps = om.generate(okv, lg[-1], 6, step_logits=True)
    m = eng.Model(path, max_pos=8192)
    s = m.session(4520)
    last = s.prefill(ids)
    assert s.len == ids.size
    assert _logit_ok(last, lg[-1])
    got_ids, got_steps = s.generate(6, step_logits=True)
    assert list(got_ids) == list(want_ids)
    for i in range(len(want_ids)):
        assert _logit_ok(got_steps[i], want_steps[i]), i
    ids2 = synth.token_ids(24, 700, vocab)
    okv2 = om.kv(720)
    want = om.forward(ids2, okv2)
    s2 = m.session(720)
    got = s2.prefill(ids2, all_logits=True)
    assert got.shape == want.shape
    for t in range(ids2.size):
        assert _logit_ok(got[t], want[t]), t


@pytest.mark.parametrize("mix", ["q4_k_m", "q8_0"])
@pytest.mark.parametrize("hidden,n_heads,ffn", [(256, 16, 12288), (256, 10, 17408), (256, 16, 25600),
                                                (5120, 8, 512)])
def test_larger_model_shapes_track_oracle(gguf_factory, mix, hidden, n_heads, ffn):
    """The shapes of the larger Qwen3 models: feed-forward widths of 12288,
    17408 and 25600 (the down projection's input wider than 10240: the wide
    operand split of the GEMMs; at decode the wave kernels, past 14563 with
    more than 64 KiB of LDS), groups of 5 and 8 query heads per KV head, and
    a hidden size of 5120 (its RMSNorm wider than the decode launches fold
    into their staging: normed first). A 130-token prefill (the GEMMs), a
    40-token segment after it (the few-token launches where they take the
    shape), then greedy decode: logits within 1e-3 of max|logit| at every
    step, ids identical."""
    path = gguf_factory("tiny", mix, hidden=hidden, n_heads=n_heads, ffn=ffn)
    vocab = synth.PRESETS["tiny"].vocab
    ids = synth.token_ids(25, 170, vocab)
    om = oracle.Model(path, threads=8)
    okv = om.kv(200)
    lg1 = om.forward(ids[:130], okv)
    lg2 = om.forward(ids[130:], okv)
    want_ids, want_steps = om.generate(okv, lg2[-1], 8, step_logits=True)
    m = eng.Model(path)
    s = m.session(200)
    assert _logit_ok(s.prefill(ids[:130]), lg1[-1])
    assert _logit_ok(s.prefill(ids[130:]), lg2[-1])
    got_ids, got_steps = s.generate(8, step_logits=True)
    assert list(got_ids) == list(want_ids)
    for i in range(len(want_ids)):
        assert _logit_ok(got_steps[i], want_steps[i]), i


@pytest.mark.parametrize("otype", [synth.Q6_K, synth.Q8_0])
def test_untied_output_matrix_tracks_oracle(gguf_factory, tmp_path, otype):
    """A GGUF with its own output.weight (the larger Qwen3 models do not tie
    it to the embedding; reference src/model.cc:214-222): the file of the
    tied model with an output matrix of other values appended. Prefill logits,
    greedy ids and step logits follow the oracle, and they differ from the
    tied model's (the matrix is the one read)."""
    from gguf_edit import Gguf
    base = gguf_factory("tiny", "q4_k_m")
    spec = synth.PRESETS["tiny"]
    g = Gguf(open(base, "rb").read())
    assert "output.weight" not in g.names()
    w32 = synth.gaussian(41, 7, spec.vocab * spec.hidden, 0.02).reshape(spec.vocab, spec.hidden)
    raw = synth.quantize(otype, w32).tobytes()
    pad = (-len(g.body)) % g.alignment
    off = len(g.body) + pad
    g.body = g.body + b"\0" * pad + raw
    g.tensors.append(["output.weight", [spec.hidden, spec.vocab], otype, off])
    path = str(tmp_path / "untied.gguf")
    with open(path, "wb") as f:
        f.write(g.dump())
    ids = synth.token_ids(27, 40, spec.vocab)
    om = oracle.Model(path, threads=8)
    okv = om.kv(128)
    lg = om.forward(ids, okv)
    want_ids, want_steps = om.generate(okv, lg[-1], 16, step_logits=True)
    tied = oracle.Model(base, threads=8).forward(ids)
    assert float(np.max(np.abs(tied[-1] - lg[-1]))) > 1e-2 * float(np.max(np.abs(lg[-1])))
    m = eng.Model(path)
    s = m.session(128)
    assert _logit_ok(s.prefill(ids), lg[-1])
    got_ids, got_steps = s.generate(16, step_logits=True)
    assert list(got_ids) == list(want_ids)
    for i in range(len(want_ids)):
        assert _logit_ok(got_steps[i], want_steps[i]), i


def test_large_capacity_session_tracks_oracle(gguf_factory):
    """A session of 20000 positions (past 8192; the cache strided by it,
    decode over 32 splits of whole tiles): a 1100-token prefill and greedy
    decode give the oracle's logits and ids."""
    path = gguf_factory("tiny", "q8_0", context_length=32768)
    ids = synth.token_ids(26, 1100, synth.PRESETS["tiny"].vocab)
    om = oracle.Model(path, threads=8, max_pos=20000)
    okv = om.kv(20000)
    lg = om.forward(ids, okv)
    want_ids, want_steps = om.generate(okv, lg[-1], 8, step_logits=True)
    m = eng.Model(path, max_pos=20000)
    s = m.session(20000)
    assert _logit_ok(s.prefill(ids), lg[-1])
    got_ids, got_steps = s.generate(8, step_logits=True)
    assert list(got_ids) == list(want_ids)
    for i in range(len(want_ids)):
        assert _logit_ok(got_steps[i], want_steps[i]), i


def test_long_context_decode_tracks_oracle(gguf_factory):
    """Decode attention past 2048 positions: more than 64 splits of 32
    positions (the merge's second group of (max, sum) records and its second
    batch of outputs), a prompt that is not a multiple of the split, steps
    that cross a split boundary (2112), and a cache size that is not one
    either."""
    path = gguf_factory("tiny", "q8_0")
    ids = synth.token_ids(21, 2105, synth.PRESETS["tiny"].vocab)
    om = oracle.Model(path, threads=8)
    okv = om.kv(2213)
    lg = om.forward(ids, okv)
    want_ids, want_steps = om.generate(okv, lg[-1], 12, step_logits=True)
    m = eng.Model(path)
    s = m.session(2213)
    s.prefill(ids)
    got_ids, got_steps = s.generate(12, step_logits=True)
    assert list(got_ids) == list(want_ids)
    for i in range(len(want_ids)):
        assert _logit_ok(got_steps[i], want_steps[i]), i


@pytest.mark.parametrize("mix", ["q4_k_m", "q6_k"])
@pytest.mark.parametrize("persistent", [False, True])
def test_decode_paths_track_oracle(gguf_factory, monkeypatch, mix, persistent):
    """Both decode paths -- one launch per projection (the default) and the
    opt-in persistent step (RPG_DECODE_STEP=1, one launch per token) -- give
    the oracle's greedy ids and step logits, and its sampled ids."""
    if persistent:
        monkeypatch.setenv("RPG_DECODE_STEP", "1")
    else:
        monkeypatch.delenv("RPG_DECODE_STEP", raising=False)
    path = gguf_factory("small", mix)
    ids = synth.token_ids(15, 21, synth.PRESETS["small"].vocab)
    om = oracle.Model(path, threads=8)
    okv = om.kv(160)
    lg = om.forward(ids, okv)
    want_ids, want_steps = om.generate(okv, lg[-1], 40, step_logits=True)
    m = eng.Model(path)
    s = m.session(160)
    assert s.persistent_decode == persistent
    s.prefill(ids)
    got_ids, got_steps = s.generate(40, step_logits=True)
    assert list(got_ids) == list(want_ids)
    for i in range(len(want_ids)):
        assert _logit_ok(got_steps[i], want_steps[i]), i
    # sampled, every step queued at once
    okv2 = om.kv(160)
    lg2 = om.forward(ids, okv2)
    want_s = om.generate(okv2, lg2[-1], 48, 0.8, 40, 0.95, seed=31)
    s2 = m.session(160)
    s2.prefill(ids)
    assert list(s2.generate(48, 0.8, 40, 0.95, seed=31)) == list(want_s)


def test_persistent_decode_long_context(gguf_factory, monkeypatch):
    """The persistent step past 2048 positions (more than 64 attention
    splits per KV head) against the oracle."""
    monkeypatch.setenv("RPG_DECODE_STEP", "1")
    path = gguf_factory("tiny", "q4_k_m")
    ids = synth.token_ids(22, 2100, synth.PRESETS["tiny"].vocab)
    om = oracle.Model(path, threads=8)
    okv = om.kv(2200)
    lg = om.forward(ids, okv)
    want_ids, want_steps = om.generate(okv, lg[-1], 16, step_logits=True)
    m = eng.Model(path)
    s = m.session(2200)
    assert s.persistent_decode
    s.prefill(ids)
    got_ids, got_steps = s.generate(16, step_logits=True)
    assert list(got_ids) == list(want_ids)
    for i in range(len(want_ids)):
        assert _logit_ok(got_steps[i], want_steps[i]), i


def test_stop_ids_and_cache_length(gguf_factory):
    path = gguf_factory("tiny", "q8_0")
    ids = synth.token_ids(13, 8, synth.PRESETS["tiny"].vocab)
    m = eng.Model(path)
    s = m.session(128)
    s.prefill(ids)
    free_run = s.generate(30)
    stop = int(free_run[5])
    first = int(np.nonzero(free_run == stop)[0][0])
    s2 = m.session(128)
    s2.prefill(ids)
    got = s2.generate(30, stop_ids=[stop])
    assert list(got) == list(free_run[: first + 1])  # stop id included
    assert s2.len == ids.size + first + 1


def test_continue_after_stop_matches_oracle(gguf_factory):
    """A stop id early in a batch of queued steps, then a continuation from
    the device logits (first_logits = None): the continuation starts from the
    logits after the stop token, as the oracle's does."""
    path = gguf_factory("tiny", "q8_0")
    ids = synth.token_ids(13, 8, synth.PRESETS["tiny"].vocab)
    m = eng.Model(path)
    s = m.session(128)
    s.prefill(ids)
    free_run = s.generate(30)
    stop = int(free_run[3])
    first = int(np.nonzero(free_run == stop)[0][0])
    assert first < 15  # inside the first batch of queued steps
    om = oracle.Model(path, threads=4)
    okv = om.kv(128)
    lg = om.forward(ids, okv)
    want, steps = om.generate(okv, lg[-1], 30, stop_ids=[stop], step_logits=True)
    want_cont = om.generate(okv, steps[-1], 12)
    s2 = m.session(128)
    s2.prefill(ids)
    got = s2.generate(30, stop_ids=[stop])
    assert list(got) == list(want)
    cont = s2.generate(12)
    assert list(cont) == list(want_cont)
    assert s2.len == ids.size + len(want) + 12


def test_graph_recaptured_after_scratch_growth(gguf_factory):
    """The captured decode graph holds pointers into the session's scratch
    buffers. A longer prefill reallocates them (the graph is dropped first),
    and the next generate captures anew: its tokens continue the
    conversation exactly as the oracle's do."""
    path = gguf_factory("tiny", "q4_k_m")
    vocab = synth.PRESETS["tiny"].vocab
    a, b = synth.token_ids(31, 6, vocab), synth.token_ids(32, 70, vocab)
    om = oracle.Model(path, threads=4)
    okv = om.kv(200)
    lg = om.forward(a, okv)
    want1 = om.generate(okv, lg[-1], 10, 0.8, 40, 0.95, seed=5)
    lg2 = om.forward(b, okv)
    want2 = om.generate(okv, lg2[-1], 10, 0.8, 40, 0.95, seed=6)
    m = eng.Model(path)
    s = m.session(200)
    s.prefill(a)  # scratch for 6 tokens
    assert list(s.generate(10, 0.8, 40, 0.95, 5)) == list(want1)  # graph captured on it
    s.prefill(b)  # 70 tokens: the scratch grows
    assert list(s.generate(10, 0.8, 40, 0.95, 6)) == list(want2)
    assert s.len == 6 + 10 + 70 + 10


def test_context_full_raises(gguf_factory):
    path = gguf_factory("tiny", "q8_0")
    m = eng.Model(path)
    s = m.session(12)
    s.prefill(synth.token_ids(14, 8, synth.PRESETS["tiny"].vocab))
    with pytest.raises(eng.EngineError, match="context full"):
        s.generate(10)


def test_bad_token_rejected(gguf_factory):
    path = gguf_factory("tiny", "q8_0")
    m = eng.Model(path)
    s = m.session(16)
    with pytest.raises(eng.EngineError):
        s.prefill(np.array([1, 2, m.vocab], np.int32))
    assert s.len == 0


def test_rope_table_bitexact(gguf_factory):
    path = gguf_factory("tiny", "q8_0")
    m = eng.Model(path)
    om = oracle.Model(path, threads=1)
    for pos in (0, 1, 7, 1000, 4095):
        want = np.empty(m.head_dim, np.float32)
        oracle.lib().orc_rope_row(om.h, pos, want.ctypes.data)
        assert np.array_equal(m.rope_row(pos).view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------- chat ABI

def _abi_call(fn, *args):
    L = eng.abi()
    return getattr(L, fn)(*args)


def test_abi_lifecycle_and_generate(gguf_factory):
    path = gguf_factory("tiny", "q8_0")
    L = eng.abi()
    h = L.rpg_engine_load_model(path.encode(), b'{"max_seq": 256}')
    assert h >= 1, L.rpg_engine_last_error()
    info = json.loads(_take(L.rpg_engine_model_info(h)))
    assert info["n_layers"] == 2 and info["vocab"] == 1024 and info["tied_embeddings"] is True
    s = L.rpg_engine_session_create(h, b'{"max_tokens": 16}')
    assert s >= 1
    ids = [int(v) for v in synth.token_ids(21, 10, 1024)]
    req = json.dumps({"input_ids": ids, "max_tokens": 12}).encode()
    r1 = json.loads(_take(L.rpg_engine_generate(s, req)))
    assert set(r1) >= {"text", "tool_calls", "finish_reason", "usage"}
    assert r1["usage"] == {"prompt_tokens": 10, "completion_tokens": len(r1["output_ids"])}
    # warm == cold: a fresh session given the same request returns the same ids
    s2 = L.rpg_engine_session_create(h, b'{"max_tokens": 16}')
    r2 = json.loads(_take(L.rpg_engine_generate(s2, req)))
    assert r1["output_ids"] == r2["output_ids"]
    # continuing the conversation reuses the cached prefix
    req3 = json.dumps({"input_ids": ids + r1["output_ids"] + [5, 6], "max_tokens": 4}).encode()
    r3 = json.loads(_take(L.rpg_engine_generate(s, req3)))
    s3 = L.rpg_engine_session_create(h, None)
    r3c = json.loads(_take(L.rpg_engine_generate(s3, req3)))
    assert r3["output_ids"] == r3c["output_ids"]
    assert L.rpg_engine_session_reset(s) == 0
    L.rpg_engine_session_destroy(s)
    assert L.rpg_engine_generate(s, req) is None
    assert b"invalid session" in L.rpg_engine_last_error()
    L.rpg_engine_unload_model(h)
    assert L.rpg_engine_generate(s2, req) is None  # cascaded
    L.rpg_engine_unload_model(h)  # no-op


def test_abi_errors_do_not_throw(gguf_factory):
    L = eng.abi()
    assert L.rpg_engine_load_model(b"/nonexistent.gguf", None) == -1
    assert L.rpg_engine_last_error()
    path = gguf_factory("tiny", "q8_0")
    h = L.rpg_engine_load_model(path.encode(), b"not json")
    assert h == -1 and b"JSON" in L.rpg_engine_last_error()
    h = L.rpg_engine_load_model(path.encode(), None)
    s = L.rpg_engine_session_create(h, b'{"max_seq": 40}')
    too_long = json.dumps({"input_ids": list(range(30)), "max_tokens": 20}).encode()
    assert L.rpg_engine_generate(s, too_long) is None
    assert b"too long" in L.rpg_engine_last_error()
    L.rpg_engine_unload_model(h)


def _take(ptr):
    assert ptr, eng.abi().rpg_engine_last_error()
    import ctypes
    s = ctypes.string_at(ptr).decode()
    eng.abi().rpg_engine_free(ptr)
    return s


@pytest.mark.parametrize("preset", ["tiny", "mid"])
def test_greedy_pick_ties_and_nan(gguf_factory, preset):
    """The decode step's greedy pick (one token from given logits) is the
    reference's ArgMax (src/kernels.h:42-52: strict > from index 0): the
    first of equal maxima, NaN never chosen, a NaN at index 0 gives 0, an
    all -inf row gives 0, -0 and +0 are equal. The 32000-entry vocabulary spreads the row over
    eight workgroups of 4096 logits: equal maxima in different workgroups,
    the later ones finishing first or last, still give the first."""
    path = gguf_factory(preset, "q8_0")
    m = eng.Model(path)
    s = m.session(64)
    V = m.vocab
    s.prefill(synth.token_ids(3, 4, V))
    rng = np.random.default_rng(9)
    cases = []
    x = rng.standard_normal(V).astype(np.float32)
    x[[17, V // 2, V - 123]] = 9.0
    cases.append((x, 17))
    x = rng.standard_normal(V).astype(np.float32)
    x[[V - 1, V // 3 + 1, V // 3]] = 11.0
    cases.append((x, V // 3))
    x = rng.standard_normal(V).astype(np.float32)
    x[V - 1] = 50.0
    cases.append((x, V - 1))
    x = rng.standard_normal(V).astype(np.float32)
    x[0] = np.nan
    x[33] = 40.0
    cases.append((x, 0))
    x = rng.standard_normal(V).astype(np.float32)
    x[[5, 6]] = np.nan
    x[7] = 30.0
    cases.append((x, 7))
    cases.append((np.full(V, -np.inf, dtype=np.float32), 0))
    x = np.full(V, -np.inf, dtype=np.float32)
    x[V - 2] = -1e30
    cases.append((x, V - 2))
    # a maximum of zero held as -0 first and +0 later (in another workgroup)
    x = -np.abs(rng.standard_normal(V)).astype(np.float32) - 1.0
    x[3] = -0.0
    x[V - 5] = 0.0
    cases.append((x, 3))
    for x, want in cases:
        s.set_len(4)
        got = s.generate(1, first_logits=x)
        assert int(got[0]) == want == int(oracle.lib().orc_argmax(oracle._p(x), V))
    s.close()
    m.close()
