"""Several sessions decoded together (rpg_hip_generate_batch): each session
must produce exactly the tokens the oracle produces for it alone (reference
src/qwen3.cc:302-355 per session), whatever the other sessions hold --
different prompt lengths, cache sizes and sampling parameters in one batch --
and must be left ready to continue, batched or alone."""

import numpy as np
import pytest

import oracle
import rpgbarengine_amd as eng
from rpgbarengine_amd import synth

pytestmark = pytest.mark.gpu

# (prompt length, cache size, temperature, top_k, top_p, seed) per session
SESSIONS = [
    (9, 80, 0.0, 0, 1.0, 0),
    (17, 128, 0.8, 40, 0.95, 11),
    (40, 100, 0.7, 0, 0.95, 12),
    (23, 64, 0.0, 0, 0.95, 0),
    (33, 96, 1.1, 5, 1.0, 13),
]


# Past the few-token launches: a hidden size of 5120 (its RMSNorm too wide
# to stage; with 16 query heads over 2 KV heads, groups of 8) and an FFN of
# 17408 (the down input too wide): the batched step's projections take the
# GEMMs, and the one-session continuation the wave kernels
SHAPES = {"small": ("small", {}), "wide_hidden": ("tiny", dict(hidden=5120, n_heads=16)),
          "wide_ffn": ("tiny", dict(ffn=17408))}


@pytest.mark.parametrize("mix", ["q4_k_m", "q8_0"])
@pytest.mark.parametrize("shape", list(SHAPES))
def test_batch_matches_solo_oracle(gguf_factory, mix, shape):
    preset, over = SHAPES[shape]
    path = gguf_factory(preset, mix, **over)
    vocab = synth.PRESETS[preset].vocab
    om = oracle.Model(path, threads=8)
    m = eng.Model(path)
    first, second = 20, 8
    sess, want1, want2, want3 = [], [], [], []
    for i, (plen, cap, t, k, p, seed) in enumerate(SESSIONS):
        ids = synth.token_ids(70 + i, plen, vocab)
        okv = om.kv(cap)
        lg = om.forward(ids, okv)
        a, steps = om.generate(okv, lg[-1], first, t, k, p, seed, step_logits=True)
        b, steps2 = om.generate(okv, steps[-1], second, t, k, p, seed, step_logits=True)
        c = om.generate(okv, steps2[-1], 4, t, k, p, seed)
        want1.append(a)
        want2.append(b)
        want3.append(c)
        s = m.session(cap)
        s.prefill(ids)
        sess.append(s)
    T = [x[2] for x in SESSIONS]
    K = [x[3] for x in SESSIONS]
    P = [x[4] for x in SESSIONS]
    S = [x[5] for x in SESSIONS]
    got1, _ = eng.generate_batch(sess, first, T, K, P, S)
    for i in range(len(SESSIONS)):
        assert list(got1[i]) == list(want1[i]), i
        assert sess[i].len == SESSIONS[i][0] + first
    # a second batch continues each session from its own logits
    got2, _ = eng.generate_batch(sess, second, T, K, P, S)
    for i in range(len(SESSIONS)):
        assert list(got2[i]) == list(want2[i]), i
    # and each session can go on alone
    for i, s in enumerate(sess):
        got3 = s.generate(4, T[i], K[i], P[i], S[i])
        assert list(got3) == list(want3[i]), i
        assert s.len == SESSIONS[i][0] + first + second + 4


def test_batch_rejects_full_cache_and_foreign_sessions(gguf_factory):
    m = eng.Model(gguf_factory("tiny", "q8_0"))
    a, b = m.session(32), m.session(20)
    a.prefill(synth.token_ids(1, 8, 1024))
    b.prefill(synth.token_ids(2, 8, 1024))
    with pytest.raises(eng.EngineError, match="context full"):
        eng.generate_batch([a, b], 13, 0.0, 0, 1.0, 0)  # b has room for 12
    assert a.len == 8 and b.len == 8  # nothing ran
    with pytest.raises(eng.EngineError, match="twice"):
        eng.generate_batch([a, a], 2, 0.0, 0, 1.0, 0)
    m2 = eng.Model(gguf_factory("tiny", "q8_0", seed=12))
    c = m2.session(32)
    c.prefill(synth.token_ids(3, 8, 1024))
    with pytest.raises(eng.EngineError, match="different models"):
        eng.generate_batch([a, c], 2, 0.0, 0, 1.0, 0)
