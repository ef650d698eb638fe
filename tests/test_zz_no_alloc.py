"""rpg_hip_sample_noalloc (the sampler with its scratch in a static device
array, for callers that cannot allocate) against rpg_hip_sample, the entry
point it is a variant of, and the oracle: identical token and bitwise
identical filtered probabilities, on two calls in a row, the second with a
smaller input, and a clear error above its size limit."""

import ctypes

import numpy as np
import pytest

import oracle
import rpgbarengine_amd as eng

pytestmark = pytest.mark.gpu


def _hip():
    eng.lib()  # the engine first: ctypes then binds the runtime it already loaded
    h = ctypes.CDLL("libamdhip64.so.7")
    h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    h.hipFree.argtypes = [ctypes.c_void_p]
    return h


class _Dev:
    def __init__(self, hip, nbytes):
        self.hip = hip
        self.p = ctypes.c_void_p()
        assert hip.hipMalloc(ctypes.byref(self.p), nbytes) == 0

    def put(self, a):
        a = np.ascontiguousarray(a)
        assert self.hip.hipMemcpy(self.p, a.ctypes.data, a.nbytes, 1) == 0

    def get(self, dtype, n):
        out = np.empty(n, dtype=dtype)
        assert self.hip.hipMemcpy(out.ctypes.data, self.p, out.nbytes, 2) == 0
        return out

    def free(self):
        self.hip.hipFree(self.p)


def _noalloc(hip, d_logits, d_tok, d_probs, logits, t, k, p, seed, counter):
    d_logits.put(logits)
    rc = eng.lib().rpg_hip_sample_noalloc(d_logits.p, logits.size, t, k, p, seed, counter, d_tok.p, d_probs.p, None)
    assert rc == 0, eng.lib().rpg_hip_last_error()
    assert hip.hipDeviceSynchronize() == 0
    return int(d_tok.get(np.int32, 1)[0]), d_probs.get(np.float32, logits.size)


def test_sample_noalloc_matches_sample():
    hip = _hip()
    n_max = 151936
    d_logits, d_tok, d_probs = _Dev(hip, 4 * n_max), _Dev(hip, 4), _Dev(hip, 4 * n_max)
    try:
        rng = np.random.default_rng(31)
        # call 1: the full vocabulary, the chat defaults (no top-k, top-p 0.95)
        big = (rng.standard_normal(n_max) * 0.9).astype(np.float32)
        # call 2: a smaller row whose top-p cut splits equal probabilities
        small = (rng.standard_normal(1000) * 0.9).astype(np.float32)
        small[rng.integers(0, 1000, 50)] = small.max()
        cases = [(big, 0.7, 0, 0.95, 11, 640), (small, 0.8, 40, 0.95, 12, 77)]
        for logits, t, k, p, seed, counter in cases:
            tok, probs = _noalloc(hip, d_logits, d_tok, d_probs, logits, t, k, p, seed, counter)
            want_tok, want_probs = eng.sample(logits, t, k, p, seed, counter, want_probs=True)
            assert tok == want_tok
            assert np.array_equal(probs.view(np.uint32), want_probs.view(np.uint32))
            u = oracle.counter_uniform(seed, counter)
            assert tok == oracle.sample_token(logits, t, k, p, u)
            ref_p = oracle.filter_to_probs(logits, t, k, p)
            assert np.array_equal(probs.view(np.uint32), ref_p.view(np.uint32))
        # above the static scratch: rejected with a clear message, nothing run
        rc = eng.lib().rpg_hip_sample_noalloc(d_logits.p, 1 << 19, 0.7, 0, 0.95, 1, 1, d_tok.p, None, None)
        assert rc == -1 and b"static scratch" in eng.lib().rpg_hip_last_error()
    finally:
        for d in (d_logits, d_tok, d_probs):
            d.free()
