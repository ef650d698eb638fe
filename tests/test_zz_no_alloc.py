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


def _capture_main():
    """Child process: the first call of rpg_hip_sample_noalloc in the process
    happens under stream capture (its per-device symbol lookup included);
    the graph is replayed with new logits each time and every replay is
    compared bit for bit with rpg_hip_sample. Prints "capture ok"."""
    hip = _hip()
    hip.hipStreamCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    hip.hipStreamBeginCapture.argtypes = [ctypes.c_void_p, ctypes.c_int]
    hip.hipStreamEndCapture.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]
    hip.hipGraphInstantiate.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_size_t]
    hip.hipGraphLaunch.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
    hip.hipGraphExecDestroy.argtypes = [ctypes.c_void_p]
    hip.hipGraphDestroy.argtypes = [ctypes.c_void_p]
    hip.hipStreamDestroy.argtypes = [ctypes.c_void_p]
    stream = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(stream)) == 0
    rng = np.random.default_rng(41)
    # (vocabulary, temperature, top-k, top-p, seed, counter): the chat
    # defaults over the full vocabulary (the launch chain over slices), and
    # a top-k row
    for n, t, k, p, seed, counter in [(151936, 0.7, 0, 0.95, 21, 900), (151936, 0.8, 40, 0.95, 22, 901)]:
        d_logits, d_tok, d_probs = _Dev(hip, 4 * n), _Dev(hip, 4), _Dev(hip, 4 * n)
        d_logits.put(np.zeros(n, dtype=np.float32))
        graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
        assert hip.hipStreamBeginCapture(stream, 1) == 0  # thread-local mode
        rc = eng.lib().rpg_hip_sample_noalloc(d_logits.p, n, t, k, p, seed, counter, d_tok.p, d_probs.p, stream)
        assert hip.hipStreamEndCapture(stream, ctypes.byref(graph)) == 0
        assert rc == 0, eng.lib().rpg_hip_last_error()
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        got = []
        rows = [(rng.standard_normal(n) * s).astype(np.float32) for s in (0.9, 2.0, 0.5)]
        for logits in rows:
            d_logits.put(logits)  # between replays, outside the graph
            assert hip.hipGraphLaunch(exe, stream) == 0
            assert hip.hipStreamSynchronize(stream) == 0
            got.append((int(d_tok.get(np.int32, 1)[0]), d_probs.get(np.float32, n)))
        for logits, (tok, probs) in zip(rows, got):
            want_tok, want_probs = eng.sample(logits, t, k, p, seed, counter, want_probs=True)
            assert tok == want_tok
            assert np.array_equal(probs.view(np.uint32), want_probs.view(np.uint32))
        hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)
        for d in (d_logits, d_tok, d_probs):
            d.free()
    hip.hipStreamDestroy(stream)
    print("capture ok", flush=True)


def test_sample_noalloc_under_graph_capture():
    """Captured into a HIP graph on a caller's stream -- as the first call of
    the process, so the scratch array's address is looked up under capture --
    and replayed with new logits: every replay gives rpg_hip_sample's token
    and probabilities bit for bit (full vocabulary without top-k, and top-k
    40). Runs in a child process so that the call really is the first."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ("import sys; sys.path.insert(0, %r); from tests.test_zz_no_alloc import _capture_main; _capture_main()"
            % root)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and "capture ok" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
