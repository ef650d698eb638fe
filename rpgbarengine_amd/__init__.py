"""MI355X-native Qwen3 token loop (HIP, gfx950) behind the RPGBarEngine C ABI.

The product is ``librpg_engine.so`` (built in-tree by ``make -C
rpgbarengine_amd``): hand-written HIP kernels and a C++ host runtime
exporting exactly the reference's 10-function chat ABI
(``include/rpg_engine.h``). ``librpg_engine_dev.so`` is the same code also
exporting the token-level entry points (``include/rpg_hip.h``) and the text
front-end (``include/rpg_text.h``). This module is a thin ctypes binding used
by the tests and ``bench.py`` -- ``abi()`` binds the drop-in, ``lib()`` the
development library; it never substitutes a CPU path -- every call fails
loudly when the library or the GPU is missing.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librpg_engine.so")  # the drop-in: the ten rpg_engine_* functions
DEV_LIB_PATH = os.path.join(HERE, "librpg_engine_dev.so")  # + rpg_hip_* and rpg_text_*

ENGINE_SYMBOLS = [
    "rpg_engine_version", "rpg_engine_last_error", "rpg_engine_load_model", "rpg_engine_unload_model",
    "rpg_engine_session_create", "rpg_engine_session_destroy", "rpg_engine_session_reset", "rpg_engine_generate",
    "rpg_engine_free", "rpg_engine_model_info",
]

_P = ctypes.c_void_p
_I32, _I64, _U32, _U64, _F = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float
_SIG = {
    "rpg_engine_version": ([], ctypes.c_char_p),
    "rpg_engine_last_error": ([], ctypes.c_char_p),
    "rpg_engine_load_model": ([ctypes.c_char_p, ctypes.c_char_p], _I32),
    "rpg_engine_unload_model": ([_I32], None),
    "rpg_engine_session_create": ([_I32, ctypes.c_char_p], _I32),
    "rpg_engine_session_destroy": ([_I32], None),
    "rpg_engine_session_reset": ([_I32], _I32),
    "rpg_engine_generate": ([_I32, ctypes.c_char_p], _P),
    "rpg_engine_free": ([_P], None),
    "rpg_engine_model_info": ([_I32], _P),
    "rpg_hip_last_error": ([], ctypes.c_char_p),
    "rpg_hip_device_count": ([], _I32),
    "rpg_hip_model_load": ([ctypes.c_char_p, _I32], _I32),
    "rpg_hip_model_free": ([_I32], None),
    "rpg_hip_model_config": ([_I32, _P], _I32),
    "rpg_hip_model_decode_bytes": ([_I32], _I64),
    "rpg_hip_model_rope_row": ([_I32, _I64, _P], _I32),
    "rpg_hip_session_new": ([_I32, _I64], _I32),
    "rpg_hip_session_free": ([_I32], None),
    "rpg_hip_session_len": ([_I32], _I64),
    "rpg_hip_session_set_len": ([_I32, _I64], _I32),
    "rpg_hip_prefill": ([_I32, _P, _I64, _P, _P], _I32),
    "rpg_hip_generate": ([_I32, _P, _I32, _F, _I32, _F, _U64, _P, _I32, _P, _P], _I32),
    "rpg_hip_kv_read": ([_I32, _I32, _I32, _I32, _I64, _P], _I32),
    "rpg_hip_session_decode_path": ([_I32], _I32),
    "rpg_hip_generate_batch": ([_P, _I32, _I32, _P, _P, _P, _P, _P, _P, _P], _I32),
    "rpg_hip_generate_forced": ([_I32, _P, _I32, _F, _I32, _F, _U64, _P, _P, _P], _I32),
    "rpg_hip_generate_batch_forced": ([_P, _I32, _I32, _P, _P, _P, _P, _P, _P, _P], _I32),
    "rpg_hip_fail_alloc_after": ([_I64], _I32),
    "rpg_hip_session_timing": ([_I32, _P, _P], _I32),
    "rpg_hip_session_bench_gate_up": ([_I32, _I32, _I32, _P], _I32),
    "rpg_hip_session_instep_gate_up": ([_I32, _I32, _P], _I32),
    "rpg_hip_bench_copy": ([_I64, _I32, _P], _I32),
    "rpg_hip_dequant": ([_U32, _P, _I64, _P], _I32),
    "rpg_hip_matmul": ([_U32, _P, _I64, _I64, _P, _I64, _P], _I32),
    "rpg_hip_matmul_swiglu": ([_U32, _P, _P, _I64, _I64, _P, _I64, _P], _I32),
    "rpg_hip_matvec_few": ([_U32, _P, _P, _I64, _I64, _P, _I64, _P, _F, _I32, _P], _I32),
    "rpg_hip_sample": ([_P, _I32, _F, _I32, _F, _U64, _I64, _P], _I32),
    "rpg_hip_sampler_fallbacks": ([], _I64),
    "rpg_hip_sampler_tie_orders": ([], _I64),
    "rpg_hip_sample_noalloc": ([_P, _I32, _F, _I32, _F, _U64, _I64, _P, _P, _P], _I32),
    "rpg_hip_attention": ([_P, _P, _P, _I32, _I32, _I32, _I32, _P], _I32),
    "rpg_hip_expf": ([_P, _I64, _P], _I32),
    "rpg_hip_bench_matmul": ([_U32, _P, _I64, _I64, _P, _I32, _I32, _I32, _P], _I32),
}

_lib = None
_abi = None


def _load(path: str, names) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with __graft_entry__.build()")
    L = ctypes.CDLL(path)
    for name in names:
        args, res = _SIG[name]
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    return L


def lib() -> ctypes.CDLL:
    """The development library (chat ABI + token-level + text entry points);
    raises when it is not built (no fallback exists)."""
    global _lib
    if _lib is None:
        _lib = _load(DEV_LIB_PATH, _SIG)
    return _lib


def abi() -> ctypes.CDLL:
    """The drop-in library, bound to its ten rpg_engine_* functions."""
    global _abi
    if _abi is None:
        _abi = _load(LIB_PATH, ENGINE_SYMBOLS)
    return _abi


class EngineError(RuntimeError):
    pass


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _ok(rc):
    if rc < 0:
        raise EngineError(lib().rpg_hip_last_error().decode())
    return rc


def device_count() -> int:
    return int(lib().rpg_hip_device_count())


def dequant(qtype: int, raw: np.ndarray, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    _ok(lib().rpg_hip_dequant(qtype, _p(raw), n, _p(out)))
    return out


def matmul(qtype: int, w: np.ndarray, rows: int, cols: int, X: np.ndarray) -> np.ndarray:
    """Y[t, r] = X[t] . W[r] with the fused dequant kernel."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    X = np.ascontiguousarray(X, dtype=np.float32).reshape(-1, cols)
    Y = np.empty((X.shape[0], rows), dtype=np.float32)
    _ok(lib().rpg_hip_matmul(qtype, _p(w), rows, cols, _p(X), X.shape[0], _p(Y)))
    return Y


def matvec_few(qtype: int, w: np.ndarray, rows: int, cols: int, X: np.ndarray, up: np.ndarray | None = None,
               norm_w: np.ndarray | None = None, eps: float = 1e-6, add_to: np.ndarray | None = None) -> np.ndarray:
    """The batched decode step's matvec for 1..8 tokens: Y = X . W^T, or
    silu(X . W^T) * (X . U^T) with `up`, of RMSNorm(X) * norm_w rows with
    `norm_w`, added to a copy of `add_to` when given."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    up = None if up is None else np.ascontiguousarray(up, dtype=np.uint8)
    X = np.ascontiguousarray(X, dtype=np.float32).reshape(-1, cols)
    nw = None if norm_w is None else np.ascontiguousarray(norm_w, dtype=np.float32)
    if add_to is None:
        Y = np.empty((X.shape[0], rows), dtype=np.float32)
    else:
        Y = np.array(add_to, dtype=np.float32, copy=True).reshape(X.shape[0], rows)
    _ok(lib().rpg_hip_matvec_few(qtype, _p(w), _p(up), rows, cols, _p(X), X.shape[0], _p(nw), eps,
                                 0 if add_to is None else 1, _p(Y)))
    return Y


def matmul_swiglu(qtype: int, gate: np.ndarray, up: np.ndarray, rows: int, cols: int, X: np.ndarray):
    """(Y, fused): Y[t, r] = silu(X[t] . G[r]) * (X[t] . U[r]); fused tells
    whether the single-launch GEMM ran."""
    gate = np.ascontiguousarray(gate, dtype=np.uint8)
    up = np.ascontiguousarray(up, dtype=np.uint8)
    X = np.ascontiguousarray(X, dtype=np.float32).reshape(-1, cols)
    Y = np.empty((X.shape[0], rows), dtype=np.float32)
    r = lib().rpg_hip_matmul_swiglu(qtype, _p(gate), _p(up), rows, cols, _p(X), X.shape[0], _p(Y))
    _ok(r)
    return Y, r == 1


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, pos0: int) -> np.ndarray:
    """Causal GQA attention of a segment: q [seq, n_heads, 128], k and v
    [n_kv, pos0 + seq, 128] (the cache), query t at position pos0 + t."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    seq, n_heads, hd = q.shape
    n_kv = k.shape[0]
    assert hd == 128 and k.shape == (n_kv, pos0 + seq, 128) and v.shape == k.shape
    out = np.empty_like(q)
    _ok(lib().rpg_hip_attention(_p(q), _p(k), _p(v), seq, n_heads, n_kv, pos0, _p(out)))
    return out


def sample(logits: np.ndarray, temperature: float, top_k: int, top_p: float, seed: int, counter: int,
           want_probs: bool = False):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    probs = np.empty_like(logits) if want_probs else None
    tok = _ok(lib().rpg_hip_sample(_p(logits), logits.size, temperature, top_k, top_p, seed, counter, _p(probs)))
    return (tok, probs) if want_probs else tok


def sampler_fallbacks() -> int:
    return int(lib().rpg_hip_sampler_fallbacks())


def sampler_tie_orders() -> int:
    """rpg_hip_sample draws whose top-p cut split equal probabilities."""
    return int(lib().rpg_hip_sampler_tie_orders())


def expf(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    _ok(lib().rpg_hip_expf(_p(x), x.size, _p(out)))
    return out


def bench_copy(nbytes: int, iters: int) -> float:
    """Mean microseconds of a plain device copy of nbytes (stream bandwidth)."""
    out = np.zeros(1, dtype=np.float64)
    _ok(lib().rpg_hip_bench_copy(nbytes, iters, _p(out)))
    return float(out[0])


def bench_matmul(qtype: int, w: np.ndarray, rows: int, cols: int, ns, copies: int, iters: int) -> np.ndarray:
    """Average milliseconds per launch of y = x . W^T for each token count in
    ns, over `copies` rotated device copies of W."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    n = np.ascontiguousarray(np.atleast_1d(ns), dtype=np.int32)
    out = np.zeros(n.size, dtype=np.float64)
    _ok(lib().rpg_hip_bench_matmul(qtype, _p(w), rows, cols, _p(n), n.size, copies, iters, _p(out)))
    return out


def generate_batch(sessions, max_tokens: int, temperature, top_k, top_p, seed, step_logits: bool = False):
    """max_tokens ids for each of several sessions of one model, decoded
    together (one weight read per step for all). Per-session parameters are
    sequences (or one value for all). Returns (ids [n, max_tokens], device
    milliseconds of the steps), and with step_logits the logits after every
    generated token, [n, max_tokens, vocab]."""
    n = len(sessions)

    def per(v, dt):
        a = np.asarray(v, dtype=dt)
        return np.ascontiguousarray(np.broadcast_to(a, (n,)) if a.ndim == 0 else a)

    h = np.array([s.h for s in sessions], dtype=np.int32)
    t, k, p, sd = per(temperature, np.float32), per(top_k, np.int32), per(top_p, np.float32), per(seed, np.uint64)
    out = np.empty((n, max_tokens), dtype=np.int32)
    ms = np.zeros(1, dtype=np.float64)
    steps = np.empty((n, max_tokens, sessions[0].model.vocab), dtype=np.float32) if step_logits else None
    _ok(lib().rpg_hip_generate_batch(_p(h), n, max_tokens, _p(t), _p(k), _p(p), _p(sd), _p(out), _p(steps),
                                     _p(ms)))
    return (out, float(ms[0]), steps) if step_logits else (out, float(ms[0]))


def generate_batch_forced(sessions, force_ids, temperature, top_k, top_p, seed):
    """Teacher-forced batched decode: session i forwards force_ids[i][t] at
    step t. Returns (drawn ids [n, steps], logits after every forced token
    [n, steps, vocab])."""
    n = len(sessions)
    force = np.ascontiguousarray(np.asarray(force_ids, dtype=np.int32).reshape(n, -1))
    steps = force.shape[1]

    def per(v, dt):
        a = np.asarray(v, dtype=dt)
        return np.ascontiguousarray(np.broadcast_to(a, (n,)) if a.ndim == 0 else a)

    h = np.array([s.h for s in sessions], dtype=np.int32)
    t, k, p, sd = per(temperature, np.float32), per(top_k, np.int32), per(top_p, np.float32), per(seed, np.uint64)
    drawn = np.empty((n, steps), dtype=np.int32)
    logits = np.empty((n, steps, sessions[0].model.vocab), dtype=np.float32)
    _ok(lib().rpg_hip_generate_batch_forced(_p(h), n, steps, _p(t), _p(k), _p(p), _p(sd), _p(force), _p(drawn),
                                            _p(logits)))
    return drawn, logits


def fail_alloc_after(n: int):
    """Test hook: the device allocation after n more successful ones fails
    as an out-of-memory hipMalloc would (n < 0: off)."""
    _ok(lib().rpg_hip_fail_alloc_after(n))


class Model:
    def __init__(self, path: str, max_pos: int = 4096):
        self.h = _ok(lib().rpg_hip_model_load(path.encode(), max_pos))
        cfg = np.zeros(9, dtype=np.int32)
        _ok(lib().rpg_hip_model_config(self.h, _p(cfg)))
        (self.n_layers, self.hidden, self.n_heads, self.n_kv_heads, self.head_dim, self.ffn, self.vocab,
         self.context_length, self.eos_id) = [int(v) for v in cfg]

    @property
    def decode_bytes(self) -> int:
        return int(_ok(lib().rpg_hip_model_decode_bytes(self.h)))

    def rope_row(self, pos: int) -> np.ndarray:
        out = np.empty(self.head_dim, dtype=np.float32)
        _ok(lib().rpg_hip_model_rope_row(self.h, pos, _p(out)))
        return out

    def session(self, max_seq: int) -> "Session":
        return Session(self, max_seq)

    def close(self):
        if getattr(self, "h", None):
            lib().rpg_hip_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Session:
    def __init__(self, model: Model, max_seq: int):
        self.model = model
        self.h = _ok(lib().rpg_hip_session_new(model.h, max_seq))

    @property
    def len(self) -> int:
        return int(_ok(lib().rpg_hip_session_len(self.h)))

    def set_len(self, n: int):
        _ok(lib().rpg_hip_session_set_len(self.h, n))

    def prefill(self, ids, all_logits: bool = False):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        last = np.empty(self.model.vocab, dtype=np.float32)
        allv = np.empty((ids.size, self.model.vocab), dtype=np.float32) if all_logits else None
        _ok(lib().rpg_hip_prefill(self.h, _p(ids), ids.size, _p(last), _p(allv)))
        return allv if all_logits else last

    def generate(self, max_tokens: int, temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0,
                 seed: int = 0, stop_ids=(), first_logits=None, step_logits: bool = False):
        stops = np.ascontiguousarray(np.array(stop_ids, dtype=np.int32))
        out = np.empty(max_tokens, dtype=np.int32)
        steps = np.empty((max_tokens, self.model.vocab), dtype=np.float32) if step_logits else None
        fl = None if first_logits is None else np.ascontiguousarray(first_logits, dtype=np.float32)
        n = _ok(lib().rpg_hip_generate(self.h, _p(fl), max_tokens, temperature, top_k, top_p, seed, _p(stops),
                                       stops.size, _p(out), _p(steps)))
        return (out[:n], steps[:n]) if step_logits else out[:n]

    def generate_forced(self, force_ids, temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0,
                        seed: int = 0, first_logits=None):
        """Teacher-forced decode: step i forwards force_ids[i] instead of the
        drawn id. Returns (drawn ids, logits after every forced token)."""
        force = np.ascontiguousarray(np.asarray(force_ids, dtype=np.int32))
        drawn = np.empty(force.size, dtype=np.int32)
        steps = np.empty((force.size, self.model.vocab), dtype=np.float32)
        fl = None if first_logits is None else np.ascontiguousarray(first_logits, dtype=np.float32)
        _ok(lib().rpg_hip_generate_forced(self.h, _p(fl), force.size, temperature, top_k, top_p, seed, _p(force),
                                          _p(drawn), _p(steps)))
        return drawn, steps

    @property
    def persistent_decode(self) -> bool:
        """True when a decode token runs as one persistent launch."""
        return _ok(lib().rpg_hip_session_decode_path(self.h)) == 1

    def kv(self, which: int, layer: int, head: int, n: int) -> np.ndarray:
        out = np.empty((n, self.model.head_dim), dtype=np.float32)
        _ok(lib().rpg_hip_kv_read(self.h, which, layer, head, n, _p(out)))
        return out

    def timing(self):
        a = np.zeros(1, dtype=np.float64)
        b = np.zeros(1, dtype=np.float64)
        _ok(lib().rpg_hip_session_timing(self.h, _p(a), _p(b)))
        return float(a[0]), float(b[0])

    def bench_gate_up(self, layer: int, iters: int):
        """(mean us per launch, algorithmic bytes per launch) of the decode
        gate+up matvec of `layer`, HIP events on the session stream."""
        out = np.zeros(2, dtype=np.float64)
        _ok(lib().rpg_hip_session_bench_gate_up(self.h, layer, iters, _p(out)))
        return float(out[0]), float(out[1])


    def instep_gate_up(self, tokens: int):
        """(mean us, algorithmic bytes) of the decode gate+up launch inside
        `tokens` greedy decode steps (HIP events around each launch); the
        session advances by `tokens`."""
        out = np.zeros(2, dtype=np.float64)
        _ok(lib().rpg_hip_session_instep_gate_up(self.h, tokens, _p(out)))
        return float(out[0]), float(out[1])
    def close(self):
        if getattr(self, "h", None):
            lib().rpg_hip_session_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
