"""CPU oracle for the Qwen3 token loop -- TEST INFRASTRUCTURE, NOT PRODUCT.

Two checkers live here:

* ``liboracle.so`` (built from ``oracle/cpu_ref/*.cc`` by ``make -C oracle
  port``): this repository's restatement of the reference's scalar + AVX2 CPU
  path, function by function, with the same floating-point operation order.
* ``_ref/ref_golden`` (built by ``make -C oracle ref`` from the reference's own
  sources, when they are present): the reference engine itself, driven through
  its internal API. Its binaries travel with the tree; its sources never do.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only to check or time the
engine against it -- the
HIP engine never routes through it.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")
REF_GOLDEN = os.path.join(HERE, "_ref", "ref_golden")

_lib = None

_P = ctypes.c_void_p
_sig = {
    "orc_last_error": ([], ctypes.c_char_p),
    "orc_dequant": ([ctypes.c_uint32, _P, ctypes.c_int64, _P], ctypes.c_int32),
    "orc_scale_min_k4": ([ctypes.c_int32, _P, _P, _P], ctypes.c_int32),
    "orc_half_to_float": ([ctypes.c_uint16], ctypes.c_float),
    "orc_dot_rows": ([ctypes.c_int32, ctypes.c_uint32, _P, _P, ctypes.c_int64, ctypes.c_int64, _P], ctypes.c_int32),
    "orc_avx2_available": ([], ctypes.c_int32),
    "orc_matmul_batch": ([ctypes.c_uint32, _P, ctypes.c_int64, ctypes.c_int64, _P, ctypes.c_int64, _P,
                          ctypes.c_int32], ctypes.c_int32),
    "orc_rmsnorm": ([_P, _P, ctypes.c_int64, ctypes.c_float, _P], None),
    "orc_softmax": ([_P, ctypes.c_int64], None),
    "orc_silu": ([_P, ctypes.c_int64], None),
    "orc_rope": ([_P, ctypes.c_int32, ctypes.c_int32, _P, _P], None),
    "orc_argmax": ([_P, ctypes.c_int64], ctypes.c_int32),
    "orc_dot": ([_P, _P, ctypes.c_int64], ctypes.c_float),
    "orc_expf": ([ctypes.c_float], ctypes.c_float),
    "orc_expf_n": ([_P, ctypes.c_int64, _P], None),
    "orc_attention": ([_P, _P, _P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                       _P], ctypes.c_int32),
    "orc_splitmix64": ([ctypes.c_uint64], ctypes.c_uint64),
    "orc_counter_uniform": ([ctypes.c_uint64, ctypes.c_uint64], ctypes.c_float),
    "orc_filter_to_probs": ([_P, ctypes.c_int64, ctypes.c_float, ctypes.c_int32, ctypes.c_float, _P],
                            ctypes.c_int32),
    "orc_sample_token": ([_P, ctypes.c_int64, ctypes.c_float, ctypes.c_int32, ctypes.c_float, ctypes.c_float],
                         ctypes.c_int32),
    "orc_model_load": ([ctypes.c_char_p, ctypes.c_int32, ctypes.c_int32], _P),
    "orc_model_free": ([_P], None),
    "orc_model_config": ([_P, _P], None),
    "orc_rope_row": ([_P, ctypes.c_int64, _P], ctypes.c_int32),
    "orc_kv_new": ([_P, ctypes.c_int64], _P),
    "orc_kv_free": ([_P], None),
    "orc_kv_set_fp16": ([_P, ctypes.c_int32], None),
    "orc_round_half_n": ([_P, ctypes.c_int64, _P], None),
    "orc_kv_len": ([_P], ctypes.c_int64),
    "orc_kv_read": ([_P, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int64, _P], ctypes.c_int32),
    "orc_forward": ([_P, _P, ctypes.c_int64, _P, _P], ctypes.c_int32),
    "orc_generate": ([_P, _P, _P, ctypes.c_int32, ctypes.c_float, ctypes.c_int32, ctypes.c_float, ctypes.c_uint64,
                      _P, ctypes.c_int32, _P, _P], ctypes.c_int32),
    "orc_time_run": ([_P, _P, ctypes.c_int64, ctypes.c_int32, ctypes.c_float, ctypes.c_int32, ctypes.c_float,
                      ctypes.c_uint64, _P], ctypes.c_int32),
}


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle port`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in _sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _check(rc):
    if rc < 0:
        raise RuntimeError(lib().orc_last_error().decode())
    return rc


def dequant(qtype: int, raw: np.ndarray, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, dtype=np.float32)
    _check(lib().orc_dequant(qtype, _p(raw), n, _p(out)))
    return out


def dot_rows(qtype: int, a: np.ndarray, w: np.ndarray, k: int, which: int = 0) -> np.ndarray:
    """which: 0 dispatched (AVX2 when present), 1 scalar reference, 2 AVX2."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    rows = w.size // ((k // _blk(qtype)[0]) * _blk(qtype)[1])
    out = np.empty(rows, dtype=np.float32)
    _check(lib().orc_dot_rows(which, qtype, _p(a), _p(w), k, rows, _p(out)))
    return out


# (elements, bytes) per block of every ggml type (reference src/quant.cc:29-45)
_BLOCKS = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34),
           9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
           15: (256, 292)}


def _blk(qtype):
    return _BLOCKS[qtype]


def matmul_batch(qtype: int, w: np.ndarray, rows: int, cols: int, X: np.ndarray, threads: int = 4) -> np.ndarray:
    X = np.ascontiguousarray(X, dtype=np.float32)
    n = X.shape[0]
    w = np.ascontiguousarray(w, dtype=np.uint8)
    out = np.zeros((n, rows), dtype=np.float32)
    _check(lib().orc_matmul_batch(qtype, _p(w), rows, cols, _p(X), n, _p(out), threads))
    return out


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, pos0: int) -> np.ndarray:
    """The reference's causal GQA attention (src/qwen3.cc:79-117) of a
    segment q [seq, n_heads, hd] over a cache k, v [n_kv, pos0 + seq, hd]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    seq, n_heads, hd = q.shape
    out = np.empty_like(q)
    _check(lib().orc_attention(_p(q), _p(k), _p(v), seq, n_heads, k.shape[0], hd, pos0, _p(out)))
    return out


def round_half(x: np.ndarray) -> np.ndarray:
    """Each value rounded to the nearest fp16 (ties to even), as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_round_half_n(_p(x), x.size, _p(out))
    return out


def filter_to_probs(logits: np.ndarray, temperature: float, top_k: int, top_p: float) -> np.ndarray:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    out = np.empty_like(logits)
    _check(lib().orc_filter_to_probs(_p(logits), logits.size, temperature, top_k, top_p, _p(out)))
    return out


def sample_token(logits: np.ndarray, temperature: float, top_k: int, top_p: float, u: float) -> int:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    return int(_check(lib().orc_sample_token(_p(logits), logits.size, temperature, top_k, top_p, u)))


def expf(x: np.ndarray) -> np.ndarray:
    """The host's glibc expf (the reference's std::exp on floats), elementwise."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_expf_n(_p(x), x.size, _p(out))
    return out


def counter_uniform(seed: int, counter: int) -> float:
    return float(lib().orc_counter_uniform(seed, counter))


class Model:
    """Loaded GGUF on the CPU oracle."""

    def __init__(self, path: str, threads: int = 0, max_pos: int = 4096):
        self.h = lib().orc_model_load(path.encode(), threads, max_pos)
        if not self.h:
            raise RuntimeError(lib().orc_last_error().decode())
        cfg = np.zeros(9, dtype=np.int32)
        lib().orc_model_config(self.h, _p(cfg))
        (self.n_layers, self.hidden, self.n_heads, self.n_kv_heads, self.head_dim, self.ffn, self.vocab,
         self.context_length, self.eos_id) = [int(v) for v in cfg]

    def close(self):
        if self.h:
            lib().orc_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def kv(self, max_seq: int, fp16: bool = False) -> "KvCache":
        return KvCache(self, max_seq, fp16)

    def forward(self, ids, kv: "KvCache | None" = None) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty((ids.size, self.vocab), dtype=np.float32)
        _check(lib().orc_forward(self.h, _p(ids), ids.size, kv.h if kv else None, _p(out)))
        return out

    def generate(self, kv: "KvCache", first_logits: np.ndarray, max_tokens: int, temperature: float = 0.0,
                 top_k: int = 0, top_p: float = 1.0, seed: int = 0, stop_ids=(), step_logits: bool = False):
        first = np.ascontiguousarray(first_logits, dtype=np.float32)
        stops = np.ascontiguousarray(np.array(stop_ids, dtype=np.int32))
        out = np.empty(max_tokens, dtype=np.int32)
        steps = np.empty((max_tokens, self.vocab), dtype=np.float32) if step_logits else None
        n = _check(lib().orc_generate(self.h, kv.h, _p(first), max_tokens, temperature, top_k, top_p, seed,
                                      _p(stops), stops.size, _p(out), _p(steps) if steps is not None else None))
        if step_logits:
            return out[:n], steps[:n]
        return out[:n]

    def time_run(self, ids, gen: int, temperature=0.0, top_k=0, top_p=1.0, seed=0):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.zeros(3, dtype=np.float64)
        _check(lib().orc_time_run(self.h, _p(ids), ids.size, gen, temperature, top_k, top_p, seed, _p(out)))
        return {"prefill_ms": out[0], "decode_ms": out[1], "threads": int(out[2])}


class KvCache:
    def __init__(self, model: Model, max_seq: int, fp16: bool = False):
        self.model = model
        self.h = lib().orc_kv_new(model.h, max_seq)
        if not self.h:
            raise RuntimeError(lib().orc_last_error().decode())
        # measurement only (the reference keeps fp32): K / V rounded to fp16
        lib().orc_kv_set_fp16(self.h, 1 if fp16 else 0)

    @property
    def len(self) -> int:
        return int(lib().orc_kv_len(self.h))

    def read(self, which: int, layer: int, head: int, n: int) -> np.ndarray:
        out = np.empty((n, self.model.head_dim), dtype=np.float32)
        _check(lib().orc_kv_read(self.h, which, layer, head, n, _p(out)))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            lib().orc_kv_free(self.h)
            self.h = None


# ---------------------------------------------------------------- reference build

def ref_available() -> bool:
    return os.path.exists(REF_GOLDEN)


def ref_run(*args: str, capture: bool = True) -> str:
    """Run oracle/_ref/ref_golden (the reference engine) with the arguments."""
    if not ref_available():
        raise RuntimeError("oracle/_ref/ref_golden is not built")
    r = subprocess.run([REF_GOLDEN, *map(str, args)], capture_output=capture, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"ref_golden {args[0]} failed: {r.stderr}")
    return r.stdout


def ref_model(gguf: str, ids, gen: int = 0, temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0,
              seed: int = 0, threads: int = 4, nocache: bool = False, step_logits: bool = False,
              all_logits: bool = False):
    """Reference prefill (+ generate). Returns a dict of numpy arrays."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    with tempfile.TemporaryDirectory() as d:
        ip = os.path.join(d, "ids.bin")
        ids.tofile(ip)
        args = ["model", gguf, "--ids", ip, "--threads", threads, "--last-logits-out", os.path.join(d, "last.bin")]
        if all_logits:
            args += ["--logits-out", os.path.join(d, "all.bin")]
        if nocache:
            args += ["--nocache-logits-out", os.path.join(d, "nocache.bin")]
        if gen:
            args += ["--gen", gen, "--temp", temperature, "--top-k", top_k, "--top-p", top_p, "--seed", seed,
                     "--gen-out", os.path.join(d, "gen.bin")]
            if step_logits:
                args += ["--step-logits-out", os.path.join(d, "steps.bin")]
        ref_run(*args)
        res = {"last_logits": np.fromfile(os.path.join(d, "last.bin"), dtype=np.float32)}
        if all_logits:
            res["logits"] = np.fromfile(os.path.join(d, "all.bin"), dtype=np.float32).reshape(ids.size, -1)
        if nocache:
            res["nocache_logits"] = np.fromfile(os.path.join(d, "nocache.bin"), dtype=np.float32).reshape(ids.size, -1)
        if gen:
            res["gen"] = np.fromfile(os.path.join(d, "gen.bin"), dtype=np.int32)
            if step_logits:
                res["step_logits"] = np.fromfile(os.path.join(d, "steps.bin"), dtype=np.float32).reshape(
                    res["gen"].size, -1)
        return res
