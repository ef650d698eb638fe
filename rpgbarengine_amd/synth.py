"""ctypes binding of librpg_synth.so: synthetic qwen3 GGUF files and block
quantizers (declared in include/rpg_synth.h). CPU only.

Presets name the model shapes the parity tests and the benchmark use:

* ``s17`` -- Qwen3-1.7B shape: 28 layers, hidden 2048, 16 Q / 8 KV heads,
  head_dim 128, FFN 6144, vocab 151936, tied embeddings.
* ``s4``  -- Qwen3-4B shape: 36 layers, hidden 2560, 32 Q / 8 KV heads,
  head_dim 128, FFN 9728, vocab 151936, tied embeddings.
* ``tiny`` / ``small`` / ``mid`` -- reduced shapes with the same structure for
  fast CPU-oracle comparisons.
"""

from __future__ import annotations

import ctypes
import dataclasses
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "librpg_synth.so")

F32, F16, Q8_0, Q4_K, Q6_K = 0, 1, 8, 12, 14
Q4_0, Q4_1, Q5_0, Q5_1, Q8_1, Q2_K, Q3_K, Q5_K, Q8_K, BF16 = 2, 3, 6, 7, 9, 10, 11, 13, 15, 30
MIX_Q8_0, MIX_Q4_K_M, MIX_F32, MIX_Q4_K, MIX_Q6_K, MIX_OTHER = 0, 1, 2, 3, 4, 5
MIXES = {"q8_0": MIX_Q8_0, "q4_k_m": MIX_Q4_K_M, "f32": MIX_F32, "q4_k": MIX_Q4_K, "q6_k": MIX_Q6_K,
         "other": MIX_OTHER}

BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q4_0: (32, 18), Q4_1: (32, 20), Q5_0: (32, 22), Q5_1: (32, 24),
         Q8_0: (32, 34), Q8_1: (32, 36), Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176),
         Q6_K: (256, 210), Q8_K: (256, 292)}
# every type the reference dequantises (reference src/quant.cc:29-45)
ALL_TYPES = [F32, F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K]
TYPE_NAMES = {F32: "f32", F16: "f16", BF16: "bf16", Q4_0: "q4_0", Q4_1: "q4_1", Q5_0: "q5_0", Q5_1: "q5_1",
              Q8_0: "q8_0", Q8_1: "q8_1", Q2_K: "q2_k", Q3_K: "q3_k", Q4_K: "q4_k", Q5_K: "q5_k", Q6_K: "q6_k",
              Q8_K: "q8_k"}


class _Spec(ctypes.Structure):
    _fields_ = [
        ("n_layers", ctypes.c_int32), ("hidden", ctypes.c_int32), ("n_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("ffn", ctypes.c_int32),
        ("vocab", ctypes.c_int32), ("context_length", ctypes.c_int32), ("rope_theta", ctypes.c_float),
        ("rms_eps", ctypes.c_float), ("mix", ctypes.c_int32), ("seed", ctypes.c_uint64),
        ("weight_std", ctypes.c_float), ("norm_std", ctypes.c_float), ("tokenizer", ctypes.c_int32),
    ]


@dataclasses.dataclass
class ModelSpec:
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    mix: int = MIX_Q8_0
    seed: int = 1
    context_length: int = 4096
    rope_theta: float = 1e6
    rms_eps: float = 1e-6
    weight_std: float = 0.02
    norm_std: float = 0.01
    tokenizer: int = 0  # 1: byte-level BPE vocabulary (include/rpg_synth.h)

    def with_(self, **kw) -> "ModelSpec":
        return dataclasses.replace(self, **kw)


PRESETS = {
    "s17": ModelSpec(28, 2048, 16, 8, 128, 6144, 151936),
    "s4": ModelSpec(36, 2560, 32, 8, 128, 9728, 151936),
    "tiny": ModelSpec(2, 256, 4, 2, 128, 512, 1024),
    "small": ModelSpec(3, 512, 8, 2, 128, 1536, 4096),
    "mid": ModelSpec(4, 1024, 8, 4, 128, 3072, 32000),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        L = ctypes.CDLL(LIB_PATH)
        L.rpg_synth_write_gguf.argtypes = [ctypes.c_char_p, ctypes.POINTER(_Spec), ctypes.c_int32]
        L.rpg_synth_write_gguf.restype = ctypes.c_int32
        L.rpg_synth_quantize.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        L.rpg_synth_quantize.restype = ctypes.c_int64
        L.rpg_synth_row_bytes.argtypes = [ctypes.c_uint32, ctypes.c_int64]
        L.rpg_synth_row_bytes.restype = ctypes.c_int64
        L.rpg_synth_gaussian.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int64, ctypes.c_float,
                                         ctypes.c_void_p]
        L.rpg_synth_token_ids.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]
        L.rpg_synth_last_error.restype = ctypes.c_char_p
        _lib = L
    return _lib


def write_gguf(path: str, spec: ModelSpec, threads: int = 0) -> str:
    s = _Spec(spec.n_layers, spec.hidden, spec.n_heads, spec.n_kv_heads, spec.head_dim, spec.ffn, spec.vocab,
              spec.context_length, spec.rope_theta, spec.rms_eps, spec.mix, spec.seed, spec.weight_std,
              spec.norm_std, spec.tokenizer)
    if lib().rpg_synth_write_gguf(path.encode(), ctypes.byref(s), threads) != 0:
        raise RuntimeError(lib().rpg_synth_last_error().decode())
    return path


def row_bytes(qtype: int, n: int) -> int:
    return int(lib().rpg_synth_row_bytes(qtype, n))


def quantize(qtype: int, x: np.ndarray) -> np.ndarray:
    """Quantise a float32 array (last dim a block multiple) row by row."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    rb = row_bytes(qtype, n)
    if rb < 0:
        raise ValueError(f"{n} is not a block multiple for type {qtype}")
    rows = x.reshape(-1, n)
    out = np.empty((rows.shape[0], rb), dtype=np.uint8)
    for r in range(rows.shape[0]):
        lib().rpg_synth_quantize(qtype, rows[r].ctypes.data, n, out[r].ctypes.data)
    return out.reshape(x.shape[:-1] + (rb,))


def gaussian(seed: int, stream: int, n: int, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().rpg_synth_gaussian(seed, stream, n, std, out.ctypes.data)
    return out


def token_ids(seed: int, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().rpg_synth_token_ids(seed, n, vocab, out.ctypes.data)
    return out


def random_blocks(qtype: int, n_blocks: int, seed: int) -> np.ndarray:
    """Structurally valid blocks with random payload bytes and finite scales
    (the construction of reference tools/selftest.cc:667-707: random bytes,
    scale fields written explicitly so no fp16 NaN/Inf appears)."""
    be, bb = BLOCK[qtype]
    rng = np.random.default_rng(seed)
    raw = rng.integers(0, 256, size=(n_blocks, bb), dtype=np.uint8)
    def half(v):  # [n] float -> [n, 2] little-endian fp16 bytes
        return np.ascontiguousarray(v.astype(np.float16)).view(np.uint8).reshape(-1, 2)
    scales = rng.uniform(0.25, 2.0, size=(n_blocks, 2)).astype(np.float32)
    if qtype in (Q8_0, Q4_0, Q5_0):
        raw[:, 0:2] = half(scales[:, 0] * 0.01)
    elif qtype in (Q4_1, Q5_1, Q8_1):
        raw[:, 0:2] = half(scales[:, 0] * 0.01)
        raw[:, 2:4] = half((scales[:, 1] - 1.0) * 0.05)
    elif qtype in (Q4_K, Q5_K):
        raw[:, 0:2] = half(scales[:, 0] * 0.001)
        raw[:, 2:4] = half(scales[:, 1] * 0.001)
    elif qtype == Q6_K:
        raw[:, 208:210] = half(scales[:, 0] * 0.001)
    elif qtype == Q2_K:
        raw[:, 80:82] = half(scales[:, 0] * 0.001)
        raw[:, 82:84] = half(scales[:, 1] * 0.001)
    elif qtype == Q3_K:
        raw[:, 108:110] = half(scales[:, 0] * 0.001)
    elif qtype == Q8_K:
        raw[:, 0:4] = np.ascontiguousarray(scales[:, 0] * 0.001).view(np.uint8).reshape(-1, 4)
    elif qtype == F16:
        raw[:] = half(rng.normal(0.0, 1.0, size=n_blocks).astype(np.float32)).reshape(n_blocks, 2)
    elif qtype == BF16:
        v = rng.normal(0.0, 1.0, size=n_blocks).astype(np.float32).view(np.uint32)
        raw[:] = (v >> 16).astype(np.uint16).view(np.uint8).reshape(n_blocks, 2)
    elif qtype == F32:
        raw[:] = rng.normal(0.0, 1.0, size=n_blocks).astype(np.float32).view(np.uint8).reshape(n_blocks, 4)
    return raw
