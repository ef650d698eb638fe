import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from rpgbarengine_amd import synth  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running parity case")


@pytest.fixture(scope="session")
def gguf_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("gguf")


_made = {}


def make_gguf(gguf_dir, preset: str, mix: str, seed: int = 11, **over) -> str:
    """Write (once per test session) a synthetic GGUF of a preset shape."""
    key = (preset, mix, seed, tuple(sorted(over.items())))
    if key not in _made:
        spec = synth.PRESETS[preset].with_(mix=synth.MIXES[mix], seed=seed, **over)
        name = f"{preset}_{mix}_{seed}_{abs(hash(key)) % 10**8}.gguf"
        path = os.path.join(str(gguf_dir), name)
        synth.write_gguf(path, spec, threads=min(16, os.cpu_count() or 1))
        _made[key] = path
    return _made[key]


@pytest.fixture(scope="session")
def gguf_factory(gguf_dir):
    def f(preset, mix, seed=11, **over):
        return make_gguf(gguf_dir, preset, mix, seed, **over)
    return f


def _f16(b) -> float:
    return float(np.ascontiguousarray(b).view(np.float16)[0])


def split_terms(qtype: int, raw_row: np.ndarray, k: int):
    """(A, B) per weight of one row, where the block format defines w = A - B
    (reference src/quant.cc:159-237): Q4_K A = d*sc*q, B = dmin*m; Q6_K
    A = d*sc*q (q unsigned, 0..63), B = 32*d*sc; Q8_0 A = d*q, B = 0. Parsed
    from the raw bytes in float64."""
    A = np.zeros(k, dtype=np.float64)
    B = np.zeros(k, dtype=np.float64)
    if qtype == synth.Q8_0:
        blk = raw_row.reshape(-1, 34)
        for b in range(blk.shape[0]):
            A[32 * b:32 * b + 32] = _f16(blk[b, 0:2]) * blk[b, 2:].view(np.int8).astype(np.float64)
        return A, B
    if qtype == synth.Q4_K:
        blk = raw_row.reshape(-1, 144)
        for b in range(blk.shape[0]):
            d, dmin = _f16(blk[b, 0:2]), _f16(blk[b, 2:4])
            s = blk[b, 4:16].astype(np.int64)
            qs = blk[b, 16:144].astype(np.int64)
            for j in range(8):
                if j < 4:
                    sc, m = s[j] & 63, s[j + 4] & 63
                else:
                    sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4)
                    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
                q = (qs[32 * (j // 2):32 * (j // 2) + 32] >> (4 * (j % 2))) & 0xF
                A[256 * b + 32 * j:256 * b + 32 * j + 32] = d * sc * q
                B[256 * b + 32 * j:256 * b + 32 * j + 32] = dmin * m
        return A, B
    blk = raw_row.reshape(-1, 210)
    l = np.arange(32)
    for b in range(blk.shape[0]):
        ql, qh = blk[b, 0:128].astype(np.int64), blk[b, 128:192].astype(np.int64)
        sc = blk[b, 192:208].view(np.int8).astype(np.float64)
        d = _f16(blk[b, 208:210])
        for h in range(2):
            for m in range(4):
                q = ((ql[64 * h + l + 32 * (m & 1)] >> (4 * (m >> 1))) & 0xF) | (((qh[32 * h + l] >> (2 * m)) & 3) << 4)
                s = sc[8 * h + 2 * m + l // 16]
                A[256 * b + 128 * h + 32 * m + l] = d * s * q
                B[256 * b + 128 * h + 32 * m + l] = 32.0 * d * s
    return A, B


def rel_row_error(y, a, w):
    """max over rows of |y - a.w| / sum|a_i w_i| against float64 (reference
    tools/check_dotrow.py:83-91: normalise by sum |a_i * w_i|, not |a.w|)."""
    a64 = np.asarray(a, dtype=np.float64)
    w64 = np.asarray(w, dtype=np.float64)
    ref = a64 @ w64.T
    scale = np.maximum(np.abs(a64) @ np.abs(w64).T, 1e-30)
    return float(np.max(np.abs(np.asarray(y, dtype=np.float64) - ref) / scale))
