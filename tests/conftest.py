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
        synth.write_gguf(path, spec)
        _made[key] = path
    return _made[key]


@pytest.fixture(scope="session")
def gguf_factory(gguf_dir):
    def f(preset, mix, seed=11, **over):
        return make_gguf(gguf_dir, preset, mix, seed, **over)
    return f


def rel_row_error(y, a, w):
    """max over rows of |y - a.w| / sum|a_i w_i| against float64 (reference
    tools/check_dotrow.py:83-91: normalise by sum |a_i * w_i|, not |a.w|)."""
    a64 = np.asarray(a, dtype=np.float64)
    w64 = np.asarray(w, dtype=np.float64)
    ref = a64 @ w64.T
    scale = np.maximum(np.abs(a64) @ np.abs(w64).T, 1e-30)
    return float(np.max(np.abs(np.asarray(y, dtype=np.float64) - ref) / scale))
