"""The drop-in boundary on the CPU: the engine library loads without a GPU,
exports exactly the C functions that include/*.h declares, the engine-ABI
calls that need no device behave like the reference's (reference
src/engine.cc:175-191: errors as -1 / NULL plus a thread-local message), and
the harness entry points keep their contracts."""

import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import oracle
import rpgbarengine_amd as eng
from rpgbarengine_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared(header):
    """Function names declared in a C header (return type, name, '(')."""
    text = open(os.path.join(INCLUDE, header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return set(re.findall(r"\b(rpg_[a-z0-9_]+)\s*\(", text))


def exported(lib_path):
    out = subprocess.run(["nm", "-D", "--defined-only", lib_path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_drop_in_library_exports_exactly_the_ten():
    """librpg_engine.so, the drop-in, exports the reference's ten functions
    and nothing else (reference include/rpg_engine.h:52-117; its Windows
    build exports these ten through a .def file)."""
    want = declared("rpg_engine.h")
    assert len(want) == 10
    assert exported(eng.LIB_PATH) == want
    out = subprocess.run(["nm", "-D", "--defined-only", eng.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    others = [ln for ln in out.splitlines() if ln.split()[-1] not in want and ln.split()[1] not in "AUw"]
    assert not others, others  # no data or weak symbols either
    lib = ctypes.CDLL(eng.LIB_PATH)
    for name in want:
        assert hasattr(lib, name)


def test_dev_library_exports_exactly_the_headers():
    """librpg_engine_dev.so (the same objects) adds the token-level and text
    entry points the tests and the benchmark call; internals stay hidden."""
    want = declared("rpg_engine.h") | declared("rpg_hip.h") | declared("rpg_text.h")
    got = exported(eng.DEV_LIB_PATH)
    assert want <= got, sorted(want - got)
    assert got <= want, sorted(got - want)
    lib = ctypes.CDLL(eng.DEV_LIB_PATH)
    for name in want:
        assert hasattr(lib, name)


def test_synth_library_exports_its_header():
    want = declared("rpg_synth.h")
    got = exported(synth.LIB_PATH)
    assert want <= got, sorted(want - got)


def test_abi_version_and_errors_without_device():
    lib = ctypes.CDLL(eng.LIB_PATH)
    lib.rpg_engine_version.restype = ctypes.c_char_p
    lib.rpg_engine_last_error.restype = ctypes.c_char_p
    lib.rpg_engine_load_model.argtypes = [ctypes.c_char_p, ctypes.c_char_p]
    lib.rpg_engine_load_model.restype = ctypes.c_int32
    lib.rpg_engine_generate.argtypes = [ctypes.c_int32, ctypes.c_char_p]
    lib.rpg_engine_generate.restype = ctypes.c_void_p
    lib.rpg_engine_session_reset.argtypes = [ctypes.c_int32]
    lib.rpg_engine_session_reset.restype = ctypes.c_int32
    lib.rpg_engine_unload_model.argtypes = [ctypes.c_int32]
    lib.rpg_engine_session_destroy.argtypes = [ctypes.c_int32]
    assert re.fullmatch(r"\d+\.\d+\.\d+", lib.rpg_engine_version().decode())
    assert lib.rpg_engine_load_model(b"/nonexistent/model.gguf", None) == -1
    assert lib.rpg_engine_last_error()
    assert lib.rpg_engine_generate(12345, b"{}") is None
    assert lib.rpg_engine_session_reset(12345) == -1
    lib.rpg_engine_unload_model(12345)     # invalid handles are no-ops
    lib.rpg_engine_session_destroy(12345)


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--no-cpu"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in (r.stdout + r.stderr)


def test_synth_gguf_is_deterministic_and_loads(tmp_path):
    spec = synth.PRESETS["tiny"].with_(mix=synth.MIXES["q4_k_m"], seed=11)
    a = synth.write_gguf(str(tmp_path / "a.gguf"), spec)
    b = synth.write_gguf(str(tmp_path / "b.gguf"), spec)
    assert open(a, "rb").read() == open(b, "rb").read()
    m = oracle.Model(a, threads=1)
    cfg = (m.n_layers, m.hidden, m.n_heads, m.n_kv_heads, m.head_dim, m.ffn, m.vocab)
    assert cfg == (2, 256, 4, 2, 128, 512, 1024)


# (max, rms) round-trip error in units of the weights' std for each type:
# 2-3 bit codes are coarse; a misplaced element or scale would give ~1.4.
ROUNDTRIP = {synth.F16: (0.002, 0.001), synth.BF16: (0.02, 0.005), synth.Q4_0: (0.3, 0.12),
             synth.Q4_1: (0.3, 0.12), synth.Q5_0: (0.2, 0.06), synth.Q5_1: (0.15, 0.05), synth.Q8_0: (0.03, 0.01),
             synth.Q8_1: (0.03, 0.01), synth.Q2_K: (1.2, 0.4), synth.Q3_K: (1.2, 0.25), synth.Q4_K: (0.3, 0.1),
             synth.Q5_K: (0.15, 0.05), synth.Q6_K: (0.1, 0.03), synth.Q8_K: (0.03, 0.01)}


@pytest.mark.parametrize("qtype", sorted(ROUNDTRIP))
def test_quantize_roundtrip_error(qtype):
    """Synthetic weights N(0, 0.02) quantise and dequantise (the oracle,
    pinned to the reference) to within the format's step."""
    x = synth.gaussian(1, qtype, 256 * 8, 0.02)
    raw = synth.quantize(qtype, x)
    y = oracle.dequant(qtype, raw.reshape(-1), x.size)
    mx, rms = ROUNDTRIP[qtype]
    assert np.max(np.abs(y - x)) <= mx * 0.02
    assert np.sqrt(np.mean((y - x) ** 2)) <= rms * 0.02
