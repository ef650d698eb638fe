"""Writes tests/golden/info.npz: what the reference's rpg_engine_model_info
returned (reference src/engine.cc:519-547) for synthetic models and load
configurations, through its own C ABI (oracle/_ref/ref_engine, compiled from
the reference sources by oracle/Makefile). The GGUF path inside each answer
is replaced by the placeholder @PATH@; the test puts its own path back.

Cases: (preset, mix, GGUF seed, tokenizer, config_json, session count); one
session is created by the driver, so every answer reports one session.

Run from the repository root after `make -C oracle ref`:
    python tests/golden/make_info_golden.py
"""

import json
import os
import struct
import subprocess
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from rpgbarengine_amd import synth  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "info.npz")
REF_ENGINE = os.path.join(ROOT, "oracle", "_ref", "ref_engine")

CASES = [
    ("tiny", "q8_0", 11, 1, ""),
    ("tiny", "q4_k_m", 5, 0, '{"max_seq": 256}'),
    ("tiny", "q8_0", 11, 1, '{"max_pos": 100000, "max_seq": 77}'),
    ("tiny", "other", 3, 0, '{"max_pos": 128}'),
]


def pack(records):
    out = bytearray()
    for r in records:
        r = r.encode() if isinstance(r, str) else bytes(r)
        out += struct.pack("<I", len(r)) + r
    return bytes(out)


def unpack(b):
    out, i = [], 0
    while i + 4 <= len(b):
        (n,) = struct.unpack_from("<I", b, i)
        out.append(b[i + 4:i + 4 + n])
        i += 4 + n
    return out


def main():
    if not os.path.exists(REF_ENGINE):
        sys.exit("oracle/_ref/ref_engine is not built: run `make -C oracle ref` first")
    g = {}
    with tempfile.TemporaryDirectory() as d:
        for i, (preset, mix, seed, tok, cfg) in enumerate(CASES):
            spec = synth.PRESETS[preset].with_(mix=synth.MIXES[mix], seed=seed, tokenizer=tok)
            path = synth.write_gguf(os.path.join(d, f"m{i}.gguf"), spec)
            script = os.path.join(d, "script.bin")
            out = os.path.join(d, "out.bin")
            with open(script, "wb") as f:
                f.write(pack([path, cfg, "", "!info"]))
            subprocess.run([REF_ENGINE, script, out], check=True)
            (info,) = unpack(open(out, "rb").read())
            text = info.decode()
            quoted = json.dumps(path)
            assert quoted in text, text
            g[f"case{i}"] = np.array([json.dumps([preset, mix, seed, tok, cfg])])
            g[f"info{i}"] = np.array([text.replace(quoted, '"@PATH@"')])
    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
