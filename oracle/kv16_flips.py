"""What an fp16 KV cache would change -- TEST INFRASTRUCTURE (a measurement).

The reference keeps K and V in fp32 (reference src/kv_cache.cc:25-26), and
so does the GPU engine. This script measures, on the CPU oracle (the
reference's token loop restated, pinned bit for bit to it), what rounding
every K / V value to fp16 on write (ties to even, oracle KvCache::fp16) does
to the full-size workloads whose reference runs tests/golden/config_*.npz
hold: the oracle runs the workload with the fp16 cache, teacher-forced on
the reference's ids (every step decides on the logits of the reference's
history), and reports per run

* the largest top-64 logit difference from the reference's step logits,
  relative to that step's max|logit| (the bar of the parity tests is 1e-3);
* the steps whose decision differs from the reference's id (greedy: the
  argmax; sampled: SampleToken with u = CounterUniform(seed, position)),
  with the reference's margin at each (how close its own decision was).

Run from the repository root after `make -C oracle port`:
    python oracle/kv16_flips.py s4_q4km s17_q4km [--threads N]
CPU time on 8 cores: ~2 minutes for s4_q4km, ~10 for s17_q4km.
"""

import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from rpgbarengine_amd import synth  # noqa: E402

GOLDEN = os.path.join(ROOT, "tests", "golden")
WORKLOADS = {"s17_q8_0": ("s17", "q8_0"), "s17_q4km": ("s17", "q4_k_m"), "s4_q4km": ("s4", "q4_k_m"),
             "s4_q4km_sessions": ("s4", "q4_k_m")}
CHUNK = 512  # prefill rows per forward call (bounds the logits buffer)


def decide(logits, temp, top_k, top_p, seed, pos):
    if temp > 0.0:
        return oracle.sample_token(logits, temp, top_k, top_p, oracle.counter_uniform(seed, pos))
    return int(np.argmax(logits))


def run(name, threads, fp16=True):
    preset, mix = WORKLOADS[name]
    g = np.load(os.path.join(GOLDEN, f"config_{name}.npz"))
    out = []
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, f"{name}.gguf")
        spec = synth.PRESETS[preset].with_(mix=synth.MIXES[mix], seed=int(g["gguf_seed"][0]))
        synth.write_gguf(path, spec, threads=threads)
        m = oracle.Model(path, threads=threads)
        runs = sorted({k.split("_")[0] for k in g.files if k.startswith("r")})
        for r in runs:
            pre = r + "_"
            pseed, plen, gen, temp, top_k, top_p, seed = g[pre + "params"]
            plen, gen, top_k, seed = int(plen), int(gen), int(top_k), int(seed)
            ids, want = g[pre + "ids"], g[pre + "gen"]
            tidx, tval, smax, marg = g[pre + "top_idx"], g[pre + "top_val"], g[pre + "step_max"], g[pre + "margin"]
            kv = m.kv(plen + gen, fp16=fp16)
            t0 = time.time()
            last = None
            for c0 in range(0, plen, CHUNK):
                last = m.forward(ids[c0:c0 + CHUNK], kv)[-1]
            worst, flips = 0.0, []
            logits = last
            for t in range(gen):
                err = float(np.max(np.abs(logits[tidx[t]].astype(np.float64) - tval[t]))) / float(smax[t])
                worst = max(worst, err)
                got = decide(logits, float(temp), top_k, float(top_p), seed, plen + t)
                if got != int(want[t]):
                    flips.append({"step": t, "id": got, "reference": int(want[t]), "margin": float(marg[t]),
                                  "err": err})
                if t + 1 < gen:
                    logits = m.forward(np.array([want[t]], dtype=np.int32), kv)[-1]
            res = {"workload": name, "run": r, "kv": "fp16" if fp16 else "fp32", "steps": gen,
                   "worst_top64_err_rel": worst, "flips": flips, "seconds": round(time.time() - t0, 1)}
            print(json.dumps(res), flush=True)
            out.append(res)
        m.close()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("names", nargs="+", choices=sorted(WORKLOADS))
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 8)
    ap.add_argument("--fp32", action="store_true", help="the fp32 cache instead (expect no difference at all)")
    a = ap.parse_args()
    for n in a.names:
        run(n, a.threads, fp16=not a.fp32)


if __name__ == "__main__":
    main()
