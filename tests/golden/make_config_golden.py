"""Writes tests/golden/config_<name>.npz: what the reference engine itself
(oracle/_ref/ref_golden, compiled from the reference sources by
oracle/Makefile) produces on the full-size synthetic workloads, so that the
GPU tests can check the HIP token loop at those sizes on a machine where the
reference is absent.

Workloads (synthetic GGUFs written by rpgbarengine_amd.synth, weights
N(0, 0.02) before quantising, GGUF seed 1):

* ``s17_q8_0``    Qwen3-1.7B shape, every matrix Q8_0: 32 random prompt ids,
                  greedy decode of 128 tokens.
* ``s17_q4km``    Qwen3-1.7B shape, Q4_K_M mix: 4000 random prompt ids, greedy
                  decode of 96 tokens (the cache ends exactly at 4096).
* ``s4_q4km``     Qwen3-4B shape, Q4_K_M mix: 512 random prompt ids, 256 tokens
                  sampled at T=0.8, top-k 40, top-p 0.95, seed 20261201 (the
                  benchmark's request).
* ``s4_q4km_sessions``  Qwen3-4B shape, Q4_K_M mix: 8 sessions, each a
                  1024-token random prefix and 128 tokens sampled at T=0.7,
                  top-p 0.95 (the chat ABI's defaults), seed 5000 + session;
                  each session run alone.

Per run the fixture holds: the prompt ids; the generated ids; the last prefill
row of logits quantised to int16 against its max|logit| (step 1/65534 of the
max, far inside the 1e-3 * max bar; first run of a config only); for every generated token the top-64
logits (index, value) and max|logit| of the logits that token was chosen from;
and the decision margin there -- greedy: top-1 minus top-2 logit; sampled:
distance of u = CounterUniform(seed, position) to the nearest edge of the
chosen token's interval of the cumulative filtered probabilities (reference
src/sampler.cc:96-112), computed by the oracle's FilterToProbs, which the
reference-written vectors in golden.npz pin bit for bit.

Run from the repository root after `make -C oracle ref port`:
    python tests/golden/make_config_golden.py [name ...]
CPU time on 8 cores: minutes for s17_q8_0 and s4_q4km, tens of minutes for
s17_q4km (single-threaded attention over 4000 positions) and the sessions.
"""

import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from rpgbarengine_amd import synth  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
TOP = 64

# name -> (preset, mix, [(prompt seed, prompt len, gen, T, top_k, top_p, seed)], full logits for sessions)
CONFIGS = {
    "s17_q8_0": ("s17", "q8_0", [(31, 32, 128, 0.0, 0, 1.0, 0)]),
    "s17_q4km": ("s17", "q4_k_m", [(33, 4000, 96, 0.0, 0, 1.0, 0)]),
    "s4_q4km": ("s4", "q4_k_m", [(42, 512, 256, 0.8, 40, 0.95, 20261201)]),
    "s4_q4km_sessions": ("s4", "q4_k_m", [(100 + s, 1024, 128, 0.7, 0, 0.95, 5000 + s) for s in range(8)]),
}
GGUF_SEED = 1


def spec_of(name):
    preset, mix, _ = CONFIGS[name]
    return synth.PRESETS[preset].with_(mix=synth.MIXES[mix], seed=GGUF_SEED)


def quantize_logits(x):
    m = float(np.max(np.abs(x)))
    q = np.round(x.astype(np.float64) / m * 32767.0).astype(np.int16)
    return q, np.float32(m)


def top_entries(x, k=TOP):
    idx = np.argpartition(-x, k)[:k]
    idx = idx[np.lexsort((idx, -x[idx]))]  # by value descending, ties by index
    return idx.astype(np.int32), x[idx].astype(np.float32)


def margin(decision, token, temperature, top_k, top_p, u):
    """Distance of the decision to its nearest flip (see module docstring)."""
    if not (temperature > 0.0):
        top2 = np.partition(decision, -2)[-2:]
        return float(top2[1] - top2[0])
    probs = oracle.filter_to_probs(decision, temperature, top_k, top_p)
    cum = np.cumsum(probs.astype(np.float64))
    lo = cum[token - 1] if token > 0 else 0.0
    return float(min(u - lo, cum[token] - u))


def run(name, d):
    preset, mix, runs = CONFIGS[name]
    spec = spec_of(name)
    path = os.path.join(d, f"{name}.gguf")
    t0 = time.time()
    synth.write_gguf(path, spec, threads=8)
    print(f"[{name}] GGUF {os.path.getsize(path) / 1e9:.2f} GB in {time.time() - t0:.0f}s", flush=True)
    g = {"gguf_seed": np.array([GGUF_SEED], np.int64)}
    for i, (pseed, plen, gen, temp, top_k, top_p, seed) in enumerate(runs):
        t0 = time.time()
        ids = synth.token_ids(pseed, plen, spec.vocab)
        r = oracle.ref_model(path, ids, gen=gen, temperature=temp, top_k=top_k, top_p=top_p, seed=seed,
                             threads=8, step_logits=True)
        last, steps, out = r["last_logits"], r["step_logits"], r["gen"]
        assert out.size == gen, (name, i, out.size)
        q, m = quantize_logits(last)
        pre = f"r{i}_"
        g[pre + "params"] = np.array([pseed, plen, gen, temp, top_k, top_p, seed], np.float64)
        g[pre + "ids"] = ids
        g[pre + "gen"] = out
        if i == 0:  # later sessions: their first step's top-64 covers the top of the row
            g[pre + "last_q"] = q
            g[pre + "last_max"] = np.array([m], np.float32)
        tidx = np.empty((gen, TOP), np.int32)
        tval = np.empty((gen, TOP), np.float32)
        smax = np.empty(gen, np.float32)
        marg = np.empty(gen, np.float64)
        for t in range(gen):
            decision = last if t == 0 else steps[t - 1]
            tidx[t], tval[t] = top_entries(decision)
            smax[t] = np.max(np.abs(decision))
            u = oracle.counter_uniform(seed, plen + t) if temp > 0 else 0.0
            marg[t] = margin(decision, int(out[t]), temp, top_k, top_p, u)
        g[pre + "top_idx"] = tidx
        g[pre + "top_val"] = tval
        g[pre + "step_max"] = smax
        g[pre + "margin"] = marg
        print(f"[{name}] run {i}: prompt {plen}, {gen} tokens in {time.time() - t0:.0f}s; "
              f"smallest margin {marg.min():.3g} at step {int(marg.argmin())}", flush=True)
    out_path = os.path.join(HERE, f"config_{name}.npz")
    np.savez_compressed(out_path, **g)
    print(f"[{name}] wrote {out_path} ({os.path.getsize(out_path)} bytes)", flush=True)


def main():
    if not oracle.ref_available():
        sys.exit("oracle/_ref/ref_golden is not built: run `make -C oracle ref` first")
    names = sys.argv[1:] or list(CONFIGS)
    for n in names:
        if n not in CONFIGS:
            sys.exit(f"unknown config {n}; known: {', '.join(CONFIGS)}")
    with tempfile.TemporaryDirectory() as d:
        for n in names:
            run(n, d)


if __name__ == "__main__":
    main()
