#!/usr/bin/env python3
"""Benchmark of the Qwen3 token loop on one MI355X.

Workload (the 4B-shape configuration the headline metric is quoted on):
Qwen3-4B-shape synthetic GGUF, Q4_K_M mix (36 layers, hidden 2560, 32 Q / 8 KV
heads, head_dim 128, FFN 9728, vocab 151936, tied embeddings, weights
N(0, 0.02)), prefill a 512-token random prompt, then decode 256 tokens sampled
at temperature 0.8, top-k 40, top-p 0.95 from a fixed seed. One "step" is one
such request (prefill 512 + decode 256) on a reset session.

Prints one JSON line: value = decode tok/s; prefill tok/s, the HBM roofline of
the dominant decode launch and of the whole decode step, the fused matmul
microbench (Q8_0 / Q4_K / Q6_K at the 1.7B shapes, M = 1, 4, 16, 64), the
batched-sessions, long-context and 1.7B Q8_0 decode legs and the reference
CPU path timed on this host's cores ride along.
Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 MFMA

PROMPT = 512
DECODE = 256
TEMP, TOP_K, TOP_P, SEED = 0.8, 40, 0.95, 20261201
CPU_THREADS_CAP = 16         # the host cores one GPU's job may use
PROBE_ITERS = 72             # gate+up launches of the roofline probe (two passes over the layers)
INSTEP_TOKENS = 8            # decode steps of the in-step gate+up measurement (x 36 launches)
COPY_BYTES = 256 << 20       # plain copy that calibrates the byte counters
# fused matmul microbench: (in, out) shapes of the 1.7B model, token counts
MB_SHAPES = [(2048, 6144), (6144, 2048), (2048, 4096), (2048, 1024), (2048, 151936)]
MB_TOKENS = [1, 4, 16, 64]
MB_ROTATE_BYTES = 320 << 20  # weight copies per shape: past the 256 MB memory-side cache
MB_ITERS = 40
# batched sessions: 8 sessions of a 1024-token prefix, 128 tokens each at
# T=0.7, top-p 0.95, seeds 5000 + i, decoded together
BATCH_SESSIONS, BATCH_PREFIX, BATCH_DECODE, BATCH_TEMP, BATCH_TOP_P = 8, 1024, 128, 0.7, 0.95
# long context: the 1.7B shape, Q4_K_M, a 4000-token prompt, 96 greedy tokens
# over the fp32 cache (positions 4000 .. 4095)
LONG_PROMPT, LONG_DECODE = 4000, 96
# the 1.7B shape with every matrix Q8_0: a 32-token prompt, 128 greedy tokens
Q8_PROMPT, Q8_DECODE = 32, 128


def kv16_bytes_per_pos(spec) -> int:
    """K and V of one position in every layer at 2 bytes per value: the KV
    term of the decode step's algorithmic bytes (the cache is held in fp32;
    the roofline counts the bytes an fp16 cache would read)."""
    return 2 * spec.n_layers * spec.n_kv_heads * spec.head_dim * 2


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def model_flops_per_token(spec) -> float:
    """2 * parameters of the matrices a token passes through (body only)."""
    H, F, L = spec.hidden, spec.ffn, spec.n_layers
    qd, kvd = spec.n_heads * spec.head_dim, spec.n_kv_heads * spec.head_dim
    per_layer = H * qd + 2 * H * kvd + qd * H + 3 * H * F
    return 2.0 * per_layer * L


def prefill_flops(spec, n: int) -> float:
    body = model_flops_per_token(spec) * n
    # causal attention: QK^T and PV over t+1 positions for every query
    attn = 4.0 * spec.n_heads * spec.head_dim * spec.n_layers * (n * (n + 1) / 2)
    lm_head = 2.0 * spec.vocab * spec.hidden  # last row only
    return body + attn + lm_head


def physical_cores() -> int:
    """Distinct (package, core) pairs of /proc/cpuinfo: the count the
    reference's DefaultThreads() picks on Linux (reference
    src/threads.cc:60-100,118-123); 0 when unknown."""
    seen, phys = set(), None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                key, _, val = line.partition(":")
                key = key.strip()
                if key == "physical id":
                    phys = val.strip()
                elif key == "core id":
                    seen.add((phys, val.strip()))
    except OSError:
        return 0
    return len(seen)


def cpu_baseline(path: str, ids_path: str, threads: int) -> dict:
    """The whole workload (prefill 512 + decode 256 sampled, same GGUF, prompt
    and options) on the reference compiled from its own sources, or on the
    oracle's restatement where that build is absent."""
    import oracle
    sample = (f"the full workload: prefill {PROMPT} + decode {DECODE} sampled tokens of the same GGUF and prompt "
              f"(T={TEMP}, top-k {TOP_K}, top-p {TOP_P}, seed {SEED})")
    if oracle.ref_available():
        out = subprocess.run(
            [oracle.REF_GOLDEN, "model", path, "--ids", ids_path, "--n", str(PROMPT), "--gen", str(DECODE),
             "--temp", str(TEMP), "--top-k", str(TOP_K), "--top-p", str(TOP_P), "--seed", str(SEED),
             "--threads", str(threads), "--time"], capture_output=True, text=True, check=True).stdout
        t = json.loads(out.strip().splitlines()[-1])
        kind = "reference"
    else:
        m = oracle.Model(path, threads=threads)
        ids = np.fromfile(ids_path, dtype=np.int32)[:PROMPT]
        m.forward(ids[:1])  # page-in
        t = m.time_run(ids, DECODE, TEMP, TOP_K, TOP_P, SEED)
        t["threads"] = threads
        kind = "port"
    default = physical_cores()
    return {
        "value": round(DECODE / (t["decode_ms"] / 1e3), 3),
        "unit": "decode tok/s",
        "prefill_tok_s": round(PROMPT / (t["prefill_ms"] / 1e3), 3),
        "cores": int(t["threads"]),
        "kind": kind,
        "sample": sample,
        "default_threads": default,
        "threads_note": (f"DefaultThreads() detects {default} physical cores here; the run uses "
                         f"{int(t['threads'])}, the cores one GPU's job may use on this host"
                         if default > int(t["threads"]) else "DefaultThreads() core count"),
    }


def batched_sessions(eng, synth, model, spec) -> dict:
    """Aggregate decode rate of 8 sessions stepped together on one weight set
    (each weight matrix read once per step for all of them)."""
    sess = []
    for i in range(BATCH_SESSIONS):
        s = model.session(BATCH_PREFIX + BATCH_DECODE)
        s.prefill(synth.token_ids(100 + i, BATCH_PREFIX, spec.vocab))
        sess.append(s)
    seeds = [5000 + i for i in range(BATCH_SESSIONS)]
    # warm (graph capture), then time a fresh decode of every session
    eng.generate_batch(sess, 2, BATCH_TEMP, 0, BATCH_TOP_P, seeds)
    for s in sess:
        s.set_len(BATCH_PREFIX)
    _, ms = eng.generate_batch(sess, BATCH_DECODE, BATCH_TEMP, 0, BATCH_TOP_P, seeds)
    for s in sess:
        s.close()
    steps_per_s = BATCH_DECODE / (ms / 1e3)
    mean_pos = BATCH_PREFIX + (BATCH_DECODE - 1) / 2.0
    step_bytes = model.decode_bytes + BATCH_SESSIONS * kv16_bytes_per_pos(spec) * mean_pos
    achieved = step_bytes * steps_per_s / 1e9
    return {
        "value": round(BATCH_SESSIONS * steps_per_s, 2),
        "unit": "tok/s (all sessions)",
        "sessions": BATCH_SESSIONS,
        "ms_per_step": round(ms / BATCH_DECODE, 4),
        "workload": f"{BATCH_SESSIONS} sessions x ({BATCH_PREFIX}-token prefix + {BATCH_DECODE} sampled tokens, "
                    f"T={BATCH_TEMP}, top-p {BATCH_TOP_P}), one decode step for all",
        "roofline": {"bound": "hbm", "unit": "GB/s", "bytes_per_step": int(step_bytes), "achieved": round(achieved, 2),
                     "peak": HBM_PEAK_GBS, "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "counted": "weights once + 8 sessions' fp16-equivalent K/V at the mean position"},
    }


def long_context(eng, synth, workdir: str) -> dict:
    """Decode over a deep cache: the 1.7B-shape Q4_K_M model, prefill a
    4000-token random prompt, then 96 greedy tokens (every step reads the
    whole K/V history of all 28 layers from the fp32 cache)."""
    spec = synth.PRESETS["s17"].with_(mix=synth.MIX_Q4_K_M, seed=3)
    path = os.path.join(workdir, "qwen3-1.7b-shape-q4_k_m.gguf")
    synth.write_gguf(path, spec, threads=16)
    ids = synth.token_ids(43, LONG_PROMPT, spec.vocab)
    model = eng.Model(path, max_pos=LONG_PROMPT + LONG_DECODE)
    sess = model.session(LONG_PROMPT + LONG_DECODE)
    runs = []
    for _ in range(2):  # the first run captures the decode graph
        sess.set_len(0)
        sess.prefill(ids)
        pf = sess.timing()[0]
        out = sess.generate(LONG_DECODE)
        assert out.size == LONG_DECODE
        runs.append((pf, sess.timing()[1]))
    pf_ms, dec_ms = runs[-1]
    decode_bytes = model.decode_bytes
    sess.close()
    model.close()
    os.remove(path)
    tps = LONG_DECODE / (dec_ms / 1e3)
    mean_pos = LONG_PROMPT + (LONG_DECODE - 1) / 2.0
    kv32 = 2 * kv16_bytes_per_pos(spec) * mean_pos  # the fp32 cache's reads per token
    step32 = decode_bytes + kv32
    step16 = decode_bytes + kv32 / 2
    return {
        "value": round(tps, 2),
        "unit": "decode tok/s",
        "prefill_tok_s": round(LONG_PROMPT / (pf_ms / 1e3), 2),
        "prefill_ms": round(pf_ms, 3),
        "workload": f"qwen3-1.7b-shape Q4_K_M synthetic GGUF: prefill {LONG_PROMPT} random ids, decode "
                    f"{LONG_DECODE} greedy (positions {LONG_PROMPT}..{LONG_PROMPT + LONG_DECODE - 1}), batch 1",
        "kv_bytes_per_token": int(kv32),
        "weight_bytes_per_token": int(decode_bytes),
        "roofline": {"bound": "hbm", "unit": "GB/s", "bytes_per_token": int(step32),
                     "achieved": round(step32 * tps / 1e9, 2), "peak": HBM_PEAK_GBS,
                     "frac": round(step32 * tps / 1e9 / HBM_PEAK_GBS, 4),
                     "frac_fp16_kv": round(step16 * tps / 1e9 / HBM_PEAK_GBS, 4),
                     "counted": "weights incl. lm_head + the fp32 K/V history at the mean position "
                                "(frac_fp16_kv: the same rate over the bytes an fp16 cache would read)"},
    }


def q8_0_decode(eng, synth, workdir: str) -> dict:
    """The 1.7B-shape model with every matrix (and the tied embedding) in
    Q8_0: prefill 32 random ids, then 128 greedy tokens; the roofline counts
    every weight once per token plus the fp16-equivalent K/V at the mean
    position."""
    spec = synth.PRESETS["s17"].with_(mix=synth.MIX_Q8_0, seed=2)
    path = os.path.join(workdir, "qwen3-1.7b-shape-q8_0.gguf")
    synth.write_gguf(path, spec, threads=16)
    ids = synth.token_ids(7, Q8_PROMPT, spec.vocab)
    model = eng.Model(path, max_pos=Q8_PROMPT + Q8_DECODE)
    sess = model.session(Q8_PROMPT + Q8_DECODE)
    runs = []
    for _ in range(3):  # the first run captures the decode graph
        sess.set_len(0)
        sess.prefill(ids)
        out = sess.generate(Q8_DECODE)
        assert out.size == Q8_DECODE
        runs.append(sess.timing()[1])
    decode_bytes = model.decode_bytes
    sess.close()
    model.close()
    os.remove(path)
    dec_ms = float(np.mean(runs[1:]))
    tps = Q8_DECODE / (dec_ms / 1e3)
    step = decode_bytes + kv16_bytes_per_pos(spec) * (Q8_PROMPT + (Q8_DECODE - 1) / 2.0)
    return {
        "value": round(tps, 2),
        "unit": "decode tok/s",
        "workload": f"qwen3-1.7b-shape Q8_0 synthetic GGUF: prefill {Q8_PROMPT} random ids, decode {Q8_DECODE} "
                    "greedy, batch 1",
        "roofline": {"bound": "hbm", "unit": "GB/s", "bytes_per_token": int(step),
                     "achieved": round(step * tps / 1e9, 2), "peak": HBM_PEAK_GBS,
                     "frac": round(step * tps / 1e9 / HBM_PEAK_GBS, 4),
                     "counted": "weights incl. lm_head, norms, embedding row + fp16-equivalent K/V at the mean "
                                "position"},
    }


def matmul_microbench(eng, synth) -> dict:
    """GB/s (and TFLOP/s) of the fused dequant matmul per type, shape and
    token count, weights N(0, 0.02) quantized, rotated over enough device
    copies (>= 320 MB) that every launch streams its weights from HBM."""
    res = {}
    names = {synth.Q8_0: "q8_0", synth.Q4_K: "q4_k", synth.Q6_K: "q6_k"}
    for k, rows in MB_SHAPES:
        w32 = synth.gaussian(21, k * 7 + rows, rows * k, 0.02).reshape(rows, k)
        for qt, name in names.items():
            raw = synth.quantize(qt, w32)
            copies = max(1, -(-MB_ROTATE_BYTES // raw.nbytes))
            ms = eng.bench_matmul(qt, raw, rows, k, MB_TOKENS, copies, MB_ITERS)
            for m, t in zip(MB_TOKENS, ms):
                moved = raw.nbytes + 4 * m * (k + rows)
                res[f"{name} {k}->{rows} m{m}"] = {
                    "us": round(float(t) * 1e3, 3),
                    "gbs": round(moved / (float(t) * 1e-3) / 1e9, 1),
                    "tflops": round(2.0 * m * k * rows / (float(t) * 1e-3) / 1e12, 3),
                }
            del raw
        del w32
        log(f"microbench {k}->{rows} done")
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--cpu-threads", type=int, default=CPU_THREADS_CAP)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-microbench", action="store_true", help="skip the fused matmul microbench")
    ap.add_argument("--no-batched", action="store_true", help="skip the batched-sessions leg")
    ap.add_argument("--no-long", action="store_true", help="skip the long-context leg")
    ap.add_argument("--no-q8", action="store_true", help="skip the 1.7B Q8_0 decode leg")
    ap.add_argument("--prefill-only", action="store_true",
                    help="counter runs: the 512-token prefill three times, nothing else on the GPU")
    ap.add_argument("--batched-only", action="store_true",
                    help="trace runs: the batched-sessions leg alone, its result as one JSON line")
    ap.add_argument("--q8-only", action="store_true",
                    help="trace runs: the 1.7B Q8_0 decode leg alone, its result as one JSON line")
    ap.add_argument("--long-only", action="store_true",
                    help="trace runs: the long-context leg alone, its result as one JSON line")
    ap.add_argument("--workdir", default=None)
    ap.add_argument("--kernel-only", action="store_true",
                    help="counter runs: the 512-token prefill, 8 sampled decode steps after it (positions "
                         "512-519), PROBE_ITERS gate+up launches and one plain device copy of COPY_BYTES (the "
                         "scale of the byte counters), nothing timed")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: runs on one GPU only (--gpus {args.gpus} requested); "
              "sessions would shard one per GPU with no communication", file=sys.stderr)
        return 2

    import rpgbarengine_amd as eng
    from rpgbarengine_amd import synth

    if eng.device_count() < 1:
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    if args.q8_only or args.long_only:
        with tempfile.TemporaryDirectory(dir=args.workdir) as d:
            print(json.dumps(q8_0_decode(eng, synth, d) if args.q8_only else long_context(eng, synth, d)), flush=True)
        return 0
    spec = synth.PRESETS["s4"].with_(mix=synth.MIX_Q4_K_M, seed=1)
    work = tempfile.TemporaryDirectory(dir=args.workdir)
    path = os.path.join(work.name, "qwen3-4b-shape-q4_k_m.gguf")
    t0 = time.time()
    synth.write_gguf(path, spec, threads=16)
    log(f"synthetic GGUF {os.path.getsize(path) / 1e9:.2f} GB in {time.time() - t0:.1f}s")
    ids = synth.token_ids(42, PROMPT, spec.vocab)
    ids_path = os.path.join(work.name, "prompt.bin")
    ids.tofile(ids_path)

    model = eng.Model(path, max_pos=4096)
    sess = model.session(PROMPT + DECODE + 8)
    log(f"model loaded, decode weight bytes/token {model.decode_bytes / 1e9:.4f} GB")

    def one_step():
        sess.set_len(0)
        sess.prefill(ids)
        pf = sess.timing()[0]
        out = sess.generate(DECODE, TEMP, TOP_K, TOP_P, SEED)
        assert out.size == DECODE
        return pf, sess.timing()[1], out

    if args.batched_only:
        print(json.dumps(batched_sessions(eng, synth, model, spec)), flush=True)
        return 0

    if args.prefill_only:
        times = []
        for _ in range(3):
            sess.set_len(0)
            sess.prefill(ids)
            times.append(sess.timing()[0])
        print(json.dumps({"prefill_ms": times, "tokens": PROMPT}), flush=True)
        return 0

    if args.kernel_only:
        sess.prefill(ids)
        sess.generate(8, TEMP, TOP_K, TOP_P, SEED)
        us, nbytes = sess.bench_gate_up(0, PROBE_ITERS)
        copy_us = eng.bench_copy(COPY_BYTES, 4)  # CopyKernel: reads and writes COPY_BYTES per launch
        print(json.dumps({"gate_up_us": us, "gate_up_bytes": nbytes, "copy_bytes": COPY_BYTES,
                          "copy_us": copy_us}), flush=True)
        return 0

    for i in range(args.warmup):
        one_step()
        log(f"warmup step {i + 1}/{args.warmup} done")
    pf_ms, dec_ms, walls = [], [], []
    first_ids = None
    for i in range(args.steps):
        t = time.perf_counter()
        pf, dc, out = one_step()
        walls.append((time.perf_counter() - t) * 1e3)
        pf_ms.append(pf)
        dec_ms.append(dc)
        if first_ids is None:
            first_ids = out
        elif not np.array_equal(first_ids, out):
            raise RuntimeError("decode is not deterministic across steps")
        log(f"step {i + 1}/{args.steps}: prefill {pf:.2f} ms, decode {dc:.2f} ms")

    decode_ms = float(np.mean(dec_ms))
    prefill_ms = float(np.mean(pf_ms))
    decode_tps = DECODE / (decode_ms / 1e3)
    prefill_tps = PROMPT / (prefill_ms / 1e3)
    # decode step: every weight once + the K/V history (fp16-equivalent) at
    # the mean position of the decode window
    mean_pos = PROMPT + (DECODE - 1) / 2.0
    bytes_per_token = model.decode_bytes + kv16_bytes_per_pos(spec) * mean_pos
    step_achieved = bytes_per_token * decode_tps / 1e9
    # the dominant kernel: the decode gate+up matvec (2 x 9728 x 2560 Q4_K),
    # timed with HIP events on the session stream where the decode step runs
    # it (INSTEP_TOKENS greedy steps after the timed prompt; each interval
    # includes the launch's dispatch after the previous kernel) ...
    sess.set_len(0)
    sess.prefill(ids)
    gu_us, gu_bytes = sess.instep_gate_up(INSTEP_TOKENS)
    gu_achieved = gu_bytes / (gu_us * 1e-6) / 1e9
    log(f"gate+up in step: {gu_us:.2f} us per launch, {gu_bytes / 1e6:.2f} MB, {gu_achieved:.1f} GB/s")
    # ... and back to back, layers rotating (no dispatch gap between launches)
    pr_us, _ = sess.bench_gate_up(0, PROBE_ITERS)
    pr_achieved = gu_bytes / (pr_us * 1e-6) / 1e9
    log(f"gate+up probe: {pr_us:.2f} us per launch, {pr_achieved:.1f} GB/s")
    stream_gbs = 2.0 * (1 << 30) / (eng.bench_copy(1 << 30, 8) * 1e-6) / 1e9  # read + write of 1 GiB
    log(f"measured copy bandwidth {stream_gbs:.1f} GB/s")
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "decode_gate_up_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    pflops = prefill_flops(spec, PROMPT)
    result = {
        "metric": "decode tok/s + %HBM roofline, prefill tok/s; Qwen3-4B Q4_K_M, 1 GPU",
        "value": round(decode_tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(float(np.mean(walls)), 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "qwen3-4b-shape Q4_K_M synthetic GGUF: prefill 512 random ids, decode 256 sampled "
                        "(T=0.8, top-k 40, top-p 0.95, fixed seed), batch 1",
            "model": "qwen3-4b-shape (36 layers, hidden 2560, 32/8 heads, head_dim 128, ffn 9728, vocab 151936)",
            "global_batch": 1,
            "seq_len": PROMPT + DECODE,
            "parallelism": "none",
        },
        "prefill_tok_s": round(prefill_tps, 2),
        "prefill_ms": round(prefill_ms, 3),
        "decode_ms_per_token": round(decode_ms / DECODE, 5),
        "prefill_mfma_frac": round(pflops / (prefill_ms / 1e3) / (BF16_PEAK_TFLOPS * 1e12), 5),
        "roofline": {
            "bound": "hbm",
            "kernel": "MatvecMfmaKernel<5, 4> decode gate+up SwiGLU matvec (int8 MFMA, tile-major Q4_K pair), "
                      "2 x 9728 x 2560",
            "achieved": round(gu_achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gu_achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": int(gu_bytes),
            "avg_launch_us": round(gu_us, 3),
            "timed": f"in step: {INSTEP_TOKENS} decode steps x {spec.n_layers} layers, HIP events around each "
                     "launch on the session stream (interval includes its dispatch)",
            "probe": {"avg_launch_us": round(pr_us, 3), "achieved": round(pr_achieved, 2),
                      "frac": round(pr_achieved / HBM_PEAK_GBS, 4),
                      "timed": f"{PROBE_ITERS} back-to-back launches, layers rotating"},
            "measured_copy_gbs": round(stream_gbs, 1),
        },
        "decode_step_roofline": {
            "bound": "hbm",
            "unit": "GB/s",
            "bytes_per_token": int(bytes_per_token),
            "achieved": round(step_achieved, 2),
            "peak": HBM_PEAK_GBS,
            "frac": round(step_achieved / HBM_PEAK_GBS, 4),
            "counted": "weights incl. lm_head, norms, embedding row + fp16-equivalent K/V at the mean position",
        },
    }
    if not args.no_batched:
        result["batched_sessions"] = batched_sessions(eng, synth, model, spec)
        log(f"batched sessions: {result['batched_sessions']['value']} tok/s aggregate")
    if not args.no_long:
        result["long_context"] = long_context(eng, synth, work.name)
        log(f"long context: {result['long_context']['value']} decode tok/s at positions {LONG_PROMPT}+")
    if not args.no_q8:
        result["q8_0_decode"] = q8_0_decode(eng, synth, work.name)
        log(f"1.7B Q8_0 decode: {result['q8_0_decode']['value']} tok/s")
    if not args.no_microbench:
        result["matmul_microbench"] = matmul_microbench(eng, synth)
    if not args.no_cpu:
        try:
            result["cpu_baseline"] = cpu_baseline(path, ids_path, args.cpu_threads)
        except Exception as e:  # reported, never substituted for the GPU figure
            result["cpu_baseline"] = {"value": None, "error": str(e)}
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    sess.close()
    model.close()
    work.cleanup()
    return 0


if __name__ == "__main__":
    sys.exit(main())
