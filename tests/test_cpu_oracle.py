"""The CPU oracle pinned against the reference: the golden vectors that the
reference engine wrote (tests/golden/golden.npz, tests/golden/make_golden.py),
the reference's own known-answer tests (reference tools/selftest.cc) and
closed forms that a plausible slip would violate. CPU only."""

import math
import os

import numpy as np
import pytest

import oracle
from rpgbarengine_amd import synth

GOLDEN = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz"))
QTYPES = [synth.Q8_0, synth.Q4_K, synth.Q6_K]
# every type the reference dequantises but F32 (a plain copy)
DEQ_TYPES = [t for t in synth.ALL_TYPES if t != synth.F32]


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------- dequant


@pytest.mark.parametrize("qtype", DEQ_TYPES)
def test_dequant_matches_reference_golden(qtype):
    raw = GOLDEN[f"dequant_{qtype}_raw"]
    want = GOLDEN[f"dequant_{qtype}_out"]
    got = oracle.dequant(qtype, raw, want.size)
    assert np.array_equal(bits(got), bits(want))


def test_q3_k_scale_unpack_per_byte():
    """Q3_K's 12 packed bytes -> 16 six-bit scales, checked against the
    reference's kmask word operations (reference src/quant.cc:231-238) done
    here on 32-bit words: every byte value at every packed position."""
    km1, km2 = 0x03030303, 0x0F0F0F0F
    for pos in range(12):
        for v in (0x00, 0x01, 0x0F, 0x10, 0x3F, 0x40, 0x80, 0xC3, 0xFF):
            packed = np.zeros(12, np.uint8)
            packed[pos] = v
            a0, a1, tmp = [int(x) for x in packed.view("<u4")]
            words = [(a0 & km2) | (((tmp >> 0) & km1) << 4), (a1 & km2) | (((tmp >> 2) & km1) << 4),
                     ((a0 >> 4) & km2) | (((tmp >> 4) & km1) << 4), ((a1 >> 4) & km2) | (((tmp >> 6) & km1) << 4)]
            want = np.array(words, "<u4").view(np.uint8).astype(np.int32)
            # a block whose codes are all 2 with every high bit set: y = d*(s-32)*2
            blk = np.zeros(110, np.uint8)
            blk[0:32] = 0xFF
            blk[32:96] = 0xAA
            blk[96:108] = packed
            blk[108:110] = np.array([1.0], np.float16).view(np.uint8)
            y = oracle.dequant(synth.Q3_K, blk, 256).reshape(16, 16)
            sub = [8 * h + 2 * j + k for h in range(2) for j in range(4) for k in range(2)]
            for e, s_idx in enumerate(sub):
                assert np.all(y[e] == np.float32(2 * (want[s_idx] - 32))), (pos, v, s_idx)


def test_q8_0_kat():
    """d = 1.0, q = -16..15 decodes to -16..15 (reference tools/selftest.cc:432-447)."""
    blk = np.zeros(34, dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), dtype=np.uint8)
    blk[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    assert np.array_equal(oracle.dequant(synth.Q8_0, blk, 32), np.arange(32, dtype=np.float32) - 16)


def _scale_min_k4_spec(j, q):
    """The 6-bit scale/min layout of the GGUF K-quants, written from the
    format: j < 4 -> low 6 bits of bytes j and j+4; j >= 4 -> low/high nibble
    of byte j+4 plus the top 2 bits of bytes j-4 and j."""
    if j < 4:
        return q[j] & 63, q[j + 4] & 63
    return (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4), (q[j + 4] >> 4) | ((q[j] >> 6) << 4)


def test_scale_min_k4_exhaustive_per_byte():
    """Every sub-block j depends on at most 3 bytes; sweep each byte through all
    256 values with the others random, against the format definition."""
    rng = np.random.default_rng(5)
    lib = oracle.lib()
    for j in range(8):
        for pos in range(12):
            for v in range(256):
                q = rng.integers(0, 256, 12, dtype=np.uint8)
                q[pos] = v
                sc = np.zeros(1, np.uint8)
                mn = np.zeros(1, np.uint8)
                lib.orc_scale_min_k4(j, q.ctypes.data, sc.ctypes.data, mn.ctypes.data)
                assert (int(sc[0]), int(mn[0])) == _scale_min_k4_spec(j, [int(b) for b in q])


def test_q4_k_closed_form():
    """Q4_K with all scales 1, mins 0, d = 1: element 64g + l (l < 32) is the
    low nibble of byte 32g + l, element 64g + 32 + l the high nibble."""
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = np.frombuffer(np.float16(1.0).tobytes(), dtype=np.uint8)
    blk[4:8] = 1    # sc[0..3] = 1, top bits 0
    blk[8:12] = 0   # m[0..3] = 0
    blk[12:16] = 1  # sc[4..7] = 1 (low nibble), m[4..7] = 0
    q = (np.arange(128) * 37 % 256).astype(np.uint8)
    blk[16:] = q
    got = oracle.dequant(synth.Q4_K, blk, 256)
    want = np.zeros(256, np.float32)
    for g in range(4):
        for l in range(32):
            want[64 * g + l] = q[32 * g + l] & 0xF
            want[64 * g + 32 + l] = q[32 * g + l] >> 4
    assert np.array_equal(got, want)


def test_q6_k_closed_form():
    """Q6_K with scales 1 and d = 1: element 128h + l + 32m = q - 32 where the
    low 4 bits come from ql[64h + l (+32 for m odd)] (low nibble for m < 2)
    and the top 2 bits from bits 2m of qh[32h + l]."""
    rng = np.random.default_rng(3)
    blk = np.zeros(210, dtype=np.uint8)
    blk[:192] = rng.integers(0, 256, 192, dtype=np.uint8)
    blk[192:208] = 1
    blk[208:210] = np.frombuffer(np.float16(1.0).tobytes(), dtype=np.uint8)
    got = oracle.dequant(synth.Q6_K, blk, 256)
    ql, qh = blk[:128].astype(int), blk[128:192].astype(int)
    want = np.zeros(256, np.float32)
    for h in range(2):
        for l in range(32):
            for m in range(4):
                lo = ql[64 * h + l + (32 if m & 1 else 0)]
                lo = (lo & 0xF) if m < 2 else (lo >> 4)
                hi = (qh[32 * h + l] >> (2 * m)) & 3
                want[128 * h + l + 32 * m] = (lo | (hi << 4)) - 32
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- dot rows


@pytest.mark.parametrize("qtype", DEQ_TYPES)
def test_dot_rows_match_reference_golden(qtype):
    """DotRowQuantRef (scalar) and DotRowQuant (the build's fused kernel)
    bit for bit (reference src/matmul.cc:73-108)."""
    w, a = GOLDEN[f"dot_{qtype}_w"], GOLDEN[f"dot_{qtype}_a"]
    k = a.size
    ref = oracle.dot_rows(qtype, a, w, k, which=1)
    fused = oracle.dot_rows(qtype, a, w, k, which=0)
    assert np.array_equal(bits(ref), bits(GOLDEN[f"dot_{qtype}_ref"]))
    if oracle.lib().orc_avx2_available():
        assert np.array_equal(bits(fused), bits(GOLDEN[f"dot_{qtype}_fused"]))


@pytest.mark.parametrize("qtype", DEQ_TYPES)
def test_dot_rows_within_row_bound(qtype):
    """Both dots within max|d|/sum|a*w| <= 1e-6 of float64 over the dequantised
    weights (reference tools/check_dotrow.py:40-41)."""
    w, a = GOLDEN[f"dot_{qtype}_w"], GOLDEN[f"dot_{qtype}_a"]
    k = a.size
    rows = GOLDEN[f"dot_{qtype}_ref"].size
    wdq = oracle.dequant(qtype, w, rows * k).reshape(rows, k).astype(np.float64)
    exact = wdq @ a.astype(np.float64)
    scale = np.abs(wdq) @ np.abs(a.astype(np.float64))
    for which in (0, 1):
        got = oracle.dot_rows(qtype, a, w, k, which=which).astype(np.float64)
        assert np.max(np.abs(got - exact) / scale) <= 1e-6


@pytest.mark.parametrize("qtype", QTYPES)
def test_split_terms_reassemble_dequant(qtype):
    """The (A, B) split the GPU outlier bound is built on: A - B equals the
    reference dequantisation (two float32 roundings apart at most), and B
    vanishes only where the format has no second term."""
    from tests.conftest import split_terms
    k = 512
    raw = synth.random_blocks(qtype, k // synth.BLOCK[qtype][0], seed=5).reshape(-1)
    A, B = split_terms(qtype, raw, k)
    w = oracle.dequant(qtype, raw, k).astype(np.float64)
    assert np.all(np.abs((A - B) - w) <= 2.0 ** -22 * (np.abs(A) + np.abs(B)) + 1e-45)
    assert (np.count_nonzero(B) == 0) == (qtype == synth.Q8_0)


# ---------------------------------------------------------------- sampler


def splitmix64(x):
    m = (1 << 64) - 1
    x = (x + 0x9E3779B97F4A7C15) & m
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & m
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & m
    return x ^ (x >> 31)


def test_counter_uniform_golden_and_closed_form():
    seed = int(GOLDEN["uniform_seed"][0])
    want = GOLDEN["uniform_u"]
    for c in range(want.size):
        u = oracle.counter_uniform(seed, c)
        assert np.float32(u).view(np.uint32) == want[c].view(np.uint32)
        bits24 = splitmix64((seed + 0x9E3779B97F4A7C15 * c) & ((1 << 64) - 1)) >> 40
        assert u == np.float32(bits24) * np.float32(1.0 / 16777216.0)


@pytest.mark.parametrize("case", range(7))
def test_filter_and_sample_match_reference_golden(case):
    n, seed, t, k, p, u = GOLDEN["sample_cases"][case]
    logits = GOLDEN[f"sample_{case}_logits"]
    probs = oracle.filter_to_probs(logits, float(t), int(k), float(p))
    assert np.array_equal(bits(probs), bits(GOLDEN[f"sample_{case}_probs"]))
    tok = oracle.sample_token(logits, float(t), int(k), float(p), float(np.float32(u)))
    assert tok == int(GOLDEN[f"sample_{case}_token"][0])


def test_sampler_kats():
    """Known answers of reference tools/selftest.cc:565-644."""
    assert oracle.sample_token(np.array([1, 9, 3], np.float32), 0.0, 0, 1.0, 0.123) == 1
    probs = oracle.filter_to_probs(np.array([5, 4, 3, 2, 1, 0], np.float32), 1.0, 2, 1.0)
    assert (probs > 0).sum() == 2 and probs[0] > 0 and probs[1] > 0 and probs[5] == 0
    lg = np.log(np.array([0.5, 0.3, 0.15, 0.05], np.float32))
    pr = oracle.filter_to_probs(lg, 1.0, 0, 0.9)
    assert (pr > 0).sum() == 3 and pr[3] == 0
    pr = oracle.filter_to_probs(lg, 1.0, 0, 0.3)
    assert pr[0] == 1.0 and pr[1] == 0.0
    flat = np.zeros(4, np.float32)
    assert [oracle.sample_token(flat, 1.0, 0, 1.0, u) for u in (0.0, 0.24, 0.26, 0.99)] == [0, 0, 1, 3]
    lg3 = np.array([4, 2, 0], np.float32)
    assert [oracle.sample_token(lg3, t, 0, 1.0, 0.95) for t in (0.5, 1.0, 2.0)] == [0, 1, 2]


def test_expf_special_values():
    """glibc expf: exact at 0, correctly rounded in these ranges (the check
    against the host libm over all floats is oracle/checks/expf_check.cc)."""
    f = oracle.lib().orc_expf
    assert f(0.0) == 1.0 and f(-0.0) == 1.0
    assert f(float("-inf")) == 0.0 and math.isinf(f(float("inf")))
    for x in np.linspace(-80, 80, 257, dtype=np.float32):
        want = np.float32(math.exp(float(x)))
        got = np.float32(f(float(x)))
        assert abs(int(got.view(np.int32)) - int(want.view(np.int32))) <= 1


def test_restated_expf_matches_glibc_on_every_float():
    """The restated glibc expf that the GPU runs (rpgbarengine_amd/csrc/
    expf_glibc.h, compiled for the host) against the host's glibc expf on
    all 2^32 float bit patterns (oracle/checks/expf_check.cc, ~15 s on 8
    threads)."""
    import subprocess
    exe = os.path.join(os.path.dirname(oracle.LIB_PATH), "expf_check")
    if not os.path.exists(exe):
        pytest.fail(f"{exe} is not built: run `make -C oracle port`")
    r = subprocess.run([exe, "0", str(1 << 32), str(min(8, os.cpu_count() or 1))], capture_output=True, text=True)
    assert r.returncode == 0 and "0 mismatches" in r.stdout, r.stdout + r.stderr


def test_tie_order_model_matches_libstdcxx_sort():
    """The partition model behind the GPU sampler's top-p tie order
    (sampler.hip, TieOrder) reproduces the order std::sort (libstdc++, the
    reference's sort, src/sampler.cc:72-76) leaves equal keys in, on random
    and structured arrays of 17..151938 keys, with the real depth budget and
    with small forced budgets that take the heap-sort branch
    (oracle/checks/tie_order_check.cc)."""
    import subprocess
    exe = os.path.join(os.path.dirname(oracle.LIB_PATH), "tie_order_check")
    if not os.path.exists(exe):
        pytest.fail(f"{exe} is not built: run `make -C oracle port`")
    r = subprocess.run([exe, "400"], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr


# ---------------------------------------------------------------- model


@pytest.fixture(scope="module")
def tiny_models(tmp_path_factory):
    d = tmp_path_factory.mktemp("golden_gguf")
    out = {}
    for mix in ("q4_k_m", "q8_0", "other"):
        spec = synth.PRESETS["tiny"].with_(mix=synth.MIXES[mix], seed=11)
        out[mix] = synth.write_gguf(str(d / f"tiny_{mix}.gguf"), spec)
    return out


@pytest.mark.parametrize("mix", ["q4_k_m", "q8_0", "other"])
def test_model_matches_reference_golden(tiny_models, mix):
    """Prefill logits bit for bit, greedy and sampled ids identical
    (reference src/qwen3.cc:208-363)."""
    m = oracle.Model(tiny_models[mix], threads=2)
    ids = GOLDEN[f"model_{mix}_ids"]
    kv = m.kv(64)
    logits = m.forward(ids, kv)
    assert np.array_equal(bits(logits[-1]), bits(GOLDEN[f"model_{mix}_last_logits"]))
    greedy = m.generate(kv, logits[-1], len(GOLDEN[f"model_{mix}_greedy"]))
    assert np.array_equal(greedy, GOLDEN[f"model_{mix}_greedy"])
    kv2 = m.kv(64)
    lg2 = m.forward(ids, kv2)
    sampled = m.generate(kv2, lg2[-1], len(GOLDEN[f"model_{mix}_sampled"]), temperature=0.8, top_k=40,
                         top_p=0.95, seed=77)
    assert np.array_equal(sampled, GOLDEN[f"model_{mix}_sampled"])


def test_cache_equals_nocache(tiny_models):
    """Prefill through the KV cache equals the cache-free forward bitwise (the
    invariant of reference tools/gen_check.cc:143-162), and two 8-token
    segments (the blocked matmul's token group) equal one 16-token pass."""
    m = oracle.Model(tiny_models["q4_k_m"], threads=2)
    ids = GOLDEN["model_q4_k_m_ids"]
    kv = m.kv(64)
    whole = m.forward(ids, kv)
    assert np.array_equal(bits(whole), bits(m.forward(ids, None)))
    kv2 = m.kv(64)
    m.forward(ids[:8], kv2)
    tail = m.forward(ids[8:], kv2)
    assert np.array_equal(bits(whole[8:]), bits(tail))


def test_softmax_rmsnorm_closed_forms():
    """Softmax and RMSNorm against float64 closed forms (reference
    src/kernels.h:56-79)."""
    x = np.array([3.0, -1.0, 2.0, 0.5], np.float32)
    s = x.copy()
    oracle.lib().orc_softmax(s.ctypes.data, 4)
    e = np.exp(x.astype(np.float64) - 3.0)
    assert np.allclose(s, e / e.sum(), rtol=1e-6)
    w = np.array([1.0, 2.0, 0.5, 1.5], np.float32)
    out = np.zeros(4, np.float32)
    oracle.lib().orc_rmsnorm(x.ctypes.data, w.ctypes.data, 4, np.float32(1e-6), out.ctypes.data)
    ref = x.astype(np.float64) / math.sqrt(float(np.mean(x.astype(np.float64) ** 2)) + 1e-6) * w
    assert np.allclose(out, ref, rtol=1e-6)


def attention_f64(q, k, v, pos0):
    """Causal GQA attention in float64: query t of head h sees positions
    0 .. pos0 + t of KV head h // G; softmax of q.k / sqrt(hd)."""
    seq, n_heads, hd = q.shape
    G = n_heads // k.shape[0]
    out = np.zeros(q.shape, np.float64)
    for h in range(n_heads):
        kh = h // G
        for t in range(seq):
            n = pos0 + t + 1
            s = k[kh, :n].astype(np.float64) @ q[t, h].astype(np.float64) / math.sqrt(hd)
            p = np.exp(s - s.max())
            out[t, h] = (p / p.sum()) @ v[kh, :n].astype(np.float64)
    return out


@pytest.mark.parametrize("seq,n_heads,n_kv,pos0,qscale", [(5, 4, 1, 0, 1.0), (9, 8, 2, 6, 1.0), (7, 4, 4, 3, 8.0)])
def test_attention_closed_form(seq, n_heads, n_kv, pos0, qscale):
    """The oracle's attention (reference src/qwen3.cc:79-117) against the float64
    softmax formula: GQA head grouping, the causal bound, a cache offset and a
    peaked softmax. A wrong group (h % n_kv), an off-by-one in the visible
    positions or a missing 1/sqrt(hd) each break it by far more than 1e-5."""
    rng = np.random.default_rng(seq * 100 + n_heads)
    q = (rng.standard_normal((seq, n_heads, 128)) * qscale).astype(np.float32)
    k = rng.standard_normal((n_kv, pos0 + seq, 128)).astype(np.float32)
    v = rng.standard_normal((n_kv, pos0 + seq, 128)).astype(np.float32)
    got = oracle.attention(q, k, v, pos0)
    want = attention_f64(q, k, v, pos0)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(v).max()


def test_round_half_matches_ieee_binary16():
    """The fp16-cache measurement's rounding (the oracle's RoundToHalf) is
    IEEE binary16 round-to-nearest-even (numpy's float16 conversion) on
    random magnitudes from 2^-30 to 2^17, the subnormal range, exact ties,
    the overflow boundary and specials."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(200000) * np.exp2(rng.uniform(-30, 17, 200000))).astype(np.float32)
    ties = np.array([1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 2.0 ** -24 * 1.5, 2.0 ** -24 * 2.5, 2.0 ** -25,
                     65504.0, 65519.996, 65520.0, 70000.0, 2.0 ** -14 * (1 + 2.0 ** -11), 0.0, -0.0,
                     np.inf, -np.inf], dtype=np.float32)
    x = np.concatenate([x, ties, -ties])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).astype(np.float32)
    got = oracle.round_half(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
