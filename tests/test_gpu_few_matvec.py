"""The few-token matvec -- the batched decode step's projections and short
prefill segments, 1..64 tokens (groups of 8 or 4 tokens per workgroup) on
the int8 matrix cores over tile-major copies -- through rpg_hip_matvec_few
against the CPU oracle: the per-row bound for every token count and the
widths the models use (a single super-block, an odd count, the longest
inputs, where the tokens are split between workgroups), extreme inputs in
one launch, the RMSNorm staging, the SwiGLU pair and the residual add.
Q8_0 launches stage four digits per input (128 bytes per token and
32-group): they take widths up to 8448 (6912 with a gain) and refuse wider
ones, which the engine runs on the GEMMs."""

import numpy as np
import pytest

import oracle
import rpgbarengine_amd as eng
from rpgbarengine_amd import synth
from tests.conftest import rel_row_error, split_terms

pytestmark = pytest.mark.gpu

TYPES = [synth.Q4_K, synth.Q6_K, synth.Q8_0]
# (K, rows): one super-block, odd super-block counts, the 4B model's widths
# (2560, 4096, 9728 -- the last splits 8 tokens over two workgroups), the
# 1.7B model's down width, the widest Q8_0 launch, the largest staged width;
# row counts off the 16-row tile
SHAPES = [(256, 37), (2304, 300), (2560, 1000), (4096, 130), (6144, 300), (8448, 40), (9728, 130), (10240, 17)]
Q8_MAX_K = 8448  # four-digit records of 4 tokens within the staging budget


def _q8_too_wide(qtype, k):
    return qtype == synth.Q8_0 and k > Q8_MAX_K


def _weights(qtype, k, rows, seed=3):
    w32 = synth.gaussian(seed, k * 7 + rows + qtype, rows * k, 0.02).reshape(rows, k)
    raw = synth.quantize(qtype, w32)
    wdq = oracle.dequant(qtype, raw.reshape(-1), rows * k).reshape(rows, k)
    return raw, wdq


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("k,rows", SHAPES)
@pytest.mark.parametrize("n", [1, 3, 4, 5, 8, 9, 16, 33, 64])
def test_few_row_bound(qtype, k, rows, n):
    """max|d| / sum|a*w| <= 1e-6 per row and token against float64
    (reference tools/check_dotrow.py:40-41)."""
    raw, wdq = _weights(qtype, k, rows)
    X = synth.gaussian(5, n + k, n * k, 1.0).reshape(n, k)
    if _q8_too_wide(qtype, k):
        with pytest.raises(eng.EngineError):
            eng.matvec_few(qtype, raw, rows, k, X)
        return
    Y = eng.matvec_few(qtype, raw, rows, k, X)
    assert rel_row_error(Y, X, wdq) <= 1e-6


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("k,n", [(2560, 8), (4096, 8), (2560, 40), (6144, 24), (9728, 24)])
def test_few_tokens_are_independent(qtype, k, n):
    """Each token's outputs are bit-identical to a launch of that token
    alone: a token's sums never depend on which other tokens share the
    launch, on its slot or on its token group (a wrong token offset fails
    here)."""
    if _q8_too_wide(qtype, k):
        pytest.skip("Q8_0 few-token launches stop at K = 8448")
    rows = 300
    raw, _ = _weights(qtype, k, rows, seed=4)
    X = synth.gaussian(6, k, n * k, 1.0).reshape(n, k)
    X[3] *= np.float32(1e-3)
    Y = eng.matvec_few(qtype, raw, rows, k, X)
    for t in range(n):
        y1 = eng.matvec_few(qtype, raw, rows, k, X[t:t + 1])
        assert np.array_equal(Y[t].view(np.uint32), y1[0].view(np.uint32)), t


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("k,rows", [(2560, 200), (6144, 64), (9728, 64)])
def test_few_extreme_inputs_in_one_launch(qtype, k, rows):
    """Tokens of different kinds side by side: uniform (the reference's
    tools/dotrow_check.cc:112-118 protocol), an outlier 3e4 times the rest,
    tiny (1e-30) and all-zero inputs. Zero rows give exact zeros; the
    outlier and tiny rows are held to the bound relative to
    sum|a|(|A| + |B|) (the format's two terms per weight, w = A - B)."""
    if _q8_too_wide(qtype, k):
        pytest.skip("Q8_0 few-token launches stop at K = 8448")
    raw, wdq = _weights(qtype, k, rows, seed=5)
    rng = np.random.default_rng(k + rows)
    kinds = ["uniform", "outlier", "tiny", "zero", "uniform", "zero", "outlier", "tiny"]
    X = np.zeros((len(kinds), k), dtype=np.float32)
    for t, kind in enumerate(kinds):
        if kind == "uniform":
            sc = np.float32([0.5, 1.0, 3.0, 12.0][t % 4])
            X[t] = (rng.random(k, dtype=np.float32) * 2.0 - 1.0) * sc
        elif kind != "zero":
            X[t] = synth.gaussian(12 + t, k, k, 1.0)
            if kind == "outlier":
                X[t, 7] = 3.0e4
                X[t, k - 3] = -1.0e-3
            else:
                X[t] *= np.float32(1e-30)
    Y = eng.matvec_few(qtype, raw, rows, k, X)
    AB = [np.abs(np.stack(split_terms(qtype, raw[r], k))).sum(axis=0) for r in range(rows)]
    for t, kind in enumerate(kinds):
        if kind == "zero":
            assert np.all(Y[t] == 0.0), t
        elif kind == "uniform":
            assert rel_row_error(Y[t:t + 1], X[t:t + 1], wdq) <= 1e-6, t
        else:
            ref = X[t].astype(np.float64) @ wdq.astype(np.float64).T
            ax = np.abs(X[t].astype(np.float64))
            bound = np.array([ax @ AB[r] for r in range(rows)])
            assert float(np.max(np.abs(Y[t].astype(np.float64) - ref) / bound)) <= 1e-6, t


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("k,n", [(2560, 8), (4096, 3), (2048, 6), (256, 1), (2560, 24), (4096, 64)])
def test_few_rmsnorm_staging(qtype, k, n):
    """RMSNorm folded into the staging: each token normalised as the
    reference does (src/qwen3.cc:131-134, the oracle's orc_rmsnorm), then
    the row bound against float64. The GPU's double sum of squares runs in
    another order: its float scale may differ by an ulp, a 1.2e-7 relative
    change, inside the bound."""
    rows = 160
    raw, wdq = _weights(qtype, k, rows, seed=6)
    X = synth.gaussian(7, k + n, n * k, 3.0).reshape(n, k)
    gain = (1.0 + synth.gaussian(8, k, k, 0.01)).astype(np.float32)
    Y = eng.matvec_few(qtype, raw, rows, k, X, norm_w=gain, eps=1e-6)
    L = oracle.lib()
    Xn = np.empty_like(X)
    for t in range(n):
        L.orc_rmsnorm(oracle._p(X[t]), oracle._p(gain), k, 1e-6, oracle._p(Xn[t]))
    assert rel_row_error(Y, Xn, wdq) <= 1e-6


def test_few_rmsnorm_width_limit():
    """The normed staging holds one 8-value chunk per thread: inputs wider
    than 4096 with a gain are refused (the engine then normalises first and
    runs the plain launch)."""
    k, rows = 4352, 16
    raw, _ = _weights(synth.Q4_K, k, rows, seed=6)
    X = synth.gaussian(7, k, k, 1.0).reshape(1, k)
    with pytest.raises(eng.EngineError):
        eng.matvec_few(synth.Q4_K, raw, rows, k, X, norm_w=np.ones(k, dtype=np.float32))


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("k,rows,n", [(2560, 200, 8), (2560, 9, 1), (256, 24, 5), (2560, 200, 40)])
def test_few_swiglu_pair(qtype, k, rows, n):
    """silu(x.g) * (x.u) from one pair launch against float64 products and
    the reference SwiGLU (src/kernels.h:82-92): the error propagated from
    the two dots' bounds (|silu'| <= 1.1) plus a few float roundings."""
    graw, gdq = _weights(qtype, k, rows, seed=9)
    uraw, udq = _weights(qtype, k, rows, seed=10)
    X = synth.gaussian(11, k, n * k, 1.0).reshape(n, k)
    Y = eng.matvec_few(qtype, graw, rows, k, X, up=uraw).astype(np.float64)
    X64 = X.astype(np.float64)
    g = X64 @ gdq.astype(np.float64).T
    u = X64 @ udq.astype(np.float64).T
    eg = 1e-6 * (np.abs(X64) @ np.abs(gdq.astype(np.float64)).T)
    eu = 1e-6 * (np.abs(X64) @ np.abs(udq.astype(np.float64)).T)
    silu = g / (1.0 + np.exp(-g))
    want = silu * u
    bound = 1.1 * np.abs(u) * eg + np.abs(silu) * eu + 1e-6 * np.abs(want) + 1e-30
    assert float(np.max(np.abs(Y - want) / bound)) <= 1.0


@pytest.mark.parametrize("qtype", TYPES)
def test_few_residual_add(qtype):
    """The residual epilogue adds the launch's own sums to y: bit for bit
    float32(y + (x . w)) of the storing launch."""
    k, rows, n = 4096, 140, 7
    raw, _ = _weights(qtype, k, rows, seed=12)
    X = synth.gaussian(13, k, n * k, 1.0).reshape(n, k)
    y0 = synth.gaussian(14, rows, n * rows, 2.0).reshape(n, rows)
    stored = eng.matvec_few(qtype, raw, rows, k, X)
    added = eng.matvec_few(qtype, raw, rows, k, X, add_to=y0)
    assert np.array_equal(added.view(np.uint32), (y0 + stored).astype(np.float32).view(np.uint32))
