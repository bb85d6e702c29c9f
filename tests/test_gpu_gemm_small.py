"""GPU parity of the small-M GEMMs (the batched decode step): the fused
launch gemmkf_kernel (every K-quant, 3 <= M <= 8, the rule), and with it
turned off (GEMMKF_MAX_M = 0) gemm2s_q4k_kernel (Q4_K, 3 <= M <= 16) and
gemmks_kernel (Q2_K, Q5_K up to M = 8, Q3_K, Q6_K up to M = 12, by option
every K-quant up to 16) against the oracle, every output, |gpu - ref| <=
1e-5 * sum|terms| + 1e-6; the M values past a format's rule run its larger
GEMM. Shapes cover a single super-block per row (fewer super-blocks than
waves per workgroup), super-block counts that the waves do not divide,
row counts that leave a 32-row block part empty, every 4-row activation
group count (M = 3 to 16), each waves-per-workgroup choice, and rows at
the ends of each format's operand range."""
import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth

from .test_gpu_gemm import _extreme_q2k, _extreme_q3k, _extreme_q5k, _extreme_q6k, _rows
from .test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu

KQ = [sa.Q2_K, sa.Q3_K, sa.Q4_K, sa.Q5_K, sa.Q6_K]


def _weights(wt, n_out, n_in, rng):
    W = synth.make_weights(wt, n_out, n_in, rng)
    if wt == sa.Q2_K:
        W = _extreme_q2k(W, n_out, n_in)
    elif wt == sa.Q3_K:
        W = _extreme_q3k(W, n_out, n_in)
    elif wt == sa.Q5_K:
        W = _extreme_q5k(W, n_out, n_in)
    elif wt == sa.Q6_K:
        W = _extreme_q6k(W, n_out, n_in)
    return W


def _check(dev, oracle, wt, n_out, n_in, M, seed, what):
    rng = np.random.default_rng(seed)
    W = _weights(wt, n_out, n_in, rng)
    X = _rows(rng, M, n_in)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1), what)


# (M, fused launch): the fused launch takes M <= 8
M_CASES = [(m, True) for m in (3, 4, 5, 8)] + [(m, False) for m in (3, 4, 5, 8, 9, 12, 16)]


@pytest.mark.parametrize("wt", KQ, ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("M,fused", M_CASES,
                         ids=[f"M{m}-{'fused' if f else 'separate'}" for m, f in M_CASES])
@pytest.mark.parametrize("n_out,n_in", [(33, 256), (200, 1024), (96, 2304)])
def test_small_m_vs_oracle(dev, oracle, option, wt, M, n_out, n_in, fused):
    option("GEMMKF_MAX_M", 8 if fused else 0)
    _check(dev, oracle, wt, n_out, n_in, M, 7000 + 97 * wt + 13 * M + n_in,
           f"{sa.NAMES[wt]} {n_out}x{n_in} M={M} {'fused' if fused else 'separate'}")


@pytest.mark.parametrize("wt", KQ, ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("waves", [2, 4, 8])
def test_small_m_waves_per_workgroup(dev, oracle, option, wt, waves):
    option("GEMMKF_MAX_M", 0)
    option("GEMMS_WAVES", waves)
    _check(dev, oracle, wt, 160, 2560, 8, 7100 + wt + waves, f"{sa.NAMES[wt]} waves={waves}")


@pytest.mark.parametrize("wt", KQ, ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("M", [9, 12, 13, 16])
def test_small_m_wide_groups_by_option(dev, oracle, option, wt, M):
    """Three and four activation groups per MFMA (M = 9 to 16), which the
    rule gives to the larger GEMMs for some formats: GEMMKS_MAX_M = 16 keeps
    every K-quant on gemmks.h (Q4_K with GEMMKS_Q4K)."""
    option("GEMMKS_MAX_M", 16)
    option("GEMMKS_Q4K", 1)
    _check(dev, oracle, wt, 200, 1024, M, 7400 + 31 * wt + M, f"{sa.NAMES[wt]} gemmks M={M}")


@pytest.mark.parametrize("M", [5, 8])
def test_small_m_q4k_on_the_generic_kernel(dev, oracle, option, M):
    """Q4_K at small M on gemmks.h (the GEMMKS_Q4K option) as well as on
    gemm2s.h (the rule)."""
    option("GEMMKF_MAX_M", 0)
    option("GEMMKS_Q4K", 1)
    _check(dev, oracle, sa.Q4_K, 200, 1024, M, 7200 + M, f"Q4_K gemmks M={M}")


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "separate"])
def test_small_m_graph_replays_match_eager(dev, option, fused):
    """A captured small-M call (the fused launch, or Q4_K on gemm2s.h, Q6_K
    and Q3_K on gemmks.h) replays bit-identically to the eager call,
    several times with eager calls in between."""
    from .test_gpu_slices import _HipGraph, bits
    option("GEMMKF_MAX_M", 8 if fused else 0)
    rng = np.random.default_rng(7300)
    n_out, n_in, M = 4096, 4096, 8
    ws = [dev.upload(wt, n_out, n_in, synth.make_weights(wt, n_out, n_in, rng))
          for wt in (sa.Q4_K, sa.Q6_K, sa.Q3_K)]
    hg = _HipGraph()
    bufs = []
    try:
        for w in ws:
            w.prepare_gemm()
        nan = np.full(M * n_out, np.nan, np.float32)
        xd = dev.to_device(rng.standard_normal((M, n_in)).astype(np.float32))
        ye = [dev.to_device(nan) for _ in ws]
        yg = [dev.to_device(nan) for _ in ws]
        bufs = [xd, *ye, *yg]
        for w, y in zip(ws, ye):
            dev.gemm_dev(w, xd.ptr, M, y.ptr, hg.stream.value)
        dev.synchronize()
        want = [y.to_host(np.float32, M * n_out).copy() for y in ye]
        hg.begin()
        for w, y in zip(ws, yg):
            dev.gemm_dev(w, xd.ptr, M, y.ptr, hg.stream.value)
        hg.end()
        for _ in range(3):
            for y in yg:
                y.fill(nan)
            hg.replay()
            for y, e in zip(yg, want):
                assert np.array_equal(bits(y.to_host(np.float32, M * n_out)), bits(e))
            for w, y in zip(ws, ye):
                y.fill(nan)
                dev.gemm_dev(w, xd.ptr, M, y.ptr, hg.stream.value)
            dev.synchronize()
            for y, e in zip(ye, want):
                assert np.array_equal(bits(y.to_host(np.float32, M * n_out)), bits(e))
    finally:
        hg.close()
        for b in bufs:
            b.free()
        for w in ws:
            w.free()
