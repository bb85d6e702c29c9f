"""The Q80_SCALAR option: Q8_0 activations by the reference's portable
scalar quantizer (reference src/kernels.c:542-558), which the reference
runs instead of the SIMD one when SI_SCALAR is set (kernels.c:80-83) or
the host has no AVX2. Checked against the oracle's scalar quantizer, which
tests/test_oracle.py pins to the compiled reference's golden blocks.

The inputs hold blocks on which the two quantizers differ (ties at .5,
which roundf sends away from zero and the SIMD path to even), so a device
that ignored the option fails here."""
import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth

TOL_REL, TOL_ABS = 1e-5, 1e-6


def tie_vector(rng, n):
    """N(0,1) activations; every fourth block is rescaled so its largest
    magnitude is exactly 127 (id = 1 on both paths) with values at k + 0.5."""
    x = rng.standard_normal(n).astype(np.float32)
    for b in range(0, n // 32, 4):
        blk = np.round(rng.uniform(-40, 40, 32)).astype(np.float32) + 0.5
        blk[rng.integers(0, 32)] = 127.0 if b % 8 == 0 else -127.0
        x[32 * b:32 * b + 32] = blk
    return x


def test_tie_vector_separates_the_quantizers(oracle):
    x = tie_vector(np.random.default_rng(1), 1024)
    assert not np.array_equal(oracle.quantize(sa.Q8_0, x),
                              oracle.quantize(sa.Q8_0, x, scalar_q8_0=True))


@pytest.mark.gpu
@pytest.mark.parametrize("n", [32, 896, 5120])
def test_quantize_q8_0_scalar_bitexact(dev, oracle, option, n):
    rng = np.random.default_rng(300 + n)
    vecs = [tie_vector(rng, n), rng.standard_normal(n).astype(np.float32),
            np.zeros(n, np.float32)]
    z = np.zeros(n, np.float32)
    z[-1] = -1e-30  # a tiny block maximum: its f16 scale underflows to zero
    vecs.append(z)
    option("Q80_SCALAR", 1)
    for x in vecs:
        assert np.array_equal(dev.quantize(sa.Q8_0, x), oracle.quantize(sa.Q8_0, x, scalar_q8_0=True))
    # back to the rule: the SIMD quantizer
    dev.set_option("Q80_SCALAR", -1)
    x = vecs[0]
    assert np.array_equal(dev.quantize(sa.Q8_0, x), oracle.quantize(sa.Q8_0, x))


def oracle_rows(oracle, wt, W, n_in, xq):
    """Per-row reference dots of W against the pair-format activation xq."""
    n_out = W.shape[0]
    y = np.zeros(n_out)
    l1 = np.zeros(n_out)
    for r in range(n_out):
        y[r], l1[r] = oracle.vec_dot(wt, n_in, W[r], xq)
    return y, l1


@pytest.mark.gpu
@pytest.mark.parametrize("wt", [sa.Q8_0, sa.Q4_0, sa.Q5_0], ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("M", [1, 8])
def test_gemv_gemm_scalar_activations(dev, oracle, option, wt, M):
    """Batch 1 runs the matvec kernel (the quantizer in its prologue),
    batch 8 the matrix-core GEMM (16-row m blocks: the quantizer in the
    GEMM launch's own prologue)."""
    rng = np.random.default_rng(400 + wt + M)
    n_out, n_in = 96, 1024
    W = synth.make_weights(wt, n_out, n_in, rng)
    X = np.stack([tie_vector(rng, n_in) for _ in range(M)])
    option("Q80_SCALAR", 1)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        Y = dev.gemv(w, X[0])[None, :] if M == 1 else dev.gemm(w, X)
    finally:
        w.free()
    for m in range(M):
        ref, l1 = oracle_rows(oracle, wt, W, n_in, oracle.quantize(sa.Q8_0, X[m], scalar_q8_0=True))
        err = np.abs(Y[m].astype(np.float64) - ref)
        bad = np.nonzero(~(err <= TOL_REL * l1 + TOL_ABS))[0]
        assert bad.size == 0, f"{sa.NAMES[wt]} M={M} row {m}: {bad.size} outputs out of tolerance"
