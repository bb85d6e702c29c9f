"""The matrix-core GEMMs' activation quantizer (gemm2_quantize_x: 16 lanes
per 256-element block, the records the Q4_K, Q6_K and small-M kernels read)
is the reference's Q8_K quantizer (reference kernels.c:561-595) bit for bit:
quants, d and the group sums of every row, read back from the records
(sihip_quantize_q8_K_rows), for every m-block height and for ragged M
(rows past M are padding). The rows include the quantizer's edge cases:
ties of the largest |x| with both signs (the first occurrence sets the
sign, which a GEMM output would not show), zeros, subnormals, huge values."""
import numpy as np
import pytest

import siphon_amd as sa

from .test_gpu_parity import edge_vectors

pytestmark = pytest.mark.gpu


def _want(oracle, X):
    return np.concatenate([oracle.quantize(sa.Q8_K, x) for x in X])


@pytest.mark.parametrize("bm", [16, 32, 64, 128])
@pytest.mark.parametrize("M,n_in", [(1, 256), (5, 4096), (37, 1024), (130, 512)])
def test_gemm_records_bitexact(dev, oracle, bm, M, n_in):
    rng = np.random.default_rng(bm * 1000 + M)
    edges = edge_vectors(rng, n_in)
    X = rng.standard_normal((M, n_in)).astype(np.float32)
    for i in range(min(M, len(edges))):
        X[i] = edges[i]
    got = dev.quantize_gemm_rows(X, bm)
    want = _want(oracle, X)
    assert np.array_equal(got, want), f"bm={bm} M={M} n_in={n_in}"


def test_gemm_records_tie_block(dev, oracle):
    """Every lane holds a tie: |x| = 3 everywhere, signs alternating, so
    only the first-occurrence rule picks the sign."""
    x = np.full(256, 3.0, np.float32)
    x[::2] = -3.0
    X = np.stack([x, -x, np.zeros(256, np.float32), np.full(256, -0.0, np.float32)])
    got = dev.quantize_gemm_rows(X, 16)
    assert np.array_equal(got, _want(oracle, X))
