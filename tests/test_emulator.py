"""CPU checks of the matvec kernel logic through its host emulation
(tests/emu compiles the product's formats.h / unit.h for the CPU): repack
layout, per-format decode, scale extraction and the lane reduction order,
for every format and every tile shape, against the oracle."""
import numpy as np
import pytest

from oracle import siq
from siphon_amd import synth

KQ = (siq.Q2_K, siq.Q3_K, siq.Q4_K, siq.Q5_K, siq.Q6_K)


@pytest.mark.parametrize("wt", siq.WEIGHT_TYPES, ids=lambda t: siq.NAMES[t])
def test_emulated_matvec_vs_oracle(oracle, emu, wt):
    rng = np.random.default_rng(500 + wt)
    shapes = [(1, 256), (37, 1024), (64, 2048), (130, 768), (3, 1792)] if wt in KQ else \
             [(1, 32), (37, 1024), (64, 2048), (130, 896), (5, 160)]
    for (n_out, n_in) in shapes:
        W = synth.make_weights(wt, n_out, n_in, rng)
        x = rng.standard_normal(n_in).astype(np.float32)
        xq = oracle.quantize(siq.PAIR[wt], x)
        ref = np.zeros(n_out)
        l1 = np.zeros(n_out)
        for r in range(n_out):
            ref[r], l1[r] = oracle.vec_dot(wt, n_in, W[r], xq)
        for G in [1, 2, 4, 8, 16, 32, 64]:  # padding columns where G does not divide
            y = emu.gemv_pair(wt, n_out, n_in, G, W, xq)
            err = np.abs(y - ref)
            assert np.all(err <= 1e-5 * l1 + 1e-6), (siq.NAMES[wt], n_out, n_in, G)


@pytest.mark.parametrize("wt", siq.WEIGHT_TYPES, ids=lambda t: siq.NAMES[t])
def test_emulated_column_slices_vs_oracle(oracle, emu, wt):
    """Rows cut into column slices (one round per slice up to the whole
    row), the partial sums added in slice order, stay within tolerance of
    the oracle; a slice length of at least the row is the unsliced kernel
    bit for bit."""
    rng = np.random.default_rng(700 + wt)
    n_out, n_in = (21, 2304) if wt in KQ else (21, 1120)
    W = synth.make_weights(wt, n_out, n_in, rng)
    x = rng.standard_normal(n_in).astype(np.float32)
    xq = oracle.quantize(siq.PAIR[wt], x)
    ref = np.zeros(n_out)
    l1 = np.zeros(n_out)
    for r in range(n_out):
        ref[r], l1[r] = oracle.vec_dot(wt, n_in, W[r], xq)
    for G in [1, 2, 8, 64]:
        whole = emu.gemv_pair(wt, n_out, n_in, G, W, xq, slice_elems=0)
        same = emu.gemv_pair(wt, n_out, n_in, G, W, xq, slice_elems=n_in)
        assert np.array_equal(whole.view(np.uint32), same.view(np.uint32))
        for elems in [1, 256, 1024]:
            y = emu.gemv_pair(wt, n_out, n_in, G, W, xq, slice_elems=elems)
            err = np.abs(y - ref)
            assert np.all(err <= 1e-5 * l1 + 1e-6), (siq.NAMES[wt], G, elems)


def test_repack_is_a_permutation(emu):
    """Device bytes hold every GGUF byte's information: repacking a matrix
    whose every bit is set gives exactly as many set bits as the GGUF bytes
    (plus zero padding), for every format."""
    for wt in siq.WEIGHT_TYPES:
        n_out, n_in = 5, 512
        be, bb = siq.GEOM[wt]
        W = np.full((n_out, n_in // be * bb), 0xFF, np.uint8)
        dev = emu.repack(wt, n_out, n_in, 4, W)
        assert int(np.unpackbits(dev).sum()) == int(np.unpackbits(W).sum()), siq.NAMES[wt]


@pytest.mark.parametrize("wt", siq.WEIGHT_TYPES, ids=lambda t: siq.NAMES[t])
def test_emulated_dequant_bitexact(oracle, emu, wt):
    """The device dequantizer's decode (unit.h) through the planar layout
    reproduces the reference dequantization bit for bit, for every tile
    width (padding rows and columns included)."""
    rng = np.random.default_rng(800 + wt)
    n_out, n_in = (37, 1792) if wt in KQ else (37, 1120)
    W = synth.make_weights(wt, n_out, n_in, rng)
    ref = np.stack([oracle.dequant(wt, W[r], n_in) for r in range(n_out)])
    for G in [1, 4, 64]:
        got = emu.dequant(wt, n_out, n_in, G, W)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (siq.NAMES[wt], G)
