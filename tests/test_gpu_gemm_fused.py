"""GPU parity of the fused small-M K-quant launch (gemmkf_kernel: the
activation quantized to Q8_K inside the launch, several matrices over one X
in one grid, K slices added in slice order by the last workgroup of a tile)
against the oracle, every output, |gpu - ref| <= 1e-5 * sum|terms| + 1e-6.

Cases: every M of the launch (3 to 8) and K-quant; slice lengths from one
super-block to the whole row, slice counts that do not divide the row, rows
longer than the largest slice (56 super-blocks, 24 at most per slice);
tiles whose last 32-row blocks are past the matrix (a wave with no block);
groups of one format, of the mixes that share one launch (Q4_K + Q6_K,
Q5_K + Q6_K, Q3_K + Q5_K, Q2_K + Q3_K) and of formats that need a launch
each; repeated calls (the arrival counters start at zero each time) and
graph replays against eager calls."""
import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth

from .test_gpu_gemm import _rows
from .test_gpu_gemm_small import _weights
from .test_gpu_parity import assert_close
from .test_gpu_slices import _HipGraph, bits

pytestmark = pytest.mark.gpu

KQ = [sa.Q2_K, sa.Q3_K, sa.Q4_K, sa.Q5_K, sa.Q6_K]


@pytest.fixture(autouse=True)
def _fused_for_every_format(option):
    """GEMMKF_MAX_M set explicitly: every K-quant takes the fused launch,
    Q3_K with short rows included (the rule sends those to the separate
    launches)."""
    option("GEMMKF_MAX_M", 8)


def _multi(dev, ws, X):
    M = X.shape[0]
    xd = dev.to_device(X)
    ys = [dev.to_device(np.full(M * w.n_out, np.nan, np.float32)) for w in ws]
    try:
        dev.gemm_multi_dev(ws, xd.ptr, M, [y.ptr for y in ys])
        dev.synchronize()
        return [y.to_host(np.float32, M * w.n_out).reshape(M, w.n_out).copy()
                for w, y in zip(ws, ys)]
    finally:
        for b in [xd] + ys:
            b.free()


@pytest.mark.parametrize("wt", KQ, ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("M", [3, 4, 5, 6, 7, 8])
def test_fused_every_m(dev, oracle, wt, M):
    """n_out 200: two tiles, the second with 3 of its 4 blocks (the fourth
    wave has no rows); n_in 2304: 9 super-blocks, sliced by the rule."""
    print(f"fused {sa.NAMES[wt]} M={M}", flush=True)
    rng = np.random.default_rng(8100 + 31 * wt + M)
    n_out, n_in = 200, 2304
    W = _weights(wt, n_out, n_in, rng)
    X = _rows(rng, M, n_in)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
        Y2 = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                 f"{sa.NAMES[wt]} M={M}")
    assert np.array_equal(bits(Y), bits(Y2)), "a second call differs"


@pytest.mark.parametrize("wt", KQ, ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("sbk", [0, 1, 2, 4, 5])
def test_fused_slice_lengths(dev, oracle, option, wt, sbk):
    """GEMMKF_SBK: 0 (no slices: one slice of the 9 super-blocks), 1 (one
    per slice), 2, 4 (a short last slice), 5."""
    option("GEMMKF_SBK", sbk)
    rng = np.random.default_rng(8200 + 11 * wt + sbk)
    n_out, n_in, M = 300, 2304, 8
    W = _weights(wt, n_out, n_in, rng)
    X = _rows(rng, M, n_in)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                 f"{sa.NAMES[wt]} SBK={sbk}")


@pytest.mark.parametrize("wt", [sa.Q4_K, sa.Q6_K, sa.Q2_K], ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("sbk", [-1, 0], ids=["rule", "fewest"])
def test_fused_long_rows(dev, oracle, option, wt, sbk):
    """56 super-blocks per row (the Llama-3-8B ffn_down shape's n_in): the
    rule's slices, and the fewest slices the LDS image allows (24, 24, 8)."""
    if sbk >= 0:
        option("GEMMKF_SBK", sbk)
    rng = np.random.default_rng(8300 + wt + sbk)
    n_out, n_in, M = 160, 14336, 8
    W = _weights(wt, n_out, n_in, rng)
    X = _rows(rng, M, n_in)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                 f"{sa.NAMES[wt]} {n_out}x{n_in} sbk={sbk}")


# groups over one X: (label, [(type, n_out)], n_in, M)
GROUPS = [
    ("q4k-q4k-q6k", [(sa.Q4_K, 300), (sa.Q4_K, 100), (sa.Q6_K, 170)], 1024, 8),
    ("q5k-q6k", [(sa.Q5_K, 260), (sa.Q6_K, 96)], 1536, 7),
    ("q3k-q5k", [(sa.Q3_K, 128), (sa.Q5_K, 64)], 1024, 5),
    ("q2k-q3k", [(sa.Q2_K, 96), (sa.Q3_K, 200)], 2048, 8),
    ("q2k-q6k-separate", [(sa.Q2_K, 64), (sa.Q6_K, 130)], 1024, 6),
    ("three-formats", [(sa.Q3_K, 40), (sa.Q4_K, 300), (sa.Q5_K, 33), (sa.Q4_K, 64)], 768, 4),
]


@pytest.mark.parametrize("label,mats,n_in,M", GROUPS, ids=[g[0] for g in GROUPS])
def test_fused_groups(dev, oracle, label, mats, n_in, M):
    print(f"fused group {label}", flush=True)
    rng = np.random.default_rng(len(label) * 1013 + M)
    Ws = [_weights(wt, n_out, n_in, rng) for wt, n_out in mats]
    ws = [dev.upload(wt, n_out, n_in, W) for (wt, n_out), W in zip(mats, Ws)]
    try:
        for call in range(2):
            X = _rows(rng, M, n_in)
            Ys = _multi(dev, ws, X)
            for i, ((wt, n_out), W, Y) in enumerate(zip(mats, Ws, Ys)):
                ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
                assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                             f"{label} call {call} weight {i} ({sa.NAMES[wt]} {n_out}x{n_in})")
    finally:
        for w in ws:
            w.free()


def test_fused_group_graph_replays(dev):
    """The Llama-3-8B q/k/v group at M = 8 (one launch, Q4_K and Q6_K
    segments) captured in a graph: every replay gives the eager bits, with
    eager calls between the replays."""
    rng = np.random.default_rng(8400)
    n_in, M = 4096, 8
    mats = [(sa.Q4_K, 4096), (sa.Q4_K, 1024), (sa.Q6_K, 1024)]
    ws = [dev.upload(wt, n, n_in, synth.make_weights(wt, n, n_in, rng)) for wt, n in mats]
    hg = _HipGraph()
    bufs = []
    try:
        for w in ws:
            w.prepare_gemm()
        xd = dev.to_device(rng.standard_normal((M, n_in)).astype(np.float32))
        nan = [np.full(M * w.n_out, np.nan, np.float32) for w in ws]
        ye = [dev.to_device(v) for v in nan]
        yg = [dev.to_device(v) for v in nan]
        bufs = [xd, *ye, *yg]
        dev.gemm_multi_dev(ws, xd.ptr, M, [y.ptr for y in ye], hg.stream.value)
        dev.synchronize()
        want = [y.to_host(np.float32, M * w.n_out).copy() for w, y in zip(ws, ye)]
        hg.begin()
        dev.gemm_multi_dev(ws, xd.ptr, M, [y.ptr for y in yg], hg.stream.value)
        hg.end()
        for _ in range(3):
            for y, v in zip(yg, nan):
                y.fill(v)
            hg.replay()
            for w, y, e in zip(ws, yg, want):
                assert np.array_equal(bits(y.to_host(np.float32, M * w.n_out)), bits(e))
            for y, v in zip(ye, nan):
                y.fill(v)
            dev.gemm_multi_dev(ws, xd.ptr, M, [y.ptr for y in ye], hg.stream.value)
            dev.synchronize()
            for w, y, e in zip(ws, ye, want):
                assert np.array_equal(bits(y.to_host(np.float32, M * w.n_out)), bits(e))
    finally:
        hg.close()
        for b in bufs:
            b.free()
        for w in ws:
            w.free()


@pytest.mark.parametrize("wt,n_in", [(sa.Q6_K, 1024), (sa.Q4_K, 1536)],
                         ids=["Q6_K-head", "Q4_K-head"])
def test_fused_output_head(dev, oracle, wt, n_in):
    """A 151936-row output head at M = 8 (config 1's vocabulary): 1187
    tiles in one grid, every output against the oracle."""
    print(f"fused head {sa.NAMES[wt]} 151936x{n_in}", flush=True)
    rng = np.random.default_rng(8600 + wt)
    n_out, M = 151936, 8
    W = synth.make_weights(wt, n_out, n_in, rng)
    X = _rows(rng, M, n_in)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                 f"{sa.NAMES[wt]} head {n_out}x{n_in}")
