"""sihip_gemm_dev_noalloc: the GEMM entry point that allocates nothing (its
workspaces are a static device scratch). It runs the kernels of
sihip_gemm_dev, so its outputs must equal that entry point's bit for bit,
except where the K-slice partial sums of sihip_gemm_dev would not fit the
scratch: then it runs the tile unsliced, which adds the same terms in
another f32 order, and both are checked against the oracle to the path's
bar. Each case makes two calls in a row, the second with fewer rows, so a
leftover of the first call in the shared scratch (activation planes,
partial sums, arrival counters) would show in the second."""
import ctypes

import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth

from .test_gpu_parity import assert_close
from .test_gpu_slices import _HipGraph, bits

pytestmark = pytest.mark.gpu


def _gemm_both(dev, w, X):
    """(gemm_dev, gemm_dev_noalloc) outputs of one X, on device buffers."""
    M = X.shape[0]
    nan = np.full(M * w.n_out, np.nan, np.float32)
    xd, ya, yb = dev.to_device(X), dev.to_device(nan), dev.to_device(nan)
    try:
        dev.gemm_dev(w, xd.ptr, M, ya.ptr)
        dev.gemm_dev_noalloc(w, xd.ptr, M, yb.ptr)
        dev.synchronize()
        return (ya.to_host(np.float32, M * w.n_out).reshape(M, w.n_out),
                yb.to_host(np.float32, M * w.n_out).reshape(M, w.n_out))
    finally:
        for b in (xd, ya, yb):
            b.free()


# (type, n_out, n_in, first M, second M): the config-3 shape on the matrix
# cores, K-sliced small batches, the matvec path (M below the matrix-core
# threshold), the Q6_K, F16 and Q8_0-pair GEMMs with K slices; the slices
# of the UNSLICED calls do not fit the scratch (the F16 and Q8_0-pair
# kernels count K in 128-element steps, the others in super-blocks, and the
# unsliced call must cover all of them)
CASES = [
    (sa.Q4_K, 14336, 4096, 512, 96),
    (sa.Q2_K, 3072, 5120, 16, 8),
    (sa.Q5_K, 1000, 2048, 70, 33),
    (sa.Q4_K, 2048, 4096, 4, 2),
    (sa.Q6_K, 1024, 4096, 8, 3),
    (sa.Q6_K, 1024, 4096, 64, 20),
    (sa.Q6_K, 4096, 14336, 512, 40),
    (sa.Q5_0, 4096, 14336, 256, 40),
    (sa.F16, 4096, 14336, 256, 24),
    (sa.Q8_0, 4864, 896, 16, 5),
    (sa.Q4_0, 5632, 2048, 64, 9),
]
UNSLICED = {(sa.Q6_K, 4096, 14336, 512), (sa.Q5_0, 4096, 14336, 256),
            (sa.F16, 4096, 14336, 256)}  # (type, n_out, n_in, M) run unsliced


@pytest.mark.parametrize("wt,n_out,n_in,M1,M2", CASES,
                         ids=[f"{sa.NAMES[c[0]]}-{c[1]}x{c[2]}-M{c[3]}-{c[4]}" for c in CASES])
def test_noalloc_matches_gemm_dev(dev, oracle, wt, n_out, n_in, M1, M2):
    print(f"noalloc {sa.NAMES[wt]} {n_out}x{n_in} M={M1} then {M2}", flush=True)
    rng = np.random.default_rng(n_out + n_in + M1)
    W = synth.make_weights(wt, n_out, n_in, rng)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        w.prepare_gemm()
        for M in (M1, M2):
            X = rng.standard_normal((M, n_in)).astype(np.float32)
            ya, yb = _gemm_both(dev, w, X)
            assert not np.isnan(ya).any()
            if (wt, n_out, n_in, M) in UNSLICED:
                ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
                for y, what in ((ya, "gemm_dev"), (yb, "noalloc")):
                    assert_close(y.reshape(-1), ref.reshape(-1).astype(np.float64),
                                 L1.reshape(-1), f"{sa.NAMES[wt]} M={M} {what}")
                continue
            assert np.array_equal(bits(ya), bits(yb)), \
                f"{sa.NAMES[wt]} M={M}: noalloc differs from gemm_dev"
    finally:
        w.free()


def test_noalloc_refuses_what_it_cannot_do(dev):
    """A weight without its GEMM copy is refused (building it would
    allocate), and so is an activation whose planes exceed the scratch."""
    rng = np.random.default_rng(5)
    n_out, n_in = 256, 28672
    W = synth.make_weights(sa.Q4_K, n_out, n_in, rng)
    w = dev.upload(sa.Q4_K, n_out, n_in, W)
    xd = dev.alloc(16)
    yd = dev.alloc(16)
    try:
        with pytest.raises(sa.SihipError) as e:
            dev.gemm_dev_noalloc(w, xd.ptr, 64, yd.ptr)
        assert e.value.code == -5 and "prepare_gemm" in str(e.value)
        w.prepare_gemm()
        with pytest.raises(sa.SihipError) as e:  # 1024 x 28672 needs 33 MB of planes
            dev.gemm_dev_noalloc(w, xd.ptr, 1024, yd.ptr)
        assert e.value.code == -7 and "scratch" in str(e.value)
    finally:
        xd.free()
        yd.free()
        w.free()


def test_noalloc_graph_replays(dev):
    """The call captured into a HIP graph (it allocates nothing) replays to
    the eager bits, with eager calls of other shapes between the replays."""
    rng = np.random.default_rng(77)
    n_out, n_in, M = 4096, 4096, 64
    W = synth.make_weights(sa.Q4_K, n_out, n_in, rng)
    w = dev.upload(sa.Q4_K, n_out, n_in, W)
    w.prepare_gemm()
    hg = _HipGraph()
    nan = np.full(M * n_out, np.nan, np.float32)
    xd = dev.to_device(rng.standard_normal((M, n_in)).astype(np.float32))
    x2 = dev.to_device(rng.standard_normal((8, n_in)).astype(np.float32))
    ye, yg, y2 = dev.to_device(nan), dev.to_device(nan), dev.to_device(nan)
    try:
        dev.gemm_dev_noalloc(w, xd.ptr, M, ye.ptr, hg.stream.value)
        dev.synchronize()
        want = ye.to_host(np.float32, M * n_out).copy()
        hg.begin()
        dev.gemm_dev_noalloc(w, xd.ptr, M, yg.ptr, hg.stream.value)
        hg.end()
        for _ in range(3):
            yg.fill(nan)
            hg.replay()
            assert np.array_equal(bits(yg.to_host(np.float32, M * n_out)), bits(want))
            dev.gemm_dev_noalloc(w, x2.ptr, 8, y2.ptr, hg.stream.value)  # other use of the scratch
            dev.synchronize()
    finally:
        hg.close()
        for b in (xd, x2, ye, yg, y2):
            b.free()
        w.free()
