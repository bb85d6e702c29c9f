"""Launches on several streams that share mutable device state: a
column-sliced weight's partial sums and arrival counters, and a context's
GEMM workspaces. The library orders such launches across streams (the
first switch drains the device, later ones wait on an event recorded after
the previous launch), so calls alternating between two streams with no
synchronization in between give the bits of eager calls on one stream,
and a stream destroyed after its calls leaves nothing behind that a later
call touches."""
import ctypes

import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth

from .test_gpu_slices import bits

pytestmark = pytest.mark.gpu


class _Streams:
    """Streams of the HIP runtime the library links (no second runtime)."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.handles = []

    def create(self):
        s = ctypes.c_void_p()
        assert self.hip.hipStreamCreate(ctypes.byref(s)) == 0
        self.handles.append(s)
        return s.value

    def sync(self, s):
        assert self.hip.hipStreamSynchronize(ctypes.c_void_p(s)) == 0

    def destroy(self, s):
        for h in self.handles:
            if h.value == s:
                assert self.hip.hipStreamDestroy(h) == 0
                self.handles.remove(h)
                return

    def close(self):
        for h in self.handles:
            self.hip.hipStreamDestroy(h)
        self.handles = []


def test_sliced_weight_on_two_streams(dev):
    rng = np.random.default_rng(31)
    n_out, n_in = 4096, 14336
    W = synth.make_weights(sa.Q6_K, n_out, n_in, rng)
    w = dev.upload(sa.Q6_K, n_out, n_in, W)
    assert w.slice_rounds > 0  # long rows: column slices with shared partial sums
    ss = _Streams()
    bufs = []
    try:
        xs = [dev.to_device(rng.standard_normal(n_in).astype(np.float32)) for _ in range(2)]
        nan = np.full(n_out, np.nan, np.float32)
        ys = [dev.to_device(nan) for _ in range(2)]
        refs = [dev.to_device(nan) for _ in range(2)]
        bufs = xs + ys + refs
        for x, r in zip(xs, refs):
            dev.gemv_dev(w, x.ptr, r.ptr, n_out)
        dev.synchronize()
        want = [r.to_host(np.float32, n_out).copy() for r in refs]
        sa_, sb = ss.create(), ss.create()
        for _ in range(8):
            dev.gemv_dev(w, xs[0].ptr, ys[0].ptr, n_out, sa_)
            dev.gemv_dev(w, xs[1].ptr, ys[1].ptr, n_out, sb)
        ss.sync(sa_)
        ss.sync(sb)
        for y, wb in zip(ys, want):
            assert np.array_equal(bits(y.to_host(np.float32, n_out)), bits(wb))
        # a stream used and destroyed, then calls on the others
        sc = ss.create()
        dev.gemv_dev(w, xs[0].ptr, ys[0].ptr, n_out, sc)
        ss.sync(sc)
        ss.destroy(sc)
        dev.gemv_dev(w, xs[1].ptr, ys[1].ptr, n_out, sa_)
        dev.gemv_dev(w, xs[0].ptr, ys[0].ptr, n_out, sb)
        ss.sync(sa_)
        ss.sync(sb)
        assert np.array_equal(bits(ys[1].to_host(np.float32, n_out)), bits(want[1]))
        assert np.array_equal(bits(ys[0].to_host(np.float32, n_out)), bits(want[0]))
    finally:
        ss.close()
        for b in bufs:
            b.free()
        w.free()


def test_gemm_workspaces_on_two_streams(dev):
    """The context's GEMM activation planes, partial sums and counters: two
    streams alternate K-sliced GEMM calls (M = 40) on two weights."""
    rng = np.random.default_rng(32)
    n_out, n_in, M = 3072, 5120, 40
    Ws = [synth.make_weights(sa.Q4_K, n_out, n_in, rng) for _ in range(2)]
    ws = [dev.upload(sa.Q4_K, n_out, n_in, W) for W in Ws]
    ss = _Streams()
    bufs = []
    try:
        Xs = [dev.to_device(rng.standard_normal((M, n_in)).astype(np.float32)) for _ in range(2)]
        nan = np.full(M * n_out, np.nan, np.float32)
        Ys = [dev.to_device(nan) for _ in range(2)]
        refs = [dev.to_device(nan) for _ in range(2)]
        bufs = Xs + Ys + refs
        for w, X, r in zip(ws, Xs, refs):
            dev.gemm_dev(w, X.ptr, M, r.ptr)
        dev.synchronize()
        want = [r.to_host(np.float32, M * n_out).copy() for r in refs]
        streams = [ss.create(), ss.create()]
        for _ in range(6):
            for w, X, Y, s in zip(ws, Xs, Ys, streams):
                dev.gemm_dev(w, X.ptr, M, Y.ptr, s)
        for s in streams:
            ss.sync(s)
        for Y, wb in zip(Ys, want):
            assert np.array_equal(bits(Y.to_host(np.float32, M * n_out)), bits(wb))
    finally:
        ss.close()
        for b in bufs:
            b.free()
        for w in ws:
            w.free()
