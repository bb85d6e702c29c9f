"""F32 weights on the device (reference pair F32, backend.c:102-103, dot
si_dot_f32, kernels.c:180-187): gemv, device-pointer gemv, batched rows,
separate launches of several F32 matrices, the per-row dot and row
dequantization, against the oracle to |gpu - ref| <= 1e-5 * sum|terms| +
1e-6. Rows whose length is a multiple of 4 take 16-byte loads; others the
scalar path."""
import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth

from .test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_out,n_in", [(300, 2048), (129, 1001), (1, 4), (4100, 512)])
def test_f32_gemv_gemm(dev, oracle, n_out, n_in):
    rng = np.random.default_rng(n_out + n_in)
    W = synth.make_weights(sa.F32, n_out, n_in, rng)
    w = dev.upload(sa.F32, n_out, n_in, W)
    try:
        x = rng.standard_normal(n_in).astype(np.float32)
        y = dev.gemv(w, x)
        ref, l1 = oracle.gemv(sa.F32, W, n_out, n_in, x)
        assert_close(y, ref, l1, f"F32 gemv {n_out}x{n_in}")
        y2 = dev.gemv(w, x, n_out=max(1, n_out // 2))
        assert np.array_equal(y2, y[:y2.size])
        for M in (3, 9):
            X = rng.standard_normal((M, n_in)).astype(np.float32)
            Y = dev.gemm(w, X)
            R, L1 = oracle.gemm(sa.F32, W, n_out, n_in, X)
            assert_close(Y.reshape(-1), R.reshape(-1), L1.reshape(-1), f"F32 gemm M={M}")
        row = dev.dequant_row(w, n_out - 1)
        assert np.array_equal(row, W[n_out - 1].view(np.float32))
        a = x.view(np.uint8)
        s = dev.vec_dot(sa.F32, n_in, W[0], a)
        d, m = oracle.vec_dot(sa.F32, n_in, W[0], a)
        assert abs(s - d) <= 1e-5 * m + 1e-6
    finally:
        w.free()


def test_f32_multi_and_device_pointers(dev, oracle):
    """Two F32 matrices sharing x in one gemv_multi_dev call (each its own
    launch) give the single-call results."""
    rng = np.random.default_rng(99)
    n_in = 768
    shapes = [(100, n_in), (37, n_in)]
    Ws = [synth.make_weights(sa.F32, o, i, rng) for o, i in shapes]
    ws = [dev.upload(sa.F32, o, i, W) for (o, i), W in zip(shapes, Ws)]
    x = rng.standard_normal(n_in).astype(np.float32)
    bufs = [dev.to_device(x)] + [dev.to_device(np.full(o, np.nan, np.float32)) for o, _ in shapes]
    try:
        dev.gemv_multi_dev(ws, bufs[0].ptr, [b.ptr for b in bufs[1:]])
        dev.synchronize()
        for (o, i), W, w, b in zip(shapes, Ws, ws, bufs[1:]):
            got = b.to_host(np.float32, o)
            assert np.array_equal(got, dev.gemv(w, x))
            ref, l1 = oracle.gemv(sa.F32, W, o, i, x)
            assert_close(got, ref, l1, f"F32 multi {o}x{i}")
    finally:
        for b in bufs:
            b.free()
        for w in ws:
            w.free()
