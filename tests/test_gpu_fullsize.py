"""GPU parity at the benchmark's full shapes: every matrix of the Llama-3-8B
Q4_K_M layer set, configs 0 and 1 (Q4_K and Q4_0 at 5632 x 2048, the Q8_0 FFN
matrix and both heads), and config 4's 32B-class shapes (attn, kv, ffn_up,
ffn_down) for Q2_K, Q3_K, Q5_K, Q5_0 and F16.

Every output row is compared with the oracle, to the bar
|gpu - ref| <= 1e-5 * sum|terms| + 1e-6:
- batch 1 (gemv) for every shape;
- batch 8 (gemm, the matrix-core path for the K-quants) for every column,
  where the benchmark runs batch 8, and batch-1 calls on two of its columns.
On top of that, every row satisfies a property the arithmetic fixes exactly:
doubling the activation leaves its Q8_K / Q8_0 quants unchanged and doubles
the block scales (scaling by 2 commutes with every rounding step: the
divisions and products of the quantizers, f16 conversion and each FMA of
the dot), so gemv(W, 2x) must equal 2 * gemv(W, x) bit for bit.

The fused decode launches the benchmark times (q/k/v and gate/up, one launch
each over the device-pointer entry point, captured in a HIP graph) are
checked the same way at the 8B shapes.
"""
import zlib

import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth

from .test_gpu_slices import _HipGraph, bits

pytestmark = pytest.mark.gpu

TOL_REL, TOL_ABS = 1e-5, 1e-6


def _shapes():
    out = [(f"llama3-8b {n}", wt, o, i, (1,)) for (n, wt, o, i) in synth.LLAMA3_8B_LAYER]
    out += [("cfg0 Q4_K", sa.Q4_K, 5632, 2048, (1,)),
            ("cfg0 Q4_0", sa.Q4_0, 5632, 2048, (1, 8)),
            ("cfg1 Q8_0", sa.Q8_0, 4864, 896, (1,)),
            ("cfg1 Q6_K head", sa.Q6_K, 151936, 1024, (1,)),
            ("cfg1 Q8_0 head", sa.Q8_0, 151936, 896, (1,))]
    for wt in (sa.Q2_K, sa.Q3_K, sa.Q5_K, sa.Q5_0, sa.F16):
        nm = sa.NAMES[wt]
        out += [(f"cfg4 {nm} attn", wt, 5120, 5120, (1, 8)),
                (f"cfg4 {nm} kv", wt, 1024, 5120, (1, 8)),
                (f"cfg4 {nm} ffn_up", wt, 27648, 5120, (1, 8)),
                (f"cfg4 {nm} ffn_down", wt, 5120, 27648, (1, 8))]
    return out


SHAPES = _shapes()


def _close(y, ref, l1, what):
    y, ref, l1 = y.reshape(-1), ref.reshape(-1), l1.reshape(-1)
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    bad = np.nonzero(~(err <= TOL_REL * l1 + TOL_ABS))[0]
    assert bad.size == 0, (f"{what}: {bad.size} outputs out of tolerance, first {bad[0]}: "
                           f"gpu {y[bad[0]]} ref {ref[bad[0]]} l1 {l1[bad[0]]}")


@pytest.mark.parametrize("label,wt,n_out,n_in,batches", SHAPES, ids=[s[0] for s in SHAPES])
def test_full_shape(dev, oracle, label, wt, n_out, n_in, batches):
    rng = np.random.default_rng(zlib.crc32(label.encode()))
    W = synth.make_weights(wt, n_out, n_in, rng)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        x = rng.standard_normal(n_in).astype(np.float32)
        y = dev.gemv(w, x)
        ref, l1 = oracle.gemv(wt, W, n_out, n_in, x)
        _close(y, ref, l1, f"{label} batch 1, every row")
        y2 = dev.gemv(w, 2.0 * x)
        assert np.array_equal(y2.view(np.uint32), (2.0 * y).astype(np.float32).view(np.uint32)), \
            f"{label}: gemv(2x) != 2 gemv(x)"
        if 8 in batches:
            X = rng.standard_normal((8, n_in)).astype(np.float32)
            Y = dev.gemm(w, X)
            refm, l1m = oracle.gemm(wt, W, n_out, n_in, X)
            _close(Y, refm, l1m, f"{label} batch 8, every row and column")
            for m in (0, 7):
                # batches of the K-quants run on the matrix cores, whose f32
                # order differs from the matvec's, so the two GPU paths agree
                # to the bar, not bit for bit
                _close(dev.gemv(w, X[m]), refm[m], l1m[m], f"{label} batch 1 on column {m}")
    finally:
        w.free()


FUSED = [("qkv", ("wq", "wk", "wv")), ("gate_up", ("ffn_gate", "ffn_up"))]


@pytest.mark.parametrize("label,names", FUSED, ids=[f[0] for f in FUSED])
def test_fused_decode_launch_full_shape(dev, oracle, label, names):
    """The fused launch as the benchmark issues it: one sihip_gemv_multi_dev
    call on a non-default stream over a device-resident activation, captured
    in a HIP graph and replayed. Every row of every matrix matches the
    oracle; the replays reproduce the eager launch bit for bit, and so does
    one gemv per matrix (row tiles and their reduction order do not depend
    on how workgroups are shared out)."""
    shapes = {n: (wt, o, i) for (n, wt, o, i) in synth.LLAMA3_8B_LAYER}
    rng = np.random.default_rng(zlib.crc32(label.encode()))
    Ws = {n: synth.make_weights(*shapes[n], rng) for n in names}
    ws = [dev.upload(*shapes[n], Ws[n]) for n in names]
    hg = _HipGraph()
    bufs = []
    try:
        n_in = shapes[names[0]][2]
        x = rng.standard_normal(n_in).astype(np.float32)
        nan = {n: np.full(shapes[n][1], np.nan, np.float32) for n in names}
        xd = dev.to_device(x)
        ys = [dev.to_device(nan[n]) for n in names]
        singles = [dev.to_device(nan[n]) for n in names]
        bufs = [xd, *ys, *singles]
        sp = hg.stream.value
        dev.gemv_multi_dev(ws, xd.ptr, [y.ptr for y in ys], sp)
        for w, y in zip(ws, singles):
            dev.gemv_dev(w, xd.ptr, y.ptr, w.n_out, sp)
        dev.synchronize()
        eager = [y.to_host(np.float32, w.n_out).copy() for y, w in zip(ys, ws)]
        for n, a, s, w in zip(names, eager, singles, ws):
            assert np.array_equal(bits(a), bits(s.to_host(np.float32, w.n_out))), \
                f"{label}: fused {n} differs from its own gemv"
            ref, l1 = oracle.gemv(shapes[n][0], Ws[n], shapes[n][1], n_in, x)
            _close(a, ref, l1, f"{label} fused {n}, every row")
        hg.begin()
        dev.gemv_multi_dev(ws, xd.ptr, [y.ptr for y in ys], sp)
        hg.end()
        for rep in range(3):
            for n, y in zip(names, ys):
                y.fill(nan[n])
            hg.replay()
            for n, y, a, w in zip(names, ys, eager, ws):
                assert np.array_equal(bits(y.to_host(np.float32, w.n_out)), bits(a)), \
                    f"{label}: graph replay {rep} differs on {n}"
    finally:
        hg.close()
        for b in bufs:
            b.free()
        for w in ws:
            w.free()
