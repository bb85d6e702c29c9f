"""sihip_gemm_multi_dev: the GEMMs of several weights that share one X (the
q/k/v and gate/up matrices of the batched forward), the activation
quantized once per record layout, and from M = 384 the Q4_K weights in one
launch of the 16x16 kernel (their n blocks one after another in one grid,
planned together). Every output is checked against the oracle to the
path's bar; a weight whose plan is its single-call plan must also give the
bits of sihip_gemm_dev (same kernels, same planes), while a weight given
its group's m-tile count, or planned with its group, may slice K
differently (same bar)."""
import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth

from .test_gpu_gemm import _rows
from .test_gpu_parity import assert_close
from .test_gpu_slices import _HipGraph, bits

pytestmark = pytest.mark.gpu


def _run(dev, ws, X, multi=True):
    """Outputs of one multi call (or of one gemm_dev call per weight)."""
    M = X.shape[0]
    xd = dev.to_device(X)
    ys = [dev.to_device(np.full(M * w.n_out, np.nan, np.float32)) for w in ws]
    try:
        if multi:
            dev.gemm_multi_dev(ws, xd.ptr, M, [y.ptr for y in ys])
        else:
            for w, y in zip(ws, ys):
                dev.gemm_dev(w, xd.ptr, M, y.ptr)
        dev.synchronize()
        return [y.to_host(np.float32, M * w.n_out).reshape(M, w.n_out) for w, y in zip(ws, ys)]
    finally:
        for b in [xd] + ys:
            b.free()


# (label, [(type, n_out)], n_in, M, indices whose plan stays the single-call
# plan): the Llama-3-8B Q4_K_M q/k/v group on the 16x16 kernels (wq and wv
# in 64-row blocks; wk, 32-row blocks on its own, joins them),
# a gate/up pair at a batch size on the 32-row kernel, a group of four
# record layouts (Q5_0, Q8_0, F16, Q4_K), a batch below every
# matrix-core threshold (the matvec kernel per weight), and a Q8_0-pair
# launch that quantizes X itself ahead of one that needs the planes
GROUPS = [
    ("qkv-q4km-M512", [(sa.Q4_K, 4096), (sa.Q4_K, 1024), (sa.Q6_K, 1024)], 4096, 512, (2,)),
    ("gate-up-q4k-M512", [(sa.Q4_K, 2816), (sa.Q4_K, 2816)], 1024, 512, ()),
    # two Q4_K segments with K slices (the second's partial sums at column
    # 128 x 3 of the shared rows) and a row count inside its last block
    ("q4k-sliced-M384", [(sa.Q4_K, 300), (sa.Q6_K, 128), (sa.Q4_K, 200)], 2048, 384, ()),
    ("gate-up-q4k-M8", [(sa.Q4_K, 2048), (sa.Q4_K, 2048)], 2048, 8, (0, 1)),
    ("mixed-M40", [(sa.Q5_0, 640), (sa.Q8_0, 384), (sa.F16, 512), (sa.Q4_K, 300)], 2048, 40, ()),
    ("matvec-M2", [(sa.Q4_K, 700), (sa.Q6_K, 300), (sa.Q5_0, 260)], 1024, 2, (0, 1, 2)),
    # one record layout, a launch that quantizes X itself (640 rows: K
    # slices of 6 steps in LDS) before one that reads the shared planes
    # (13312 rows: slices of 32 steps, past the LDS image)
    ("q50-fused-then-ring-M5", [(sa.Q5_0, 640), (sa.Q5_0, 13312)], 16384, 5, (0, 1)),
]


@pytest.mark.parametrize("label,mats,n_in,M,same", GROUPS, ids=[g[0] for g in GROUPS])
def test_gemm_multi_vs_oracle(dev, oracle, label, mats, n_in, M, same):
    print(f"gemm_multi {label}", flush=True)
    rng = np.random.default_rng(len(label) * 1000 + M)
    Ws = [synth.make_weights(wt, n_out, n_in, rng) for wt, n_out in mats]
    ws = [dev.upload(wt, n_out, n_in, W) for (wt, n_out), W in zip(mats, Ws)]
    try:
        X = _rows(rng, M, n_in)
        Ys = _run(dev, ws, X)
        Ysingle = _run(dev, ws, X, multi=False)
        for i, ((wt, n_out), W, Y) in enumerate(zip(mats, Ws, Ys)):
            ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
            assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                         f"{label} weight {i} ({sa.NAMES[wt]} {n_out}x{n_in})")
            if i in same:
                assert np.array_equal(bits(Y), bits(Ysingle[i])), \
                    f"{label} weight {i}: differs from sihip_gemm_dev"
        # a second call on the same planes' buffers: nothing stale carries over
        X2 = _rows(rng, M, n_in)[::-1].copy()
        Ys2 = _run(dev, ws, X2)
        for i, ((wt, n_out), W, Y) in enumerate(zip(mats, Ws, Ys2)):
            ref, L1 = oracle.gemm(wt, W, n_out, n_in, X2)
            assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                         f"{label} second call, weight {i}")
    finally:
        for w in ws:
            w.free()


def test_gemm_multi_graph_replays(dev):
    """Captured after an eager call (GEMM copies and workspaces exist), the
    multi call replays to the bits of the eager call, with eager work of
    another shape on the shared planes between the replays."""
    rng = np.random.default_rng(77)
    n_in, M = 4096, 512
    mats = [(sa.Q4_K, 512), (sa.Q4_K, 256), (sa.Q6_K, 256)]
    ws = [dev.upload(wt, n, n_in, synth.make_weights(wt, n, n_in, rng)) for wt, n in mats]
    other = dev.upload(sa.Q5_0, 384, n_in, synth.make_weights(sa.Q5_0, 384, n_in, rng))
    xd = dev.to_device(rng.standard_normal((M, n_in)).astype(np.float32))
    nans = [np.full(M * w.n_out, np.nan, np.float32) for w in ws]
    ye = [dev.to_device(n) for n in nans]
    yg = [dev.to_device(n) for n in nans]
    yo = dev.to_device(np.full(64 * 384, np.nan, np.float32))
    hg = _HipGraph()
    try:
        dev.gemm_multi_dev(ws, xd.ptr, M, [y.ptr for y in ye], hg.stream.value)
        dev.synchronize()
        want = [y.to_host(np.float32, M * w.n_out).copy() for w, y in zip(ws, ye)]
        hg.begin()
        dev.gemm_multi_dev(ws, xd.ptr, M, [y.ptr for y in yg], hg.stream.value)
        hg.end()
        for _ in range(3):
            for y, n in zip(yg, nans):
                y.fill(n)
            hg.replay()
            for w, y, wb in zip(ws, yg, want):
                assert np.array_equal(bits(y.to_host(np.float32, M * w.n_out)), bits(wb))
            dev.gemm_dev(other, xd.ptr, 64, yo.ptr, hg.stream.value)  # other use of the planes
            dev.synchronize()
    finally:
        hg.close()
        for b in [xd, yo] + ye + yg:
            b.free()
        for w in ws + [other]:
            w.free()


def test_gemm_multi_refuses_bad_groups(dev):
    rng = np.random.default_rng(5)
    a = dev.upload(sa.Q4_K, 256, 1024, synth.make_weights(sa.Q4_K, 256, 1024, rng))
    b = dev.upload(sa.Q4_K, 256, 2048, synth.make_weights(sa.Q4_K, 256, 2048, rng))
    xd = dev.to_device(np.zeros(8 * 2048, np.float32))
    ys = [dev.to_device(np.zeros(8 * 256, np.float32)) for _ in range(5)]
    try:
        with pytest.raises(sa.SihipError, match="n_in differs"):
            dev.gemm_multi_dev([a, b], xd.ptr, 8, [ys[0].ptr, ys[1].ptr])
        with pytest.raises(sa.SihipError, match="bad arguments"):
            dev.gemm_multi_dev([a] * 5, xd.ptr, 8, [y.ptr for y in ys])
        with pytest.raises(sa.SihipError, match="M must be positive"):
            dev.gemm_multi_dev([a], xd.ptr, 0, [ys[0].ptr])
    finally:
        for buf in [xd] + ys:
            buf.free()
        a.free()
        b.free()


def test_gemm_multi_q4k_group_vs_separate(dev, oracle, option):
    """The grouped Q4_K launch against the same weights launched one by one
    (GEMM_GROUP = 0): both within the bar of the oracle, and the group's
    results do not depend on the order of its weights."""
    rng = np.random.default_rng(9100)
    n_in, M = 2048, 512
    mats = [(sa.Q4_K, 1536), (sa.Q4_K, 384), (sa.Q4_K, 130)]
    Ws = [synth.make_weights(wt, n, n_in, rng) for wt, n in mats]
    ws = [dev.upload(wt, n, n_in, W) for (wt, n), W in zip(mats, Ws)]
    try:
        X = _rows(rng, M, n_in)
        grouped = _run(dev, ws, X)
        rev = _run(dev, ws[::-1], X)[::-1]
        option("GEMM_GROUP", 0)
        separate = _run(dev, ws, X)
        for i, ((wt, n_out), W) in enumerate(zip(mats, Ws)):
            ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
            for label, Y in (("grouped", grouped[i]), ("separate", separate[i])):
                assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                             f"{label} weight {i}")
            assert np.array_equal(bits(grouped[i]), bits(rev[i])), f"weight {i}: order matters"
    finally:
        for w in ws:
            w.free()
