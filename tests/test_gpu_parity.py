"""GPU parity: the HIP path through the C-ABI against the oracle (and, for
the matvec, the host emulation of the same kernel code).

Bars: activation quantizers bit-exact (quants, d, bsums); every dot within
|gpu - ref| <= 1e-5 * sum|terms| + 1e-6 (sum|terms| from the oracle), and
bit-identical to the host emulation for the integer formats.
"""
import os

import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth

pytestmark = pytest.mark.gpu

KQ = (sa.Q2_K, sa.Q3_K, sa.Q4_K, sa.Q5_K, sa.Q6_K)
TOL_REL, TOL_ABS = 1e-5, 1e-6


def edge_vectors(rng, n):
    """Activation rows exercising the quantizers' edge cases."""
    out = []
    out.append(rng.standard_normal(n).astype(np.float32))
    out.append((rng.standard_normal(n) * 1e-3).astype(np.float32))
    out.append((rng.standard_normal(n) * 1e4).astype(np.float32))
    z = rng.standard_normal(n).astype(np.float32)
    z[:256] = 0.0
    z[256:288] = -0.0
    out.append(z)
    t = np.round(rng.standard_normal(n) * 3).astype(np.float32)  # many |x| ties
    out.append(t)
    s = (rng.standard_normal(n) * 1e-38).astype(np.float32)  # subnormal range
    out.append(s)
    h = rng.uniform(-1, 1, n).astype(np.float32)
    h[5] = 7.0
    h[9] = -7.0  # tie of |max|: the first (positive) occurrence sets the sign
    out.append(h)
    g = rng.uniform(-1, 1, n).astype(np.float32)
    g[3] = -9.0
    g[200] = 9.0
    out.append(g)
    return out


def assert_close(y, ref, l1, what):
    err = np.abs(y.astype(np.float64) - ref)
    bound = TOL_REL * l1 + TOL_ABS
    bad = np.nonzero(~(err <= bound))[0]  # NaN fails
    assert bad.size == 0, (f"{what}: {bad.size} outputs out of tolerance, first row {bad[0]}: "
                           f"gpu {y[bad[0]]} ref {ref[bad[0]]} l1 {l1[bad[0]]}")


@pytest.mark.parametrize("n", [256, 1024, 4096, 14336])
def test_quantize_q8_K_bitexact(dev, oracle, n):
    rng = np.random.default_rng(100 + n)
    for x in edge_vectors(rng, n):
        got = dev.quantize(sa.Q8_K, x)
        want = oracle.quantize(sa.Q8_K, x)
        assert np.array_equal(got, want), f"Q8_K mismatch n={n}"


@pytest.mark.parametrize("n", [32, 896, 4096, 5120])
def test_quantize_q8_0_bitexact(dev, oracle, n):
    rng = np.random.default_rng(200 + n)
    vecs = edge_vectors(rng, max(n, 512))
    for x in vecs:
        x = x[:n].copy()
        got = dev.quantize(sa.Q8_0, x)
        want = oracle.quantize(sa.Q8_0, x)
        assert np.array_equal(got, want), f"Q8_0 mismatch n={n}"


def test_convert_f16_bitexact(dev, oracle):
    rng = np.random.default_rng(7)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 100,
                        (rng.standard_normal(4096) * 1e-6).astype(np.float32),
                        (rng.standard_normal(1024) * 1e-8).astype(np.float32),
                        np.array([65504, 65519.99, 65520, 1e10, -1e10, 6e-8, 2.98e-8,
                                  5.96e-8, 0.0, -0.0, np.inf, -np.inf], np.float32)])
    got = dev.quantize(sa.F16, x).view(np.uint16)
    want = oracle.quantize(sa.F16, x).view(np.uint16)
    assert np.array_equal(got, want)


def shapes_for(wt):
    if wt in KQ:
        return [(1, 256), (37, 1024), (64, 2048), (130, 768), (8, 5120), (3, 1792)]
    return [(1, 32), (37, 1024), (64, 2048), (130, 896), (5, 160)]


def tile_cols_for(wt):
    return [1, 2, 4, 8, 16, 32, 64]


@pytest.mark.parametrize("wt", sa.WEIGHT_TYPES, ids=lambda t: sa.NAMES[t])
def test_gemv_pair_vs_emulator_and_oracle(dev, oracle, emu, wt, option):
    rng = np.random.default_rng(wt)
    for (n_out, n_in) in shapes_for(wt):
        W = synth.make_weights(wt, n_out, n_in, rng)
        x = rng.standard_normal(n_in).astype(np.float32)
        xq = oracle.quantize(sa.PAIR[wt], x)
        ref = np.zeros(n_out)
        l1 = np.zeros(n_out)
        for r in range(n_out):
            ref[r], l1[r] = oracle.vec_dot(wt, n_in, W[r], xq)
        for G in tile_cols_for(wt):
            # every power-of-two tile width, also those that leave padding
            # columns in the last round of a tile
            option("TILE_COLS", str(G))
            y = dev.gemv_pair(wt, n_out, n_in, W, xq)
            assert_close(y, ref, l1, f"{sa.NAMES[wt]} {n_out}x{n_in} G={G}")
            if wt != sa.F16:
                ye = emu.gemv_pair(wt, n_out, n_in, G, W, xq)
                assert np.array_equal(y.view(np.uint32), ye.view(np.uint32)), \
                    f"{sa.NAMES[wt]} {n_out}x{n_in} G={G}: GPU differs from emulation"


@pytest.mark.parametrize("wt", sa.WEIGHT_TYPES, ids=lambda t: sa.NAMES[t])
def test_gemv_f32_vs_oracle(dev, oracle, wt):
    """Full path: f32 activation -> in-kernel quantization -> matvec."""
    rng = np.random.default_rng(1000 + wt)
    n_out, n_in = (300, 2048)
    W = synth.make_weights(wt, n_out, n_in, rng)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        for x in edge_vectors(rng, n_in)[:5]:
            y = dev.gemv(w, x)
            ref, l1 = oracle.gemv(wt, W, n_out, n_in, x)
            assert_close(y, ref.astype(np.float64), l1, f"{sa.NAMES[wt]} gemv")
        # n_out smaller than the uploaded rows (reference gemv takes n_out)
        x = rng.standard_normal(n_in).astype(np.float32)
        y = dev.gemv(w, x, n_out=77)
        ref, l1 = oracle.gemv(wt, W[:77], 77, n_in, x)
        assert_close(y, ref.astype(np.float64), l1, f"{sa.NAMES[wt]} gemv n_out=77")
    finally:
        w.free()


@pytest.mark.parametrize("wt", [sa.Q8_0, sa.Q5_0, sa.Q4_0, sa.F16], ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("n_in", [32, 896, 2048, 5120, 9216])
def test_gemv_prologue_bitexact(dev, oracle, option, wt, n_in):
    """The matvec's own conversion of an f32 activation (Q8_0: a quad of
    lanes per block, passes of 64 blocks loaded four at a time; F16: groups
    of 8 float4 per thread) stages the same LDS image as the oracle's
    converted activation: gemv from f32 is bit for bit gemv_pair on
    oracle.quantize(x) with the same tile width, on the edge vectors and on
    blocks holding inf and NaN."""
    rng = np.random.default_rng(4100 + wt * 7 + n_in)
    n_out = 96
    W = synth.make_weights(wt, n_out, n_in, rng)
    vecs = edge_vectors(rng, max(n_in, 512))
    v = rng.standard_normal(n_in).astype(np.float32)
    v[min(40, n_in - 1)] = np.inf
    v[n_in - 3] = np.nan
    vecs.append(v)
    # rows of 9216 also unsliced: 288 blocks, two groups of four Q8_0 passes
    # or of eight float4 per thread
    for G, split in [(4, -1), (16, -1)] + ([(16, 0)] if n_in == 9216 else []):
        option("TILE_COLS", str(G))
        option("SPLIT_ELEMS", split)
        w = dev.upload(wt, n_out, n_in, W)
        try:
            for i, x in enumerate(vecs):
                x = x[:n_in].copy()
                y = dev.gemv(w, x)
                yp = dev.gemv_pair(wt, n_out, n_in, W, oracle.quantize(sa.PAIR[wt], x))
                assert np.array_equal(y.view(np.uint32), yp.view(np.uint32)), \
                    f"{sa.NAMES[wt]} n_in={n_in} G={G} split={split} vector {i}"
        finally:
            w.free()


@pytest.mark.parametrize("wt", [sa.Q4_K, sa.Q5_K, sa.Q2_K, sa.Q3_K, sa.Q6_K, sa.Q8_0, sa.Q5_0, sa.Q4_0,
                                sa.F16, sa.F32], ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("M", [1, 3, 8, 13])
def test_gemm_small_M_vs_oracle(dev, oracle, wt, M):
    rng = np.random.default_rng(2000 + wt * 31 + M)
    n_out, n_in = 200, 1024
    W = synth.make_weights(wt, n_out, n_in, rng)
    X = rng.standard_normal((M, n_in)).astype(np.float32)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                 f"{sa.NAMES[wt]} gemm M={M}")


def test_errors_leave_outputs_untouched(dev):
    rng = np.random.default_rng(5)
    W = synth.make_weights(sa.Q4_K, 16, 256, rng)
    with pytest.raises(sa.SihipError):
        dev.upload(sa.Q4_K, 16, 256, W[:, :100])  # wrong byte count
    with pytest.raises(sa.SihipError):
        dev.upload(99, 16, 256, W)  # unsupported type
    w = dev.upload(sa.Q4_K, 16, 256, W)
    try:
        with pytest.raises(sa.SihipError):
            dev.gemv(w, np.zeros(256, np.float32), n_out=17)  # more rows than uploaded
    finally:
        w.free()


@pytest.mark.parametrize("combo", [
    (sa.Q4_K, sa.Q4_K, sa.Q6_K),        # Q4_K_M attention q, k, v: one mixed launch
    (sa.Q4_K, sa.Q4_K),                 # ffn gate + up
    (sa.Q8_0, sa.Q5_0, sa.Q4_0),        # no mixed kernel: one launch per matrix
    (sa.Q5_K, sa.Q6_K, sa.Q5_K, sa.Q6_K),
], ids=lambda c: "+".join(sa.NAMES[t] for t in c))
def test_gemv_multi_matches_single_and_oracle(dev, oracle, combo):
    """Several matrices sharing one activation in one call give bit-identical
    results to one gemv per matrix (row tiles and their reduction order do
    not depend on how workgroups are shared out), and match the oracle."""
    rng = np.random.default_rng(77 + len(combo))
    n_in = 2048
    shapes = [(wt, int(n)) for wt, n in zip(combo, rng.integers(100, 1500, len(combo)))]
    Ws = [synth.make_weights(wt, n, n_in, rng) for wt, n in shapes]
    ws = [dev.upload(wt, n, n_in, W) for (wt, n), W in zip(shapes, Ws)]
    bufs = []
    try:
        x = rng.standard_normal(n_in).astype(np.float32)
        xd = dev.to_device(x)
        nan = lambda n: np.full(n, np.nan, np.float32)  # noqa: E731
        ys = [dev.to_device(nan(n)) for _, n in shapes]
        singles = [dev.to_device(nan(n)) for _, n in shapes]
        bufs = [xd, *ys, *singles]
        dev.gemv_multi_dev(ws, xd.ptr, [y.ptr for y in ys])
        for w, y, (_, n) in zip(ws, singles, shapes):
            dev.gemv_dev(w, xd.ptr, y.ptr, n)
        dev.synchronize()
        for (wt, n), W, y, y1 in zip(shapes, Ws, ys, singles):
            a, b = y.to_host(np.float32, n), y1.to_host(np.float32, n)
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), sa.NAMES[wt]
            ref, l1 = oracle.gemv(wt, W, n, n_in, x)
            assert_close(a, ref.astype(np.float64), l1, f"multi {sa.NAMES[wt]} {n}x{n_in}")
    finally:
        for b in bufs:
            b.free()
        for w in ws:
            w.free()


@pytest.mark.parametrize("wt", sa.WEIGHT_TYPES, ids=lambda t: sa.NAMES[t])
def test_dequant_rows_bitexact(dev, oracle, option, wt):
    """row_to_f32 from the device copy: bit-identical to the reference
    dequantizer, for one row at a time (host pointer) and for a range of rows
    into device memory, at a narrow and a wide tile (padding included)."""
    rng = np.random.default_rng(3000 + wt)
    n_out, n_in = (37, 1792) if wt in KQ else (37, 1120)
    W = synth.make_weights(wt, n_out, n_in, rng)
    ref = np.stack([oracle.dequant(wt, W[r], n_in) for r in range(n_out)])
    for G in (1, 16):
        option("TILE_COLS", str(G))
        w = dev.upload(wt, n_out, n_in, W)
        buf = dev.alloc(n_out * n_in * 4)
        try:
            for r in (0, 17, n_out - 1):
                got = dev.dequant_row(w, r)
                assert np.array_equal(got.view(np.uint32), ref[r].view(np.uint32)), (sa.NAMES[wt], G, r)
            dev.dequant_rows_dev(w, 3, n_out - 3, buf.ptr, n_in)
            dev.synchronize()
            got = buf.to_host(np.float32, (n_out - 3) * n_in).reshape(n_out - 3, n_in)
            assert np.array_equal(got.view(np.uint32), ref[3:].view(np.uint32)), (sa.NAMES[wt], G)
            with pytest.raises(sa.SihipError):
                dev.dequant_row(w, n_out)  # past the last row
        finally:
            buf.free()
            w.free()


@pytest.mark.parametrize("wt,n_out,n_in,G", [
    (sa.Q8_0, 4864, 896, 8),      # narrowest tile with <= 6 rounds: 608 row tiles
    (sa.Q5_0, 5120, 5120, 32),    # 5 rounds, 2560 row tiles
    (sa.F16, 1024, 5120, 32),     # 5 rounds, 512 row tiles
    (sa.Q4_0, 5632, 2048, 16),    # 4 rounds, 1408 row tiles
    (sa.Q8_0, 896, 896, 32),      # 8 wide would give 112 row tiles: the tile-count rule
    (sa.Q5_0, 27648, 5120, 16),   # 32 wide would give 13824 row tiles: the tile-count rule
    (sa.Q4_K, 4096, 4096, 16),    # K-quants keep the tile-count rule
])
def test_tile_width_rule(dev, wt, n_out, n_in, G):
    """The batch-1 tile width chosen at upload for unit-column formats: the
    narrowest tile with at most 6 rounds per lane where that gives 512-4096
    row tiles, the tile-count rule otherwise."""
    rng = np.random.default_rng(n_out + n_in)
    w = dev.upload(wt, n_out, n_in, synth.make_weights(wt, n_out, n_in, rng))
    try:
        assert w.tile_cols == G, (sa.NAMES[wt], n_out, n_in, w.tile_cols)
    finally:
        w.free()
