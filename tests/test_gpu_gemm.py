"""GPU parity of the prefill GEMM on the matrix cores (Q4_K, Q5_K, Q2_K, Q3_K
and Q6_K weights x Q8_K rows) against the oracle, to the same tolerance as the
matvec: |gpu - ref| <= 1e-5 * sum|terms| + 1e-6 per output."""
import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth

from .test_gpu_parity import assert_close, edge_vectors

pytestmark = pytest.mark.gpu


def _rows(rng, M, n_in):
    X = rng.standard_normal((M, n_in)).astype(np.float32)
    edges = edge_vectors(rng, n_in)
    for i in range(min(M, len(edges))):  # quantizer edge cases in the first rows
        X[i] = edges[i]
    return X


MFMA_TYPES = [sa.Q4_K, sa.Q5_K, sa.Q2_K, sa.Q3_K, sa.Q6_K, sa.F16, sa.Q4_0, sa.Q5_0, sa.Q8_0]


def _force_mfma(option):
    """The matrix-core path at every M (Q6_K, F16 and the Q8_0-pair formats
    have thresholds of their own)."""
    option("GEMM_MIN_M", "1")
    option("GEMM6_MIN_M", "1")
    option("GEMMH_MIN_M", "1")
    option("GEMMQ_MIN_M", "1")


def _extreme_q2k(W, n_out, n_in):
    """Q2_K rows 0 and 1 at the largest operand: every group scale and min
    15 and every quant 3 (sc * q = 45), one with d, dmin at their f16 maxima
    of the test range."""
    blk = W.reshape(n_out, n_in // 256, 84)
    blk[:2, :, 0:16] = 0xFF
    blk[:2, :, 16:80] = 0xFF
    return W


def _extreme_q3k(W, n_out, n_in):
    """Q3_K rows 0-3 at the ends of the operand range: 6-bit scales 0 and 63
    (sc = -32 and 31) against quants -4 and 3, so that -sc * q takes -128,
    96, 124 and -93 (the GEMM's bytes P - 128 at P = 0 and P = 248)."""
    blk = W.reshape(n_out, n_in // 256, 110)
    for row, (scale_byte, quant_byte) in enumerate([(0x00, 0x00), (0x00, 0xFF), (0xFF, 0x00), (0xFF, 0xFF)]):
        if row < n_out:
            blk[row, :, 96:108] = scale_byte
            blk[row, :, 0:96] = quant_byte  # high-mask bits and 2-bit quants
    return W


def _extreme_q6k(W, n_out, n_in):
    """Q6_K rows 0-3 at the ends of the digit operands: scales -128 and 127
    against quants 0 and 63, so v = (q - 32) * sc takes 4096, 3937, -3968 and
    -4064 (digits hi = 32, lo = 0 up to hi = -32, lo = 32)."""
    blk = W.reshape(n_out, n_in // 256, 210)
    for row, (scale_byte, quant_byte) in enumerate([(0x80, 0x00), (0x7F, 0xFF), (0x80, 0xFF),
                                                    (0x7F, 0x00)]):
        if row < n_out:
            blk[row, :, 0:192] = quant_byte  # ql and qh
            blk[row, :, 192:208] = scale_byte
    return W


def _extreme_q80(W, wt, n_out, n_in):
    """Rows at the ends of the Q4_0 / Q5_0 / Q8_0 quant ranges: every quant
    at its largest and at its smallest stored value (Q4_0 nibbles 15 and 0,
    Q5_0 fifth bits and nibbles all set and all clear, Q8_0 bytes 127 and
    -128), scales as drawn."""
    bb = {sa.Q4_0: 18, sa.Q5_0: 22, sa.Q8_0: 34}[wt]
    blk = W.reshape(n_out, n_in // 32, bb)
    for row, byte in enumerate([0xFF, 0x00] if wt != sa.Q8_0 else [0x7F, 0x80]):
        if row < n_out:
            blk[row, :, 2:] = byte
    return W


def _extreme_q5k(W, n_out, n_in):
    """Q5_K rows 0-1 with every 6-bit scale and min 63 (sh = sl = 7) and
    every quant 31 or 0: operand bytes sh * q - 128 = 89 and -128."""
    blk = W.reshape(n_out, n_in // 256, 176)
    for row, quant_byte in enumerate([0xFF, 0x00]):
        if row < n_out:
            blk[row, :, 4:16] = 0xFF
            blk[row, :, 16:176] = quant_byte  # fifth bits and nibbles
    return W


@pytest.mark.parametrize("wt", MFMA_TYPES, ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("n_out,n_in,M", [
    (200, 1024, 16), (333, 2048, 64), (1000, 256, 100), (130, 4096, 130), (64, 512, 1),
    (129, 768, 65),
])
def test_gemm_mfma_vs_oracle(dev, oracle, option, wt, n_out, n_in, M):
    _force_mfma(option)  # the MFMA path even for tiny M
    rng = np.random.default_rng(n_out * 7 + n_in + M + wt)
    W = synth.make_weights(wt, n_out, n_in, rng)
    if wt == sa.Q2_K:
        W = _extreme_q2k(W, n_out, n_in)
    if wt == sa.Q3_K:
        W = _extreme_q3k(W, n_out, n_in)
    if wt == sa.Q5_K:
        W = _extreme_q5k(W, n_out, n_in)
    if wt == sa.Q6_K:
        W = _extreme_q6k(W, n_out, n_in)
    if wt in (sa.Q4_0, sa.Q5_0, sa.Q8_0):
        W = _extreme_q80(W, wt, n_out, n_in)
    X = _rows(rng, M, n_in)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                 f"mfma gemm {sa.NAMES[wt]} {n_out}x{n_in} M={M}")


@pytest.mark.parametrize("wt", MFMA_TYPES, ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("G", [1, 4, 16, 64])
def test_gemm_mfma_every_tile_width(dev, oracle, option, wt, G):
    """The GEMM reads the matvec layout of any tile width."""
    _force_mfma(option)
    option("TILE_COLS", str(G))
    rng = np.random.default_rng(900 + G + wt)
    n_out, n_in, M = 300, 1792, 40
    W = synth.make_weights(wt, n_out, n_in, rng)
    X = _rows(rng, M, n_in)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        assert w.tile_cols == G
        Y = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                 f"mfma gemm {sa.NAMES[wt]} G={G}")


@pytest.mark.parametrize("M", [64, 128, 512, 2048])
def test_gemm_config3_full_size(dev, oracle, M):
    """Config 3 at full size (Q4_K 14336 x 4096) over its M sweep on the
    default dispatch. Up to M = 512 every output is checked against the
    oracle; above that, 160 weight rows spread over every workgroup tile for
    all M activation rows, and every weight row for four activation rows
    (first, last and two inside)."""
    rng = np.random.default_rng(3 + M)
    n_out, n_in = 14336, 4096
    W = synth.make_weights(sa.Q4_K, n_out, n_in, rng)
    X = rng.standard_normal((M, n_in)).astype(np.float32)
    w = dev.upload(sa.Q4_K, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
    finally:
        w.free()
    if M <= 512:
        ref, L1 = oracle.gemm(sa.Q4_K, W, n_out, n_in, X)
        assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                     f"config 3 M={M}, every output")
        return
    rows = np.unique(np.concatenate([rng.choice(n_out, 128, replace=False),
                                     np.arange(0, n_out, 509), [0, n_out - 1]]))
    ref, L1 = oracle.gemm(sa.Q4_K, W[rows], len(rows), n_in, X)
    assert_close(Y[:, rows].reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                 f"config 3 M={M} sampled rows")
    cols = np.array([0, 37, M // 2 + 5, M - 1])
    ref, L1 = oracle.gemm(sa.Q4_K, W, n_out, n_in, X[cols])
    assert_close(Y[cols].reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                 f"config 3 M={M} every row of activation rows {cols.tolist()}")


@pytest.mark.parametrize("wt", [sa.Q2_K, sa.Q3_K, sa.Q5_K], ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("n_out,n_in,M", [(27648, 5120, 8), (5120, 27648, 8), (5120, 5120, 512)])
def test_gemm_config4_sampled_rows(dev, oracle, wt, n_out, n_in, M):
    """Config 4's Q2_K, Q3_K and Q5_K matrices at batch 8 (ffn_up, ffn_down) and
    the attention matrix at M = 512 on the default dispatch; about 96 weight
    rows spread over every workgroup tile are checked for every activation
    row."""
    rng = np.random.default_rng(n_out + n_in + M + wt)
    W = synth.make_weights(wt, n_out, n_in, rng)
    X = rng.standard_normal((M, n_in)).astype(np.float32)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
    finally:
        w.free()
    rows = np.unique(np.concatenate([rng.choice(n_out, 64, replace=False),
                                     np.arange(0, n_out, 997), [0, n_out - 1]]))
    ref, L1 = oracle.gemm(wt, W[rows], len(rows), n_in, X)
    assert_close(Y[:, rows].reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                 f"{sa.NAMES[wt]} {n_out}x{n_in} M={M} sampled rows")


@pytest.mark.parametrize("wt", MFMA_TYPES, ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("mt,sbk", [(1, 1), (1, 3), (1, 4), (1, 0), (2, 3), (2, 0)])
def test_gemm_k_slices(dev, oracle, option, wt, mt, sbk):
    """K slices of the small-M GEMM (11 super-blocks: ragged last slice,
    several m tiles, a ragged last n tile): every slicing and tile height
    within tolerance of the oracle, and a repeated call gives the same bits
    (the last slice of each tile resets its arrival counter)."""
    _force_mfma(option)
    option("GEMM_MT", str(mt))
    option("GEMM_SBK", str(sbk))
    rng = np.random.default_rng(1100 + 10 * mt + sbk + 1000 * wt)
    n_out, n_in, M = 333, 2816, 70
    W = synth.make_weights(wt, n_out, n_in, rng)
    X = _rows(rng, M, n_in)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
        Y2 = dev.gemm(w, X)
        Y3 = dev.gemm(w, X[:5])
    finally:
        w.free()
    ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
    what = f"gemm {sa.NAMES[wt]} MT={mt} SBK={sbk}"
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1), what)
    assert np.array_equal(Y.view(np.uint32), Y2.view(np.uint32)), what + ": repeat differs"
    assert_close(Y3.reshape(-1), ref[:5].reshape(-1).astype(np.float64), L1[:5].reshape(-1),
                 what + " M=5")


def test_prepare_gemm_matches_lazy_copy(dev, oracle):
    """sihip_weight_prepare_gemm builds the GEMM copies at once (device bytes
    grow by them, a second call adds nothing; Q4_K has two, one per GEMM
    kernel, and a lazy call builds only the one it uses; Q6_K and Q8_0 have
    one); a later gemm gives the bits of a weight whose copy its first gemm
    built. F32, with no matrix-core GEMM: a no-op."""
    rng = np.random.default_rng(4242)
    n_out, n_in, M = 700, 2048, 40
    W = synth.make_weights(sa.Q4_K, n_out, n_in, rng)
    X = _rows(rng, M, n_in)
    eager, lazy = dev.upload(sa.Q4_K, n_out, n_in, W), dev.upload(sa.Q4_K, n_out, n_in, W)
    W6 = synth.make_weights(sa.Q6_K, 64, 512, rng)
    w6 = dev.upload(sa.Q6_K, 64, 512, W6)
    W8 = synth.make_weights(sa.Q8_0, 64, 512, rng)
    w8 = dev.upload(sa.Q8_0, 64, 512, W8)
    W32 = synth.make_weights(sa.F32, 64, 512, rng)
    w32 = dev.upload(sa.F32, 64, 512, W32)
    try:
        before = eager.device_bytes
        eager.prepare_gemm()
        grown = eager.device_bytes
        assert grown > before
        eager.prepare_gemm()
        assert eager.device_bytes == grown
        Ye, Yl = dev.gemm(eager, X), dev.gemm(lazy, X)
        assert before < lazy.device_bytes < grown
        assert np.array_equal(Ye.view(np.uint32), Yl.view(np.uint32))
        ref, L1 = oracle.gemm(sa.Q4_K, W, n_out, n_in, X)
        assert_close(Ye.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                     f"prepared gemm {n_out}x{n_in} M={M}")
        b6 = w6.device_bytes
        w6.prepare_gemm()
        assert w6.device_bytes > b6
        b8 = w8.device_bytes
        w8.prepare_gemm()
        assert w8.device_bytes > b8
        b32 = w32.device_bytes
        w32.prepare_gemm()
        assert w32.device_bytes == b32
    finally:
        for w in (eager, lazy, w6, w8, w32):
            w.free()


def _extreme_q4k(W, n_out, n_in, huge_dmin):
    """Q4_K rows at the ends of the 16x16 GEMM's operand ranges: row 0 with
    every 6-bit scale and min 63 and every quant 15 (sh * q = sl * q = 105),
    row 1 with d = 0, row 2 with dmin = 0 and, when huge_dmin, row 3 with
    dmin = 1000 (which lowers the tensor's min-operand exponent E below 0)."""
    blk = W.reshape(n_out, n_in // 256, 144)
    blk[0, :, 4:144] = 0xFF
    if n_out > 1:
        blk[1, :, 0:2] = 0
    if n_out > 2:
        blk[2, :, 2:4] = 0
    if n_out > 3 and huge_dmin:
        blk[3, :, 2:4] = np.frombuffer(np.float16(1000.0).tobytes(), np.uint8)
    return W


@pytest.mark.parametrize("n_out,n_in,M,mt,huge,sbk", [
    (200, 1024, 16, 8, False, -1), (333, 2048, 130, 8, True, -1), (1000, 256, 100, 4, False, -1),
    (129, 768, 65, 2, True, -1), (130, 4096, 257, 8, False, -1), (4096, 1280, 384, 8, True, -1),
    (4096, 1280, 384, 8, False, 0), (333, 2816, 130, 4, True, 3), (1024, 4096, 512, 8, False, -1),
])
def test_gemm2_q4k_vs_oracle(dev, oracle, option, n_out, n_in, M, mt, huge, sbk):
    """The 16x16 Q4_K GEMM (gemm2.h) forced at every M, m-tile count 2, 4
    and 8, with K slices as planned, none, and 3 super-blocks per slice
    (ragged last slice), ragged M and n_out, one super-block per row, and
    rows at the ends of its operand ranges, against the oracle."""
    option("GEMM2_MIN_M", "1")
    option("GEMM_MT", str(mt))
    option("GEMM_SBK", str(sbk))
    rng = np.random.default_rng(n_out + 3 * n_in + M + mt)
    W = _extreme_q4k(synth.make_weights(sa.Q4_K, n_out, n_in, rng), n_out, n_in, huge)
    X = _rows(rng, M, n_in)
    w = dev.upload(sa.Q4_K, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
        Y2 = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(sa.Q4_K, W, n_out, n_in, X)
    what = f"gemm2 Q4_K {n_out}x{n_in} M={M} MT={mt} SBK={sbk}"
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1), what)
    assert np.array_equal(Y.view(np.uint32), Y2.view(np.uint32)), what + ": repeat differs"


@pytest.mark.parametrize("n_out,n_in,M", [(4096, 14336, 512), (1024, 4096, 512), (4096, 14336, 8),
                                          (1024, 4096, 8), (4096, 14336, 64)])
def test_gemm6_q6k_bench_shapes(dev, oracle, option, n_out, n_in, M):
    """The Q6_K GEMM (gemm6.h) at the 8B layer's Q6_K shapes (ffn_down and
    wv), M = 512, 64 and 8 (below its default threshold, forced): every
    output against the oracle, and a repeat gives the same bits (K slices
    reset their counters)."""
    option("GEMM6_MIN_M", "1")
    rng = np.random.default_rng(n_out + n_in + M)
    W = _extreme_q6k(synth.make_weights(sa.Q6_K, n_out, n_in, rng), n_out, n_in)
    X = _rows(rng, M, n_in)
    w = dev.upload(sa.Q6_K, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
        Y2 = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(sa.Q6_K, W, n_out, n_in, X)
    what = f"gemm6 Q6_K {n_out}x{n_in} M={M}"
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1), what)
    assert np.array_equal(Y.view(np.uint32), Y2.view(np.uint32)), what + ": repeat differs"


@pytest.mark.parametrize("n_out,n_in,M,mt,sbk", [
    (333, 2816, 70, 4, -1), (4096, 1280, 384, 4, -1), (129, 768, 65, 2, 0),
    (200, 1024, 16, 1, 1), (1000, 512, 130, 4, 0), (130, 4096, 257, 4, 3), (300, 3072, 40, 2, 5),
])
def test_gemm6_q6k_tiles(dev, oracle, option, n_out, n_in, M, mt, sbk):
    """The Q6_K GEMM at every m-tile count (1, 2, 4), with and without K
    slices (ragged last slice), ragged M and n_out, rows at the ends of its
    operand range."""
    option("GEMM6_MIN_M", "1")
    option("GEMM_MT", str(mt))
    option("GEMM_SBK", str(sbk))
    rng = np.random.default_rng(7 * n_out + n_in + M + mt)
    W = _extreme_q6k(synth.make_weights(sa.Q6_K, n_out, n_in, rng), n_out, n_in)
    X = _rows(rng, M, n_in)
    w = dev.upload(sa.Q6_K, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(sa.Q6_K, W, n_out, n_in, X)
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                 f"gemm6 Q6_K {n_out}x{n_in} M={M} MT={mt} SBK={sbk}")


@pytest.mark.parametrize("n_out,n_in,M,mt,sbk", [
    (27648, 5120, 8, -1, -1), (5120, 27648, 8, -1, -1), (300, 1280, 70, 4, 0), (129, 384, 33, 2, 1),
    (1000, 2048, 130, 8, -1), (64, 896, 3, 1, -1),
])
def test_gemmh_f16_vs_oracle(dev, oracle, option, n_out, n_in, M, mt, sbk):
    """The F16 GEMM (gemmh.h) at the config-4 batch-8 shapes and at every
    m-tile height, with and without K slices, ragged M and n_out, against
    the oracle; a repeat gives the same bits."""
    option("GEMMH_MIN_M", "1")
    option("GEMM_MT", str(mt))
    option("GEMM_SBK", str(sbk))
    rng = np.random.default_rng(n_out + n_in + M + mt)
    W = synth.make_weights(sa.F16, n_out, n_in, rng)
    X = _rows(rng, M, n_in)
    w = dev.upload(sa.F16, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
        Y2 = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(sa.F16, W, n_out, n_in, X)
    what = f"gemmh F16 {n_out}x{n_in} M={M} MT={mt} SBK={sbk}"
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1), what)
    assert np.array_equal(Y.view(np.uint32), Y2.view(np.uint32)), what + ": repeat differs"


def test_gemmh_converting_launch_matches(dev, oracle, option):
    """At 16-row m blocks the F16 GEMM converts X itself as it stages each
    step's record; the results are the bits of the launch after a
    conversion launch (GEMMH_FUSE 0), call after call, with and without K
    slices, M of 1, 7 and 16 (rows past M zero), one and two m blocks
    (M = 20 at GEMM_MT 1), and within the bar of the oracle."""
    option("GEMMH_MIN_M", "1")
    rng = np.random.default_rng(4242)
    for n_out, n_in, M, mt, sbk in [(1024, 5120, 7, -1, -1), (300, 1280, 16, -1, 0),
                                    (5120, 5120, 1, -1, -1), (129, 384, 20, 1, 1),
                                    (27648, 5120, 8, -1, -1)]:
        W = synth.make_weights(sa.F16, n_out, n_in, rng)
        X = _rows(rng, M, n_in)
        w = dev.upload(sa.F16, n_out, n_in, W)
        try:
            option("GEMM_MT", str(mt))
            option("GEMM_SBK", str(sbk))
            outs = []
            for fuse in ("-1", "0", "-1"):
                option("GEMMH_FUSE", fuse)
                outs.append(dev.gemm(w, X))
        finally:
            w.free()
        what = f"F16 {n_out}x{n_in} M={M} MT={mt} SBK={sbk}"
        for y in outs[1:]:
            assert np.array_equal(y.view(np.uint32), outs[0].view(np.uint32)), what + ": launches differ"
        if n_out <= 1024:
            ref, L1 = oracle.gemm(sa.F16, W, n_out, n_in, X)
            assert_close(outs[0].reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1), what)


def test_f16_rows_not_multiple_of_128_take_the_matvec(dev, oracle):
    """F16 rows whose length is not a multiple of 128 elements (288 = 9 x
    32) have no GEMM copy: batches run on the matvec kernel, within the
    bar."""
    rng = np.random.default_rng(77)
    n_out, n_in, M = 200, 288, 12
    W = synth.make_weights(sa.F16, n_out, n_in, rng)
    X = _rows(rng, M, n_in)
    w = dev.upload(sa.F16, n_out, n_in, W)
    try:
        before = w.device_bytes
        w.prepare_gemm()
        assert w.device_bytes == before
        Y = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(sa.F16, W, n_out, n_in, X)
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1), "F16 288-wide rows")


@pytest.mark.parametrize("wt", [sa.Q4_0, sa.Q5_0, sa.Q8_0], ids=lambda t: sa.NAMES[t])
@pytest.mark.parametrize("n_out,n_in,M,mt,sbk", [
    (27648, 5120, 8, -1, -1), (5120, 27648, 8, -1, -1), (300, 1280, 70, 4, 0), (129, 384, 33, 2, 1),
    (4864, 896, 16, -1, -1), (64, 896, 3, 1, -1), (200, 1024, 40, 1, -1),
])
def test_gemmq_vs_oracle(dev, oracle, option, wt, n_out, n_in, M, mt, sbk):
    """The Q4_0 / Q5_0 / Q8_0 GEMM (gemmq.h) at the config-4 batch-8 shapes
    and config 1's 4864 x 896, every m-tile height, with and without K
    slices, the launch that quantizes X itself with one and with three
    16-row m blocks (M = 40 at GEMM_MT 1), rows at the ends of the quant
    ranges, against the oracle; a repeat gives the same bits."""
    option("GEMMQ_MIN_M", "1")
    option("GEMM_MT", str(mt))
    option("GEMM_SBK", str(sbk))
    rng = np.random.default_rng(n_out + n_in + M + mt + wt)
    W = _extreme_q80(synth.make_weights(wt, n_out, n_in, rng), wt, n_out, n_in)
    X = _rows(rng, M, n_in)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        Y = dev.gemm(w, X)
        Y2 = dev.gemm(w, X)
    finally:
        w.free()
    ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
    what = f"gemmq {sa.NAMES[wt]} {n_out}x{n_in} M={M} MT={mt} SBK={sbk}"
    assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1), what)
    assert np.array_equal(Y.view(np.uint32), Y2.view(np.uint32)), what + ": repeat differs"


@pytest.mark.parametrize("wt", [sa.Q4_0, sa.Q5_0, sa.Q8_0], ids=lambda t: sa.NAMES[t])
def test_gemmq_record_modes_match(dev, option, wt):
    """The Q8_0-pair GEMM's record modes give the same bits, call after
    call: records through the register ring (mode 0), a K slice's records
    in LDS up front (1, GEMMQ_FUSE 0) and, with 16-row m blocks, the slice
    quantized by the launch itself into LDS (1 with its rule: mode 2, no
    quantization launch); on weights whose n blocks leave idle workgroups
    (300 rows), with and without K slices, 16- and 32-row m blocks, and M
    past a multiple of 8."""
    option("GEMMQ_MIN_M", "1")
    rng = np.random.default_rng(4040 + wt)
    cases = [(300, 1280, 5, -1), (27648, 5120, 8, -1), (5120, 27648, 13, -1), (1024, 5120, 16, 0),
             (4864, 896, 3, 2), (5120, 5120, 24, -1)]
    for n_out, n_in, M, sbk in cases:
        W = synth.make_weights(wt, n_out, n_in, rng)
        w = dev.upload(wt, n_out, n_in, W)
        try:
            option("GEMM_SBK", str(sbk))
            outs = []
            for mode, fuse in (("0", "-1"), ("1", "0"), ("1", "-1"), ("0", "-1")):
                option("GEMMQ_XMODE", mode)
                option("GEMMQ_FUSE", fuse)
                X = _rows(np.random.default_rng(n_out + M), M, n_in)
                outs.append(dev.gemm(w, X).view(np.uint32))
            what = f"{sa.NAMES[wt]} {n_out}x{n_in} M={M} SBK={sbk}"
            for y in outs[1:]:
                assert np.array_equal(y, outs[0]), what + ": record modes differ"
        finally:
            w.free()
