"""The shortcuts of the device Q8_K block quantizer's usual path
(q8k_block_row16 in siphon_amd/csrc/quant.h), restated in numpy, against
the oracle's quantizer (reference kernels.c:561-595) on blocks of every
kind the shortcuts have to get right: the lane maxima taken as integer
maxima of the bit patterns, the block's first occurrence taken from the
lowest lane holding the maximum, the quant byte as the low byte of
iscale * x + 12582912 (no cap at 127), including blocks so small that
-127 / vmax overflows. Blocks the device sends to the element-by-element
scan (a non-finite element, or a lane whose largest |x| occurs with both
signs) are counted, not compared here; the GPU tests compare both paths
with the oracle bit for bit."""
import numpy as np

import siphon_amd as sa


def fast_block(x):
    """(d, quants, group sums) of one 256-element block, or None when the
    device takes the scan."""
    b = x.view(np.uint32).reshape(16, 16)  # lane l holds elements 16 l .. 16 l + 15
    pmax = b.view(np.int32).max(axis=1)
    nmax = b.max(axis=1)
    pa = np.where(pmax >= 0, pmax.astype(np.int64), 0).astype(np.uint32)
    na = np.where(nmax >= 0x80000000, nmax & 0x7FFFFFFF, 0).astype(np.uint32)
    la = np.maximum(pa, na)
    if np.any((la >= 0x7F800000) | ((pa == na) & (pa != 0))):
        return None
    abits = la.max()
    key = np.where(la == abits, ((15 - np.arange(16)) << 1) | (na > pa).astype(np.int64), 0).max()
    if abits == 0:
        return np.float32(0), np.zeros(256, np.int8), np.zeros(16, np.int16)
    vmax = np.array([abits | ((int(key) & 1) << 31)], np.uint32).view(np.float32)[0]
    with np.errstate(all="ignore"):
        iscale = np.float32(-127.0) / vmax
        t = ((iscale * x).astype(np.float32) + np.float32(12582912.0)).astype(np.float32)
        d = np.float32(1.0) / iscale
    q = (t.view(np.uint32) & 0xFF).astype(np.uint8).view(np.int8)
    return d, q, q.reshape(16, 16).astype(np.int32).sum(axis=1).astype(np.int16)


def blocks(rng, count):
    n = 256
    for i in range(count):
        k = i % 12
        if k == 0:
            x = rng.standard_normal(n)
        elif k == 1:
            x = rng.standard_normal(n) * 1e-3
        elif k == 2:
            x = rng.standard_normal(n) * 1e4
        elif k == 3:
            x = rng.standard_normal(n)
            x[rng.integers(0, n, 100)] = 0.0
            x[rng.integers(0, n, 30)] = -0.0
        elif k == 4:
            x = np.round(rng.standard_normal(n) * 3)  # ties of |x|
        elif k == 5:
            x = rng.standard_normal(n) * 1e-38  # subnormal
        elif k == 6:
            x = rng.uniform(-1, 1, n)
            a, c = rng.integers(0, n, 2)
            x[a], x[c] = 7.0, -7.0
        elif k == 7:
            x = rng.standard_normal(n) * 1e-44  # -127 / vmax overflows
        elif k == 8:
            x = np.zeros(n) * (-1.0 if i % 24 == 8 else 1.0)
        elif k == 9:
            x = np.zeros(n)
            x[rng.integers(0, n)] = rng.standard_normal()
        elif k == 10:
            x = rng.standard_normal(n) * 3e38
        else:
            x = rng.uniform(-1, 1, n) * 2.0 ** float(rng.integers(-140, 120))
        with np.errstate(all="ignore"):  # float32 overflow to inf: those blocks take the scan
            yield x.astype(np.float32)


def test_q8k_fast_path_matches_oracle(oracle):
    rng = np.random.default_rng(20261202)
    fast = scan = 0
    for x in blocks(rng, 6000):
        f = fast_block(x)
        if f is None:
            scan += 1
            continue
        fast += 1
        out = oracle.quantize(sa.Q8_K, x)
        assert out[:4].view(np.uint32)[0] == np.array([f[0]], np.float32).view(np.uint32)[0]
        assert np.array_equal(out[4:260].view(np.int8), f[1])
        assert np.array_equal(out[260:292].view(np.int16), f[2])
    assert fast > 4000 and scan > 500, (fast, scan)


def test_q8k_fast_path_declines_non_finite():
    x = np.ones(256, np.float32)
    for v in (np.inf, -np.inf, np.nan):
        y = x.copy()
        y[77] = v
        assert fast_block(y) is None
    y = x.copy()
    y[16] = -1.0  # lane 1 holds +1 and -1 at its maximum: the scan decides
    assert fast_block(y) is None
