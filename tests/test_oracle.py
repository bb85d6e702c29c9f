"""Pins the CPU oracle (oracle/siq_oracle.c) before it is trusted as the
checker of the HIP path.

- golden vectors written by the compiled reference (tests/golden): f16
  conversion, both quantizers (bit-exact), dequantization (bit-exact), and
  every dot product of the reference's AVX2 and scalar paths;
- a library routine: numpy's IEEE binary16 conversion, exhaustively;
- an independent formulation: each exact dot recomputed element-wise from
  the dequantized weights;
- the quantizer invariants of reference tests/test_kernels.c:264-321;
- the compiled reference itself on fresh seeded inputs, when oracle/_ref is
  built (this container).
"""
import os

import numpy as np
import pytest

from oracle import siq

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden_v1.npz")
N = 1024


@pytest.fixture(scope="module")
def gold():
    return dict(np.load(GOLDEN))


def mask_zero_block_bsums(q8k: np.ndarray) -> np.ndarray:
    """bsums of an all-zero Q8_K block are unwritten by the reference
    (reference kernels.c:574-579); compare them only where d != 0."""
    b = q8k.reshape(-1, 292).copy()
    d = b[:, :4].copy().view(np.float32).reshape(-1)
    b[d == 0, 260:] = 0
    return b


# ---- f16 ------------------------------------------------------------------------

def test_f16_to_f32_exhaustive_vs_numpy(oracle):
    h = np.arange(65536, dtype=np.uint32)
    got = np.array([oracle.f16_to_f32(int(v)) for v in h], dtype=np.float32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f16_roundtrip_exhaustive(oracle):
    for h in range(65536):
        if (h & 0x7C00) == 0x7C00:
            continue  # inf / nan
        assert oracle.f32_to_f16(oracle.f16_to_f32(h)) == h


def test_f32_to_f16_vs_numpy(oracle):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(20000) * 100, rng.standard_normal(20000) * 1e-5,
                        rng.standard_normal(5000) * 1e-8,
                        [65504, 65519.99, 65520, 1e10, -1e10, 6e-8, 2.98e-8, 2.9802322e-8,
                         5.96e-8, 0, -0.0, np.inf, -np.inf]]).astype(np.float32)
    got = np.array([oracle.f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_golden(oracle, gold):
    got = np.array([oracle.f32_to_f16(float(v)) for v in gold["f16_in"]], dtype=np.uint16)
    assert np.array_equal(got, gold["f16_out"])


# ---- quantizers -------------------------------------------------------------------

def test_q8_K_golden(oracle, gold):
    for row, want in zip(gold["act"], gold["q8K"]):
        got = oracle.quantize(siq.Q8_K, row)
        assert np.array_equal(mask_zero_block_bsums(got), mask_zero_block_bsums(want))


def test_q8_0_simd_golden(oracle, gold):
    for row, want in zip(gold["act"], gold["q80_simd"]):
        assert np.array_equal(oracle.quantize(siq.Q8_0, row), want)


def test_q8_0_scalar_golden(oracle, gold):
    for row, want in zip(gold["act"], gold["q80_scalar"]):
        assert np.array_equal(oracle.quantize(siq.Q8_0, row, scalar_q8_0=True), want)


def test_quantizer_invariants(oracle):
    """reference tests/test_kernels.c:264-321, over many random rows."""
    rng = np.random.default_rng(11)
    for _ in range(20):
        x = rng.uniform(-1, 1, N).astype(np.float32)
        q0 = oracle.quantize(siq.Q8_0, x).reshape(-1, 34)
        d0 = q0[:, :2].copy().view(np.float16).astype(np.float32).reshape(-1)
        qs0 = q0[:, 2:].view(np.int8).astype(np.float32)
        xb = x.reshape(-1, 32)
        amax = np.abs(xb).max(axis=1)
        assert np.all(np.abs(d0 - amax / 127) < 1e-3 * (amax / 127 + 1e-6))
        assert np.all(np.abs(qs0 * d0[:, None] - xb) <= d0[:, None] * 0.5 + np.abs(xb) * 5e-4 + 1e-6)
        assert np.all(np.abs(qs0) <= 127)
        qk = oracle.quantize(siq.Q8_K, x).reshape(-1, 292)
        dk = qk[:, :4].copy().view(np.float32).reshape(-1)
        qsk = qk[:, 4:260].view(np.int8).astype(np.int32)
        bs = qk[:, 260:].copy().view(np.int16).reshape(-1, 16)
        xk = x.reshape(-1, 256)
        idx = np.argmax(np.abs(xk), axis=1)  # first occurrence, like the reference
        vmax = xk[np.arange(xk.shape[0]), idx]
        assert np.all(np.abs(dk - vmax / -127) < np.abs(vmax / -127) * 1e-5 + 1e-9)
        assert np.all(np.abs(qsk) <= 127)
        assert np.all(np.abs(qsk * dk[:, None] - xk) <= np.abs(dk)[:, None] * 1.01)
        assert np.array_equal(bs, qsk.reshape(-1, 16, 16).sum(axis=2))
    z = np.zeros(N, np.float32)
    assert np.all(oracle.quantize(siq.Q8_0, z).reshape(-1, 34)[:, :2] == 0)
    assert np.all(oracle.quantize(siq.Q8_K, z) == 0)


# ---- dequantization and dots ----------------------------------------------------------

@pytest.mark.parametrize("wt", siq.WEIGHT_TYPES, ids=lambda t: siq.NAMES[t])
def test_dequant_golden(oracle, gold, wt):
    name = siq.NAMES[wt]
    for W, want in zip(gold[f"w_{name}"], gold[f"deq_{name}"]):
        assert np.array_equal(oracle.dequant(wt, W, N).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("wt", siq.WEIGHT_TYPES, ids=lambda t: siq.NAMES[t])
def test_dot_golden(oracle, gold, wt):
    """The exact dot agrees with both reference paths to their own f32
    rounding (measured ~1e-7 of sum|terms|); a dropped term, wrong sign or
    wrong scale would be off by orders of magnitude more."""
    name = siq.NAMES[wt]
    xq = gold[f"xq_{name}"]
    for r, W in enumerate(gold[f"w_{name}"]):
        d, l1 = oracle.vec_dot(wt, N, W, xq)
        for path in ("avx2", "scalar"):
            ref = float(gold[f"dot_{path}_{name}"][r])
            assert abs(ref - d) <= 1e-6 * l1, (name, path, r, ref, d, l1)


@pytest.mark.parametrize("wt", siq.WEIGHT_TYPES, ids=lambda t: siq.NAMES[t])
def test_dot_formulations_agree(oracle, wt):
    """Integer-sum/scale formulation vs element-wise dequantized formulation.
    The element-wise form rounds each weight value to f32 (at most two
    roundings in d*sc*q - dmin*m), so the two agree to ~2^-22 of sum|terms|;
    a wrong scale, sign or index is off by orders of magnitude more."""
    rng = np.random.default_rng(40 + wt)
    from siphon_amd import synth
    W = synth.make_weights(wt, 6, N, rng)
    x = rng.standard_normal(N).astype(np.float32)
    xq = oracle.quantize(siq.PAIR[wt], x)
    for r in range(6):
        a, l1 = oracle.vec_dot(wt, N, W[r], xq)
        b, _ = oracle.vec_dot(wt, N, W[r], xq, dequant_form=True)
        assert abs(a - b) <= 3e-7 * l1


def test_closed_form_q4_K():
    """One Q4_K block written by hand: every sub-block scale 1 and min 0, all
    nibbles 1, d = 1, dmin = 0; activation Q8_K with d = 0.5 and quants 2:
    the dot is 256 * 1 * (2 * 0.5) = 256."""
    from oracle import siq as s
    o = s.Oracle()
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.array([1.0], np.float16).view(np.uint8)     # d
    blk[2:4] = np.array([0.0], np.float16).view(np.uint8)     # dmin
    blk[4:8] = 1                                              # scales 0..3 = 1, mins 0..3 = 0
    blk[12:16] = 0x01                                         # scales 4..7 low nibble 1, mins 0
    blk[16:144] = 0x11                                        # both nibbles 1
    act = np.zeros(292, np.uint8)
    act[0:4] = np.array([0.5], np.float32).view(np.uint8)
    act[4:260] = 2
    act[260:292] = np.full(16, 32, np.int16).view(np.uint8)
    d, l1 = o.vec_dot(s.Q4_K, 256, blk, act)
    assert d == 256.0 and l1 == 256.0


# ---- the compiled reference on fresh inputs ------------------------------------------

def test_against_compiled_reference(oracle, ref):
    rng = np.random.default_rng(99)
    for _ in range(30):
        x = (rng.standard_normal(N) * rng.choice([1e-3, 1.0, 1e3])).astype(np.float32)
        x[rng.integers(0, N, 8)] = 0.0
        assert np.array_equal(mask_zero_block_bsums(oracle.quantize(siq.Q8_K, x)),
                              mask_zero_block_bsums(ref.quant_q8_K(x)))
        assert np.array_equal(oracle.quantize(siq.Q8_0, x), ref.quant_q8_0(x, simd=True))
    from siphon_amd import synth
    for wt in siq.WEIGHT_TYPES:
        W = synth.make_weights(wt, 8, N, rng)
        x = rng.standard_normal(N).astype(np.float32)
        xq = oracle.quantize(siq.PAIR[wt], x)
        for r in range(8):
            assert np.array_equal(oracle.dequant(wt, W[r], N), ref.dequant(wt, W[r], N))
            d, l1 = oracle.vec_dot(wt, N, W[r], xq)
            for simd in (True, False):
                assert abs(ref.dot(wt, N, W[r], xq, simd=simd) - d) <= 1e-6 * l1


def test_f32_dot_exact_and_vs_reference(oracle):
    """F32 weights (reference pair F32: x passes through, si_dot_f32 sums
    float products in double, kernels.c:180-187): the oracle's dot is the
    exact sum of exact products, so it equals numpy's float64 dot of the
    same values to double rounding; against the compiled reference's own
    gemv (where oracle/_ref is built) each row is within the reference's
    float-product rounding, at most 2^-24 of the terms' L1."""
    rng = np.random.default_rng(32)
    n_out, n_in = 37, 1001  # odd length: no vector assumption
    W = rng.uniform(-0.05, 0.05, (n_out, n_in)).astype(np.float32)
    x = rng.standard_normal(n_in).astype(np.float32)
    Wb = W.view(np.uint8)
    y, l1 = oracle.gemv(siq.F32, Wb, n_out, n_in, x)
    exact = W.astype(np.float64) @ x.astype(np.float64)
    assert np.all(np.abs(y.astype(np.float64) - exact) <= 2.0 ** -24 * np.abs(exact) + 1e-30)
    assert np.allclose(l1, np.abs(W.astype(np.float64) * x.astype(np.float64)).sum(axis=1))
    d, m = oracle.vec_dot(siq.F32, n_in, Wb[5], x.view(np.uint8))
    assert abs(d - exact[5]) <= 1e-12 * m
    assert np.array_equal(oracle.dequant(siq.F32, Wb[3], n_in), W[3])
    r = siq.Reference.load()
    if r is not None:
        yr, _ = r.gemv_timed(siq.F32, Wb, n_out, n_in, x, 1, 1)
        assert np.all(np.abs(yr.astype(np.float64) - exact) <= 2.0 ** -24 * l1 + 2.0 ** -24 * np.abs(exact))
