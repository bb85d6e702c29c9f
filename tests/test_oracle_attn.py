"""Pins the oracle's decode attention (siq_attn_decode and its pieces in
oracle/siq_oracle.c) before it is trusted as the checker of the HIP
attention kernels.

- golden fixture written by the compiled reference (tests/golden/
  golden_attn_v1.npz): scores, f16 probabilities and outputs, bit-exact;
- the compiled reference's own exp polynomial, softmax and attention
  composition on fresh seeded inputs, when oracle/_ref is built;
- mathematics: the exp polynomial against double-precision exp, softmax
  rows summing to one, the f16 dot against its exact value, and the output
  against a double-precision contraction of the f16 probabilities.
"""
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "golden_attn_v1.npz")


@pytest.fixture(scope="module")
def gold():
    return dict(np.load(GOLDEN))


def bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


def f16f(u):
    return np.asarray(u, np.uint16).view(np.float16).astype(np.float64)


def test_golden_attention_bitexact(oracle, gold):
    saturated = 0
    for i, case in enumerate(gold["cases"]):
        n_head, n_kv, hd, n_ctx, pos = (int(v) for v in case[:5])
        out, sc, pr = oracle.attn_decode(gold[f"q{i}"], gold[f"k{i}"], gold[f"v{i}"], n_head,
                                         n_kv, hd, n_ctx, pos, float(gold[f"kq{i}"]))
        assert np.array_equal(bits(sc), bits(gold[f"scores{i}"])), f"case {i} scores"
        assert np.array_equal(pr, gold[f"probs{i}"]), f"case {i} probabilities"
        assert np.array_equal(bits(out), bits(gold[f"out{i}"])), f"case {i} output"
        n = pos + 1
        mx = sc[:, :n].max(axis=1, keepdims=True)
        saturated += int(np.count_nonzero((sc[:, :n] - mx) * 1.4426950408889634 < -192.0))
    assert saturated > 0, "no case reaches the exp polynomial's saturated branch"


def test_exp_poly_vs_reference_and_math(oracle, ref):
    rng = np.random.default_rng(41)
    x = np.concatenate([rng.uniform(-110, 0, 4000), rng.uniform(-300, 90, 2000),
                        [0.0, -0.0, -87.33, -87.34, -88.0, -103.9, -104.0, -133.0, -134.0,
                         88.0, 88.7, 89.0, np.inf, -np.inf]]).astype(np.float32)
    a = oracle.expf_poly(x)
    assert np.array_equal(bits(a), bits(ref.expf(x)))


def test_exp_poly_accuracy(oracle):
    """Within 2 ulp of exp in the normal range; 0 far below it."""
    rng = np.random.default_rng(43)
    x = rng.uniform(-87.0, 0.0, 20000).astype(np.float32)
    a = oracle.expf_poly(x).astype(np.float64)
    e = np.exp(x.astype(np.float64))
    ulp = np.spacing(e.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(a - e) <= 2 * ulp)
    assert np.all(oracle.expf_poly(np.array([-200.0, -500.0, -np.inf], np.float32)) == 0.0)
    assert oracle.expf_poly(np.array([0.0], np.float32))[0] == 1.0


@pytest.mark.parametrize("n", [1, 5, 8, 13, 64, 333])
def test_softmax_vs_reference_and_math(oracle, ref, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 4).astype(np.float32)
    y = oracle.softmax(x, float(x.max()))
    assert np.array_equal(bits(y), bits(ref.softmax(x, float(x.max()))))
    e = np.exp(x.astype(np.float64) - x.max())
    assert np.allclose(y, e / e.sum(), rtol=2e-6, atol=0)
    assert abs(y.astype(np.float64).sum() - 1.0) < 1e-6


@pytest.mark.parametrize("n", [1, 31, 32, 33, 64, 80, 128, 1000])
def test_dot_f16_vs_exact(oracle, n):
    rng = np.random.default_rng(1000 + n)
    a = rng.standard_normal(n).astype(np.float16)
    b = rng.standard_normal(n).astype(np.float16)
    terms = a.astype(np.float64) * b.astype(np.float64)
    got = oracle.dot_f16(a.view(np.uint16), b.view(np.uint16))
    assert abs(got - terms.sum()) <= 1e-6 * np.abs(terms).sum() + 1e-30


def test_dot_f16_golden(oracle):
    """The reference's AVX2 f16 dots of the kernel golden fixture (n = 1024)."""
    g = np.load(os.path.join(os.path.dirname(GOLDEN), "golden_v1.npz"))
    W, xq = g["w_F16"], g["xq_F16"]
    for r in range(W.shape[0]):
        got = np.float32(oracle.dot_f16(W[r].view(np.uint16), xq.view(np.uint16)))
        assert got.view(np.uint32) == np.float32(g["dot_avx2_F16"][r]).view(np.uint32)


@pytest.mark.parametrize("n_head,n_kv,hd,n_ctx,pos", [
    (4, 2, 64, 40, 37), (8, 8, 80, 48, 47), (6, 2, 128, 100, 0), (4, 1, 32, 36, 31),
    (2, 2, 96, 70, 69),
])
def test_attention_vs_reference(oracle, ref, n_head, n_kv, hd, n_ctx, pos):
    rng = np.random.default_rng(n_head * 1000 + hd + pos)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    k = rng.standard_normal(n_kv * n_ctx * hd).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(n_kv * n_ctx * hd).astype(np.float16).view(np.uint16)
    kq = float(np.float32(1.0 / np.sqrt(hd)))
    for a, b in zip(oracle.attn_decode(q, k, v, n_head, n_kv, hd, n_ctx, pos, kq),
                    ref.attn_decode(q, k, v, n_head, n_kv, hd, n_ctx, pos, kq)):
        assert np.array_equal(bits(a), bits(b))


def test_attention_vs_double_math(oracle):
    """Scores within the dot tolerance of exact q16.k, probabilities within
    an f16 rounding of the exact softmax of those scores, and the output
    within the dot tolerance of the exact contraction of the f16
    probabilities."""
    rng = np.random.default_rng(77)
    n_head, n_kv, hd, n_ctx, pos = 8, 2, 64, 90, 85
    n = pos + 1
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    k = rng.standard_normal((n_kv, n_ctx, hd)).astype(np.float16)
    v = rng.standard_normal((n_kv, hd, n_ctx)).astype(np.float16)
    kq = np.float32(0.125)
    out, sc, pr = oracle.attn_decode(q, k.view(np.uint16), v.view(np.uint16), n_head, n_kv, hd,
                                     n_ctx, pos, float(kq))
    for h in range(n_head):
        hk = h // (n_head // n_kv)
        q16 = q[h * hd:(h + 1) * hd].astype(np.float16).astype(np.float64)
        terms = k[hk, :n].astype(np.float64) * q16
        exact = terms.sum(axis=1) * np.float64(kq)
        assert np.all(np.abs(sc[h, :n] - exact) <= 1e-6 * np.abs(terms).sum(axis=1) + 1e-30)
        s = sc[h, :n].astype(np.float64)
        e = np.exp(s - s.max())
        p = e / e.sum()
        p16 = f16f(pr[h, :n])
        assert np.all(np.abs(p16 - p) <= np.spacing(p.astype(np.float16)).astype(np.float64) + 1e-9)
        vt = v[hk, :, :n].astype(np.float64) * p16
        got = out[h * hd:(h + 1) * hd].astype(np.float64)
        assert np.all(np.abs(got - vt.sum(axis=1)) <= 1e-5 * np.abs(vt).sum(axis=1) + 1e-6)


def test_attention_bad_arguments(oracle):
    import ctypes
    z = np.zeros(64, np.float32)
    u = np.zeros(64, np.uint16)
    L = oracle.L
    for args in ((4, 3, 8, 8, 0), (4, 2, 8, 8, 8), (4, 2, 8, 8, -1), (0, 1, 8, 8, 0)):
        nh, nkv, hd, n_ctx, pos = args
        assert L.siq_attn_decode(z.ctypes.data, u.ctypes.data, u.ctypes.data, nh, nkv, hd, n_ctx,
                                 pos, ctypes.c_float(1.0), z.ctypes.data, None, None) == 0
