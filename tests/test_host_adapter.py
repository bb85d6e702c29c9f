"""The C17 "hip" si_backend adapter (siphon_amd/host/backend_hip.c): the
drop-in for the reference's backend vtable (reference
include/siphon/tensor.h:43-55), driven through its test harness.

CPU tests: loading and failure behaviour (missing library, no device).
GPU tests: gemv / gemm / row_to_f32 through the vtable against the oracle,
upload-once caching, the load-time upload hook, and the reference's error
contract (message set, output untouched)."""
import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth
from siphon_amd.build import HIP_SO

SI_ENOENT, SI_EIO, SI_EINVAL = -6, -2, -5


@pytest.fixture(scope="module")
def harness():
    from tests import host_py
    return host_py.Harness()


def test_missing_library_is_reported(harness, tmp_path):
    rc, be = harness.open(str(tmp_path / "libsiphon_hip.so"))
    assert rc == SI_ENOENT and be is None
    assert "cannot load" in harness.errstr()


def test_open_reports_no_device_or_opens(harness):
    """Without a GPU (this container) opening fails with SI_EIO and a
    message; with one it succeeds and the backend is named "hip"."""
    rc, be = harness.open(HIP_SO)
    if rc == 0:
        assert harness.name(be) == "hip"
        harness.close(be)
    else:
        assert rc == SI_EIO, (rc, harness.errstr())
        assert "device" in harness.errstr()


def test_cpu_vtable_gemm_slot(harness, oracle):
    """The gemm slot as the CPU backend fills it (one gemv per activation
    row, the fill a maintainer adds to the reference backend.c) gives the
    rows of M separate gemv calls, for every weight type."""
    be = harness.cpu()
    rng = np.random.default_rng(41)
    for wt, n_out, n_in in ((sa.Q4_K, 40, 512), (sa.Q6_K, 17, 256), (sa.Q8_0, 9, 96),
                            (sa.F16, 8, 64), (sa.Q2_K, 5, 256)):
        W = synth.make_weights(wt, n_out, n_in, rng)
        X = rng.standard_normal((3, n_in)).astype(np.float32)
        Y = np.full((3, n_out), np.nan, np.float32)
        assert harness.vtable_gemm(be, wt, n_out, n_in, W, X, Y) == 0, harness.errstr()
        R, _ = oracle.gemm(wt, W, n_out, n_in, X)
        assert np.array_equal(Y, R.astype(np.float32)), sa.NAMES[wt]


@pytest.mark.gpu
def test_vtable_gemm_slot_both_backends(harness, oracle):
    """be->gemm through the vtable on the hip backend and on the CPU backend
    (one gemv per row), each against the oracle's M per-row gemvs, for
    every weight type; the hip slot fills Y and leaves it untouched on a
    bad call."""
    rc, be = harness.open(HIP_SO)
    assert rc == 0, harness.errstr()
    keep = []
    try:
        rng = np.random.default_rng(43)
        for wt, n_out, n_in in ((sa.Q4_K, 300, 2048), (sa.Q6_K, 129, 1024), (sa.Q8_0, 77, 896),
                                (sa.Q4_0, 64, 512), (sa.Q5_0, 65, 512), (sa.Q2_K, 96, 512),
                                (sa.Q3_K, 96, 512), (sa.Q5_K, 96, 512), (sa.F16, 64, 512)):
            W = synth.make_weights(wt, n_out, n_in, rng)
            keep.append(W)
            X = rng.standard_normal((5, n_in)).astype(np.float32)
            R, L1 = oracle.gemm(wt, W, n_out, n_in, X)
            for b in (be, harness.cpu()):
                Y = np.full((5, n_out), np.nan, np.float32)
                assert harness.vtable_gemm(b, wt, n_out, n_in, W, X, Y) == 0, harness.errstr()
                assert np.all(np.abs(Y.astype(np.float64) - R) <= 1e-5 * L1 + 1e-6), \
                    (sa.NAMES[wt], b == be)
        Y = np.full((0, 300), np.nan, np.float32)
        assert harness.vtable_gemm(be, sa.Q4_K, 300, 2048, keep[0], np.zeros((0, 2048), np.float32),
                                   Y) == SI_EINVAL
        assert "bad arguments" in harness.errstr()
    finally:
        harness.close(be)


@pytest.mark.gpu
def test_vtable_gemv_gemm_row_to_f32(harness, oracle):
    rc, be = harness.open(HIP_SO)
    assert rc == 0, harness.errstr()
    keep = []  # weights stay alive like an mmap: the adapter keys uploads by address
    try:
        rng = np.random.default_rng(17)
        for wt, n_out, n_in in ((sa.Q4_K, 300, 2048), (sa.Q6_K, 129, 1024), (sa.Q8_0, 77, 896),
                                (sa.F16, 64, 512), (sa.F32, 65, 501)):
            W = synth.make_weights(wt, n_out, n_in, rng)
            keep.append(W)
            x = rng.standard_normal(n_in).astype(np.float32)
            y = np.full(n_out, np.nan, np.float32)
            assert harness.gemv(be, wt, n_out, n_in, W, x, y, n_out) == 0, harness.errstr()
            ref, l1 = oracle.gemv(wt, W, n_out, n_in, x)
            assert np.all(np.abs(y.astype(np.float64) - ref) <= 1e-5 * l1 + 1e-6), sa.NAMES[wt]
            # a second call reuses the uploaded copy
            n_before, _ = harness.weights(be)
            y2 = np.zeros(n_out, np.float32)
            assert harness.gemv(be, wt, n_out, n_in, W, x, y2, n_out) == 0
            assert harness.weights(be)[0] == n_before
            assert np.array_equal(y, y2)
            # prefill slot
            X = rng.standard_normal((5, n_in)).astype(np.float32)
            Y = np.zeros((5, n_out), np.float32)
            assert harness.gemm(be, wt, n_out, n_in, W, X, Y) == 0, harness.errstr()
            R, L1 = oracle.gemm(wt, W, n_out, n_in, X)
            assert np.all(np.abs(Y.astype(np.float64) - R) <= 1e-5 * L1 + 1e-6)
            # embedding row lookup: the CPU dequantizer on the mmap'd row
            out = np.zeros(n_in, np.float32)
            assert harness.row_to_f32(be, wt, n_out, n_in, W, 3, out) == 0
            assert np.array_equal(out.view(np.uint32),
                                  oracle.dequant(wt, W[3], n_in).view(np.uint32))
        n, nbytes = harness.weights(be)
        assert n == 5 and nbytes > 0
    finally:
        harness.close(be)


@pytest.mark.gpu
def test_vtable_error_contract(harness):
    """On failure gemv sets the message and leaves y untouched (reference
    backend.c:90-98)."""
    rc, be = harness.open(HIP_SO)
    assert rc == 0, harness.errstr()
    try:
        rng = np.random.default_rng(5)
        W = synth.make_weights(sa.Q4_K, 16, 256, rng)
        x = rng.standard_normal(256).astype(np.float32)
        y = np.full(17, 7.0, np.float32)
        assert harness.gemv(be, sa.Q4_K, 16, 256, W, x, y, 17) == -1  # more rows than W has
        assert "n_out" in harness.errstr()
        assert np.all(y == 7.0)
        bad = np.zeros(10, np.uint8)  # byte count does not match the shape
        assert harness.gemv(be, sa.Q4_K, 16, 256, bad, x, y, 16) == -1
        assert "upload" in harness.errstr()
        assert np.all(y == 7.0)
    finally:
        harness.close(be)


@pytest.mark.gpu
def test_reused_address_is_not_served_stale(harness, oracle):
    """A host buffer that is freed and reused for a different tensor (a
    different type or shape at the same address, or the same type and
    shape with other contents, told apart by a fingerprint of 16 spans of
    the tensor: its edges and 14 evenly spaced inside) gets a fresh upload,
    also when only the inside changed."""
    rc, be = harness.open(HIP_SO)
    assert rc == 0, harness.errstr()
    try:
        rng = np.random.default_rng(23)
        buf = np.zeros(64 * 512 * 2, np.uint8)  # one address, two tensors over time
        W1 = synth.make_weights(sa.Q8_0, 32, 1024, rng)  # 32 x 32 blocks x 34 B
        buf[:W1.nbytes] = W1.reshape(-1)
        x1 = rng.standard_normal(1024).astype(np.float32)
        y1 = np.zeros(32, np.float32)
        assert harness.gemv(be, sa.Q8_0, 32, 1024, buf[:W1.nbytes], x1, y1, 32) == 0
        ref1, l1 = oracle.gemv(sa.Q8_0, W1, 32, 1024, x1)
        assert np.all(np.abs(y1.astype(np.float64) - ref1) <= 1e-5 * l1 + 1e-6)
        W2 = synth.make_weights(sa.F16, 64, 512, rng)
        buf[:W2.nbytes] = W2.reshape(-1)
        x2 = rng.standard_normal(512).astype(np.float32)
        y2 = np.zeros(64, np.float32)
        assert harness.gemv(be, sa.F16, 64, 512, buf[:W2.nbytes], x2, y2, 64) == 0
        ref2, l2 = oracle.gemv(sa.F16, W2, 64, 512, x2)
        assert np.all(np.abs(y2.astype(np.float64) - ref2) <= 1e-5 * l2 + 1e-6)
        assert harness.weights(be)[0] == 1  # the stale copy was replaced, not kept
        W3 = synth.make_weights(sa.F16, 64, 512, rng)  # same type and shape, new contents
        buf[:W3.nbytes] = W3.reshape(-1)
        y3 = np.zeros(64, np.float32)
        assert harness.gemv(be, sa.F16, 64, 512, buf[:W3.nbytes], x2, y3, 64) == 0
        ref3, l3 = oracle.gemv(sa.F16, W3, 64, 512, x2)
        assert np.all(np.abs(y3.astype(np.float64) - ref3) <= 1e-5 * l3 + 1e-6)
        assert harness.weights(be)[0] == 1
        # same edges, new rows 16..47 (16 KiB in the middle of 64 KiB)
        W4 = W3.copy()
        W4[16:48] = synth.make_weights(sa.F16, 32, 512, rng)
        buf[:W4.nbytes] = W4.reshape(-1)
        y4 = np.zeros(64, np.float32)
        assert harness.gemv(be, sa.F16, 64, 512, buf[:W4.nbytes], x2, y4, 64) == 0
        ref4, l4 = oracle.gemv(sa.F16, W4, 64, 512, x2)
        assert np.all(np.abs(y4.astype(np.float64) - ref4) <= 1e-5 * l4 + 1e-6)
        assert harness.weights(be)[0] == 1
    finally:
        harness.close(be)


@pytest.mark.gpu
def test_load_time_upload(harness, oracle):
    """si_backend_hip_upload puts every tensor of a model on the device at
    load time, the matrix-core GEMM copy of Q4_K included: later gemv / gemm
    calls on them allocate nothing, a second upload of the same tensor is a
    no-op, and a bad tensor is refused with a message."""
    rc, be = harness.open(HIP_SO)
    assert rc == 0, harness.errstr()
    try:
        rng = np.random.default_rng(31)
        shapes = ((sa.Q4_K, 256, 4096), (sa.Q6_K, 96, 9216), (sa.Q5_0, 33, 640))
        Ws = [synth.make_weights(wt, n_out, n_in, rng) for wt, n_out, n_in in shapes]
        for (wt, n_out, n_in), W in zip(shapes, Ws):
            assert harness.upload(be, wt, n_out, n_in, W) == 0, harness.errstr()
        n, nbytes = harness.weights(be)
        assert n == len(shapes) and nbytes >= sum(W.nbytes for W in Ws)
        for (wt, n_out, n_in), W in zip(shapes, Ws):
            assert harness.upload(be, wt, n_out, n_in, W) == 0
            x = rng.standard_normal(n_in).astype(np.float32)
            y = np.full(n_out, np.nan, np.float32)
            assert harness.gemv(be, wt, n_out, n_in, W, x, y, n_out) == 0, harness.errstr()
            ref, l1 = oracle.gemv(wt, W, n_out, n_in, x)
            assert np.all(np.abs(y.astype(np.float64) - ref) <= 1e-5 * l1 + 1e-6), sa.NAMES[wt]
            X = rng.standard_normal((8, n_in)).astype(np.float32)
            Y = np.zeros((8, n_out), np.float32)
            assert harness.gemm(be, wt, n_out, n_in, W, X, Y) == 0, harness.errstr()
            R, L1 = oracle.gemm(wt, W, n_out, n_in, X)
            assert np.all(np.abs(Y.astype(np.float64) - R) <= 1e-5 * L1 + 1e-6), sa.NAMES[wt]
        assert harness.weights(be) == (n, nbytes)
        bad = np.zeros(10, np.uint8)  # byte count does not match the shape
        assert harness.upload(be, sa.Q4_K, 16, 256, bad) == SI_EINVAL
        assert "upload" in harness.errstr()
        assert harness.weights(be) == (n, nbytes)
    finally:
        harness.close(be)


@pytest.mark.gpu
def test_si_scalar_selects_the_scalar_q8_0_quantizer(harness, oracle, monkeypatch):
    """With SI_SCALAR set the reference quantizes Q8_0 activations with its
    scalar routine (reference kernels.c:80-83, 542-558); the adapter opened
    then makes the device do the same."""
    from tests.test_gpu_q80_scalar import oracle_rows, tie_vector
    rng = np.random.default_rng(23)
    n_out, n_in = 64, 1024
    W = synth.make_weights(sa.Q8_0, n_out, n_in, rng)
    x = tie_vector(rng, n_in)
    for scalar in (True, False):
        if scalar:
            monkeypatch.setenv("SI_SCALAR", "1")
        else:
            monkeypatch.delenv("SI_SCALAR", raising=False)
        rc, be = harness.open(HIP_SO)
        assert rc == 0, harness.errstr()
        try:
            y = np.zeros(n_out, np.float32)
            assert harness.gemv(be, sa.Q8_0, n_out, n_in, W, x, y, n_out) == 0, harness.errstr()
        finally:
            harness.close(be)
        ref, l1 = oracle_rows(oracle, sa.Q8_0, W, n_in,
                              oracle.quantize(sa.Q8_0, x, scalar_q8_0=scalar))
        assert np.all(np.abs(y.astype(np.float64) - ref) <= 1e-5 * l1 + 1e-6), scalar
