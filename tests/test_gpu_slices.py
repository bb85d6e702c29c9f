"""GPU checks of column-sliced matvecs: long rows are cut into slices that
separate workgroups compute, and the last workgroup of each row group to
arrive adds the partial sums in slice order (an arrival counter per group,
reset by that workgroup for the next launch).

Bars as in test_gpu_parity: within 1e-5 * sum|terms| + 1e-6 of the oracle,
and bit-identical to the host emulation of the same slicing for the integer
formats. Repeated calls, calls with fewer rows, batched columns, fused
multi-matrix launches and HIP-graph replays must give the same bits as a
fresh eager call, which fails if a counter is left non-zero or a partial sum
is read before it is written.
"""
import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth

from tests.test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu

KQ = (sa.Q2_K, sa.Q3_K, sa.Q4_K, sa.Q5_K, sa.Q6_K)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("wt", sa.WEIGHT_TYPES, ids=lambda t: sa.NAMES[t])
def test_slices_vs_emulator_and_oracle(dev, oracle, emu, wt, option):
    rng = np.random.default_rng(900 + wt)
    n_out, n_in = (150, 2304) if wt in KQ else (150, 1120)
    W = synth.make_weights(wt, n_out, n_in, rng)
    x = rng.standard_normal(n_in).astype(np.float32)
    xq = oracle.quantize(sa.PAIR[wt], x)
    ref = np.zeros(n_out)
    l1 = np.zeros(n_out)
    for r in range(n_out):
        ref[r], l1[r] = oracle.vec_dot(wt, n_in, W[r], xq)
    for G in (1, 4, 16):
        option("TILE_COLS", str(G))
        for elems in (1, 256, 1024, 0):
            option("SPLIT_ELEMS", str(elems))
            what = f"{sa.NAMES[wt]} {n_out}x{n_in} G={G} slice={elems}"
            y = dev.gemv_pair(wt, n_out, n_in, W, xq)
            assert_close(y, ref, l1, what)
            if wt != sa.F16:
                ye = emu.gemv_pair(wt, n_out, n_in, G, W, xq, slice_elems=elems)
                assert np.array_equal(bits(y), bits(ye)), f"{what}: GPU differs from emulation"


@pytest.mark.parametrize("wt", [sa.Q4_K, sa.Q6_K, sa.Q8_0, sa.F16], ids=lambda t: sa.NAMES[t])
def test_sliced_calls_repeat_bit_exact(dev, oracle, option, wt):
    """Default slicing of long rows (n_in >= 8192; here 3 slices, the last
    one shorter): a sequence of calls with different activations, fewer rows
    and batched columns, each against the oracle, and the first activation
    again at the end gives the same bits."""
    option("GEMM_MIN_M", "1000")  # batches take the matvec kernel
    option("GEMM6_MIN_M", "1000")
    option("TILE_COLS", "4")  # several rounds per tile (the default is 1 here)
    rng = np.random.default_rng(950 + wt)
    n_out, n_in = 300, 9216
    W = synth.make_weights(wt, n_out, n_in, rng)
    w = dev.upload(wt, n_out, n_in, W)
    try:
        cols = n_in // (256 if wt in KQ else 32)
        rounds = -(-cols // w.tile_cols)
        assert w.slice_rounds < rounds, "rows of 9216 in tiles 4 wide are expected to be sliced"
        xs = [rng.standard_normal(n_in).astype(np.float32) for _ in range(3)]
        first = None
        for x in xs:
            y = dev.gemv(w, x)
            ref, l1 = oracle.gemv(wt, W, n_out, n_in, x)
            assert_close(y, ref.astype(np.float64), l1, f"{sa.NAMES[wt]} sliced gemv")
            first = y if first is None else first
        y = dev.gemv(w, xs[0], n_out=77)
        ref, l1 = oracle.gemv(wt, W[:77], 77, n_in, xs[0])
        assert_close(y, ref.astype(np.float64), l1, f"{sa.NAMES[wt]} sliced gemv n_out=77")
        assert np.array_equal(bits(y), bits(first[:77]))
        for M in (2, 5):
            X = rng.standard_normal((M, n_in)).astype(np.float32)
            X[0] = xs[0]
            Y = dev.gemm(w, X)
            ref, L1 = oracle.gemm(wt, W, n_out, n_in, X)
            assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                         f"{sa.NAMES[wt]} sliced gemm M={M}")
        assert np.array_equal(bits(dev.gemv(w, xs[0])), bits(first))
    finally:
        w.free()


def test_sliced_multi_matches_single(dev, oracle, option):
    """A fused launch of sliced and unsliced matrices gives the bits of one
    launch per matrix."""
    rng = np.random.default_rng(977)
    n_in = 8192
    shapes = [(sa.Q4_K, 333), (sa.Q6_K, 64), (sa.Q4_K, 1000)]
    Ws = [synth.make_weights(wt, n, n_in, rng) for wt, n in shapes]
    ws = []
    for (wt, n), W, (G, elems) in zip(shapes, Ws, [(8, 4096), (4, 4096), (8, 0)]):
        option("TILE_COLS", str(G))
        option("SPLIT_ELEMS", str(elems))
        ws.append(dev.upload(wt, n, n_in, W))
    assert [w.slice_rounds for w in ws] == [2, 4, 4]
    bufs = []
    try:
        x = rng.standard_normal(n_in).astype(np.float32)
        xd = dev.to_device(x)
        nan = lambda n: np.full(n, np.nan, np.float32)  # noqa: E731
        ys = [dev.to_device(nan(n)) for _, n in shapes]
        singles = [dev.to_device(nan(n)) for _, n in shapes]
        bufs = [xd, *ys, *singles]
        for _ in range(2):
            dev.gemv_multi_dev(ws, xd.ptr, [y.ptr for y in ys])
            for w, y, (_, n) in zip(ws, singles, shapes):
                dev.gemv_dev(w, xd.ptr, y.ptr, n)
            dev.synchronize()
            for (wt, n), W, y, y1 in zip(shapes, Ws, ys, singles):
                a, b = y.to_host(np.float32, n), y1.to_host(np.float32, n)
                assert np.array_equal(bits(a), bits(b)), sa.NAMES[wt]
                ref, l1 = oracle.gemv(wt, W, n, n_in, x)
                assert_close(a, ref.astype(np.float64), l1, f"multi {sa.NAMES[wt]} {n}x{n_in}")
    finally:
        for b in bufs:
            b.free()
        for w in ws:
            w.free()


class _HipGraph:
    """Stream capture and replay through the HIP runtime the library itself
    links (libamdhip64), so no second runtime (torch's) enters the process."""

    def __init__(self):
        import ctypes

        self.ct = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.stream = ctypes.c_void_p()
        self._ok(self.hip.hipStreamCreate(ctypes.byref(self.stream)))
        self.graph = ctypes.c_void_p()
        self.exec = ctypes.c_void_p()

    def _ok(self, rc):
        assert rc == 0, f"HIP error {rc}"

    def begin(self):
        self._ok(self.hip.hipStreamBeginCapture(self.stream, 0))  # global capture mode

    def end(self):
        ct = self.ct
        self._ok(self.hip.hipStreamEndCapture(self.stream, ct.byref(self.graph)))
        self._ok(self.hip.hipGraphInstantiate(ct.byref(self.exec), self.graph, None, None,
                                              ct.c_size_t(0)))

    def replay(self):
        self._ok(self.hip.hipGraphLaunch(self.exec, self.stream))
        self._ok(self.hip.hipStreamSynchronize(self.stream))

    def close(self):
        if self.exec.value:
            self.hip.hipGraphExecDestroy(self.exec)
        if self.graph.value:
            self.hip.hipGraphDestroy(self.graph)
        self.hip.hipStreamDestroy(self.stream)


def test_sliced_graph_replays(dev):
    """A captured sliced launch replayed several times, with eager launches
    of the same weight between the replays, gives the eager bits each time."""
    rng = np.random.default_rng(991)
    n_out, n_in = 4096, 14336
    W = synth.make_weights(sa.Q6_K, n_out, n_in, rng)
    w = dev.upload(sa.Q6_K, n_out, n_in, W)
    # the default layout slices these rows (4096 elements per slice)
    assert w.slice_rounds * w.tile_cols * 256 == 4096
    hg = _HipGraph()
    bufs = []
    try:
        nan = np.full(n_out, np.nan, np.float32)
        xd = dev.to_device(rng.standard_normal(n_in).astype(np.float32))
        y_eager, y_graph = dev.to_device(nan), dev.to_device(nan)
        bufs = [xd, y_eager, y_graph]
        dev.gemv_dev(w, xd.ptr, y_eager.ptr, n_out, hg.stream.value)
        dev.synchronize()
        want = y_eager.to_host(np.float32, n_out).copy()
        hg.begin()
        dev.gemv_dev(w, xd.ptr, y_graph.ptr, n_out, hg.stream.value)
        hg.end()
        for _ in range(3):
            y_graph.fill(nan)
            hg.replay()
            assert np.array_equal(bits(y_graph.to_host(np.float32, n_out)), bits(want))
            y_eager.fill(nan)
            dev.gemv_dev(w, xd.ptr, y_eager.ptr, n_out, hg.stream.value)
            dev.synchronize()
            assert np.array_equal(bits(y_eager.to_host(np.float32, n_out)), bits(want))
    finally:
        hg.close()
        for b in bufs:
            b.free()
        w.free()
