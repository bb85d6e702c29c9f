"""GPU parity of the decode attention kernels (sihip_attn_decode_dev)
against the oracle's restatement of the reference's attn_head (reference
engine.c:90-147), itself pinned bit-exact to the compiled reference by
tests/test_oracle_attn.py.

Bar: scores, f16 probabilities and outputs bit-identical to the oracle.
The kernels sum the softmax's group totals in a different double order and
evaluate the last n % 8 exponentials in double rather than with libm's
expf; either can change a result only in rare cases, which the seeds used
here do not hit (a change would show as a failure, not be tolerated).
"""
import os

import numpy as np
import pytest

import siphon_amd as sa

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "golden_attn_v1.npz")


def bits(a):
    return np.ascontiguousarray(a).view(np.uint8)


def run_attn(dev, q, k, v, n_head, n_kv, hd, n_ctx, pos, kq, caller_buffers=True):
    bufs = []
    try:
        qd, kd, vd = dev.to_device(q), dev.to_device(k), dev.to_device(v)
        od = dev.to_device(np.full(n_head * hd, np.nan, np.float32))
        bufs = [qd, kd, vd, od]
        sd = pd = None
        if caller_buffers:
            sd = dev.to_device(np.zeros((n_head, n_ctx), np.float32))
            pd = dev.to_device(np.zeros((n_head, n_ctx), np.uint16))
            bufs += [sd, pd]
        dev.attn_decode_dev(qd.ptr, kd.ptr, vd.ptr, n_head, n_kv, hd, n_ctx, pos, kq, od.ptr,
                            sd.ptr if sd else None, pd.ptr if pd else None)
        dev.synchronize()
        out = od.to_host(np.float32, n_head * hd)
        if not caller_buffers:
            return out, None, None
        return (out, sd.to_host(np.float32, n_head * n_ctx).reshape(n_head, n_ctx),
                pd.to_host(np.uint16, n_head * n_ctx).reshape(n_head, n_ctx))
    finally:
        for b in bufs:
            b.free()


def check(got, want, n, what):
    out, sc, pr = got
    wout, wsc, wpr = want
    assert np.array_equal(bits(sc[:, :n]), bits(wsc[:, :n])), f"{what}: scores"
    assert np.array_equal(pr[:, :n], wpr[:, :n]), f"{what}: probabilities"
    assert np.array_equal(bits(out), bits(wout)), f"{what}: output"


def test_golden_cases(dev):
    g = dict(np.load(GOLDEN))
    for i, case in enumerate(g["cases"]):
        n_head, n_kv, hd, n_ctx, pos = (int(v) for v in case[:5])
        got = run_attn(dev, g[f"q{i}"], g[f"k{i}"], g[f"v{i}"], n_head, n_kv, hd, n_ctx, pos,
                       float(g[f"kq{i}"]))
        check(got, (g[f"out{i}"], g[f"scores{i}"], g[f"probs{i}"]), pos + 1, f"golden case {i}")


@pytest.mark.parametrize("n_head,n_kv,hd,n_ctx,pos", [
    (32, 8, 128, 4096, 4095),   # Llama-3-8B at a full 4096 context
    (32, 8, 128, 4100, 4098),   # dot and softmax tails
    (12, 2, 64, 300, 31),       # n = 32: dot body only
    (5, 5, 80, 64, 40),         # head dim with a dot tail, no GQA
    (16, 1, 96, 200, 199),      # 16 query heads on one KV head (4 passes)
    (6, 2, 256, 33, 0),         # position 0
    (3, 1, 8, 20, 17),          # head dim below one 32-element step
    (4, 2, 66, 40, 39),         # head dim not a multiple of 4: narrow key loads
    (8, 2, 128, 700, 511),      # n = 512: one 8-group per lane of a wave
    (4, 1, 64, 520, 504),       # n = 505: the tail in the wave's last lane
    (8, 2, 128, 700, 515),      # n = 516: a second group per lane, a tail
    (8, 2, 128, 2048, 1800),    # n = 1801: four groups per lane (ATTN_FUSE 4)
])
@pytest.mark.parametrize("fuse", [-1, 0, 4], ids=["rule", "three_launches", "two_to_2048"])
def test_vs_oracle(dev, oracle, option, n_head, n_kv, hd, n_ctx, pos, fuse):
    """Up to 1024 positions (ATTN_FUSE k: 512 k) the value launch's waves
    compute their heads' softmax themselves, with no softmax launch
    (ATTN_FUSE 0: three launches); each against the oracle, twice in a
    row."""
    option("ATTN_FUSE", fuse)
    rng = np.random.default_rng(n_head * 7919 + hd * 31 + pos)
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    k = (rng.standard_normal(n_kv * n_ctx * hd) * 2).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(n_kv * hd * n_ctx).astype(np.float16).view(np.uint16)
    kq = float(np.float32(1.0 / np.sqrt(np.float32(hd))))
    want = oracle.attn_decode(q, k, v, n_head, n_kv, hd, n_ctx, pos, kq)
    for _ in range(2):
        got = run_attn(dev, q, k, v, n_head, n_kv, hd, n_ctx, pos, kq)
        check(got, want, pos + 1, f"{n_head}/{n_kv} heads hd={hd} pos={pos} fuse={fuse}")
    # the context's workspace instead of caller buffers: the same output
    out_ws, _, _ = run_attn(dev, q, k, v, n_head, n_kv, hd, n_ctx, pos, kq,
                            caller_buffers=False)
    assert np.array_equal(bits(out_ws), bits(want[0]))


def test_bad_arguments(dev):
    buf = dev.to_device(np.zeros(4096, np.float32))
    try:
        p = buf.ptr
        for args, msg in (((4, 3, 64, 16, 0), "multiple"), ((4, 2, 600, 16, 0), "head_dim"),
                          ((4, 2, 64, 16, 16), "pos"), ((4, 2, 64, 16, -1), "pos")):
            n_head, n_kv, hd, n_ctx, pos = args
            with pytest.raises(sa.SihipError, match=msg):
                dev.attn_decode_dev(p, p, p, n_head, n_kv, hd, n_ctx, pos, 1.0, p)
    finally:
        buf.free()


def test_two_launch_graph_replays(dev, oracle):
    """The two-launch attention captured in a HIP graph: every replay, with
    eager calls between the replays, gives the oracle's bits."""
    from .test_gpu_slices import _HipGraph

    rng = np.random.default_rng(5120)
    n_head, n_kv, hd, n_ctx, pos = 32, 8, 128, 1024, 300
    q = rng.standard_normal(n_head * hd).astype(np.float32)
    k = (rng.standard_normal(n_kv * n_ctx * hd) * 2).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(n_kv * hd * n_ctx).astype(np.float16).view(np.uint16)
    kq = float(np.float32(1.0 / np.sqrt(np.float32(hd))))
    want = oracle.attn_decode(q, k, v, n_head, n_kv, hd, n_ctx, pos, kq)[0]
    hg = _HipGraph()
    bufs = []
    try:
        qd, kd, vd = dev.to_device(q), dev.to_device(k), dev.to_device(v)
        nan = np.full(n_head * hd, np.nan, np.float32)
        oe, og = dev.to_device(nan), dev.to_device(nan)
        bufs = [qd, kd, vd, oe, og]
        args = (qd.ptr, kd.ptr, vd.ptr, n_head, n_kv, hd, n_ctx, pos, kq)
        dev.attn_decode_dev(*args, oe.ptr, None, None, hg.stream.value)
        dev.synchronize()
        assert np.array_equal(bits(oe.to_host(np.float32, n_head * hd)), bits(want))
        hg.begin()
        dev.attn_decode_dev(*args, og.ptr, None, None, hg.stream.value)
        hg.end()
        for _ in range(3):
            og.fill(nan)
            hg.replay()
            assert np.array_equal(bits(og.to_host(np.float32, n_head * hd)), bits(want))
            oe.fill(nan)
            dev.attn_decode_dev(*args, oe.ptr, None, None, hg.stream.value)
            dev.synchronize()
            assert np.array_equal(bits(oe.to_host(np.float32, n_head * hd)), bits(want))
    finally:
        hg.close()
        for b in bufs:
            b.free()
