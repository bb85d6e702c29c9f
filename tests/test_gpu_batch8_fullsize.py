"""The batched decode step the benchmark times (bench.py decode_batch8: 8
sequences through the Llama-3-8B Q4_K_M layer, engine.c:317-319, 368,
375-378 run for 8 rows at once) at its full shapes, on the default dispatch,
every output against the oracle's per-row dots (reference kernels.c:349-410
for Q4_K, 480-523 for Q6_K) to the path's bar |gpu - ref| <= 1e-5 *
sum|terms| + 1e-6:
- each matrix alone through sihip_gemm_dev: Q4_K 14336 x 4096 (gate, up),
  4096 x 4096 (wq, wo), 1024 x 4096 (wk), Q6_K 1024 x 4096 (wv);
- the q/k/v and gate/up groups through sihip_gemm_multi_dev, as the step
  makes them, twice (the second call with other rows: nothing stale).
The rows start with the quantizer's edge vectors (ties, zeros, huge and
tiny values)."""
import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth

from .test_gpu_gemm import _rows
from .test_gpu_gemm_multi import _run
from .test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu

M = 8
K = 4096
SINGLE = [(sa.Q4_K, 14336), (sa.Q4_K, 4096), (sa.Q4_K, 1024), (sa.Q6_K, 1024)]


def _weights(rng, mats):
    return [synth.make_weights(wt, n_out, K, rng,
                               d_range=(1e-4, 2e-3) if wt == sa.Q6_K else (1e-4, 4e-3))
            for wt, n_out in mats]


@pytest.mark.parametrize("wt,n_out", SINGLE, ids=[f"{sa.NAMES[t]}-{n}x{K}" for t, n in SINGLE])
def test_batch8_single_fullsize(dev, oracle, wt, n_out):
    print(f"batch8 gemm_dev {sa.NAMES[wt]} {n_out}x{K}", flush=True)
    rng = np.random.default_rng(n_out + wt)
    (W,) = _weights(rng, [(wt, n_out)])
    w = dev.upload(wt, n_out, K, W)
    try:
        X = _rows(rng, M, K)
        (Y,) = _run(dev, [w], X, multi=False)
        ref, L1 = oracle.gemm(wt, W, n_out, K, X)
        assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                     f"M=8 {sa.NAMES[wt]} {n_out}x{K}")
    finally:
        w.free()


GROUPS = [("qkv", [(sa.Q4_K, 4096), (sa.Q4_K, 1024), (sa.Q6_K, 1024)]),
          ("gate_up", [(sa.Q4_K, 14336), (sa.Q4_K, 14336)])]


@pytest.mark.parametrize("label,mats", GROUPS, ids=[g[0] for g in GROUPS])
def test_batch8_group_fullsize(dev, oracle, label, mats):
    print(f"batch8 gemm_multi_dev {label}", flush=True)
    rng = np.random.default_rng(len(label))
    Ws = _weights(rng, mats)
    ws = [dev.upload(wt, n_out, K, W) for (wt, n_out), W in zip(mats, Ws)]
    try:
        for call in range(2):
            X = _rows(rng, M, K)
            if call:
                X = X[::-1].copy()
            Ys = _run(dev, ws, X)
            for i, ((wt, n_out), W, Y) in enumerate(zip(mats, Ws, Ys)):
                ref, L1 = oracle.gemm(wt, W, n_out, K, X)
                assert_close(Y.reshape(-1), ref.reshape(-1).astype(np.float64), L1.reshape(-1),
                             f"M=8 {label} call {call} weight {i} ({sa.NAMES[wt]} {n_out}x{K})")
    finally:
        for w in ws:
            w.free()
