"""Write tests/golden/golden_v1.npz from the compiled reference (oracle/_ref).

The fixtures are data only: seeded inputs and the outputs the reference's own
kernels produce for them (f16 conversion, Q8_K and Q8_0 quantizers,
dequantization, and every dot product in both the AVX2 path production
dispatches to and the portable scalar path). The scalar values come from a
child process started with SI_SCALAR=1 (the reference picks its kernels once
per process, reference kernels.c:56-85).

Run in a container where oracle/_ref is built:
    python tests/golden/gen_golden.py
"""
from __future__ import annotations

import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import siq  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_v1.npz")
N = 1024        # elements per row (4 super-blocks), as in reference tests/test_kernels.c:89
ROWS = 4        # weight rows per format


def activation_rows(rng):
    """f32 rows hitting the quantizer edge cases."""
    rows = []
    rows.append(rng.standard_normal(N).astype(np.float32))
    rows.append(rng.uniform(-1, 1, N).astype(np.float32))
    rows.append((rng.standard_normal(N) * 1e-3).astype(np.float32))
    rows.append((rng.standard_normal(N) * 3e4).astype(np.float32))
    z = rng.standard_normal(N).astype(np.float32)
    z[:256] = 0.0
    z[300:332] = 0.0
    rows.append(z)
    t = np.round(rng.standard_normal(N) * 4).astype(np.float32)
    rows.append(t)
    h = rng.uniform(-1, 1, N).astype(np.float32)
    h[7], h[100], h[300], h[301] = 5.0, -5.0, -3.0, 3.0
    rows.append(h)
    s = (rng.standard_normal(N) * 1e-30).astype(np.float32)
    rows.append(s)
    return np.stack(rows)


def weight_rows(rng, wtype):
    """Random block bytes with tamed f16 scales (reference tests/test_kernels.c:91-140)."""
    be, bb = siq.GEOM[wtype]
    if wtype == siq.F16:
        return rng.uniform(-1, 1, (ROWS, N)).astype(np.float16).view(np.uint8)
    b = rng.integers(0, 256, size=(ROWS * (N // be), bb), dtype=np.uint8)
    d = (0.01 * (1.0 + rng.integers(0, 100, b.shape[0]) / 100.0)).astype(np.float16)
    dmin = (0.001 * rng.integers(0, 100, b.shape[0]) / 100.0).astype(np.float16)
    off = {siq.Q4_0: (0,), siq.Q5_0: (0,), siq.Q8_0: (0,), siq.Q2_K: (80, 82),
           siq.Q3_K: (108,), siq.Q4_K: (0, 2), siq.Q5_K: (0, 2), siq.Q6_K: (208,)}[wtype]
    b[:, off[0]:off[0] + 2] = d.view(np.uint8).reshape(-1, 2)
    if len(off) > 1:
        b[:, off[1]:off[1] + 2] = dmin.view(np.uint8).reshape(-1, 2)
    return b.reshape(ROWS, -1)


def main_scalar(path_in, path_out):
    """Child process (SI_SCALAR=1): scalar-path quantizer and dots."""
    ref = siq.Reference()
    assert not ref.avx2
    data = dict(np.load(path_in))
    out = {"q80_scalar": np.stack([ref.quant_q8_0(r, simd=False) for r in data["act"]])}
    for wt in siq.WEIGHT_TYPES:
        name = siq.NAMES[wt]
        W = data[f"w_{name}"]
        xq = data[f"xq_{name}"]
        out[f"dot_scalar_{name}"] = np.array(
            [ref.dot(wt, N, W[r], xq, simd=False) for r in range(ROWS)], np.float32)
    np.savez(path_out, **out)


def main():
    ref = siq.Reference.load()
    if ref is None:
        sys.exit("oracle/_ref is not built; run `make -C oracle ref` where /root/reference exists")
    assert ref.avx2, "the golden AVX2 outputs need an AVX2 host"
    rng = np.random.default_rng(20260101)
    data = {}
    # f16: random magnitudes across the whole range, plus the edges
    f = np.concatenate([rng.standard_normal(2000) * 100, rng.standard_normal(1000) * 1e-5,
                        rng.standard_normal(500) * 1e-7,
                        [65504, 65519.99, 65520, 1e10, -1e10, 6e-8, 2.98e-8, 5.96e-8, 0.0, -0.0,
                         np.inf, -np.inf]]).astype(np.float32)
    data["f16_in"] = f
    data["f16_out"] = ref.f16(f)
    act = activation_rows(rng)
    data["act"] = act
    data["q8K"] = np.stack([ref.quant_q8_K(r) for r in act])
    data["q80_simd"] = np.stack([ref.quant_q8_0(r, simd=True) for r in act])
    for wt in siq.WEIGHT_TYPES:
        name = siq.NAMES[wt]
        W = weight_rows(rng, wt)
        x = rng.uniform(-1, 1, N).astype(np.float32)
        pair = siq.PAIR[wt]
        if pair == siq.Q8_K:
            xq = ref.quant_q8_K(x)
        elif pair == siq.Q8_0:
            xq = ref.quant_q8_0(x, simd=True)
        else:
            xq = ref.f16(x).view(np.uint8)
        data[f"w_{name}"] = W
        data[f"x_{name}"] = x
        data[f"xq_{name}"] = xq
        data[f"deq_{name}"] = np.stack([ref.dequant(wt, W[r], N) for r in range(ROWS)])
        data[f"dot_avx2_{name}"] = np.array([ref.dot(wt, N, W[r], xq, simd=True)
                                             for r in range(ROWS)], np.float32)
    tmp_in, tmp_out = OUT + ".in.npz", OUT + ".scalar.npz"
    np.savez(tmp_in, **data)
    env = dict(os.environ, SI_SCALAR="1")
    subprocess.run([sys.executable, __file__, "--scalar", tmp_in, tmp_out], check=True, env=env)
    data.update(dict(np.load(tmp_out)))
    os.remove(tmp_in)
    os.remove(tmp_out)
    np.savez_compressed(OUT, **data)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    if len(sys.argv) == 4 and sys.argv[1] == "--scalar":
        main_scalar(sys.argv[2], sys.argv[3])
    else:
        main()
