"""Seeded synthetic GGUF weight blocks with the field distributions of the
benchmark configurations (every quant field uniform over its bit width,
f16 block scales uniform in a stated range), plus the config table.

Block layouts are those of the reference (include/siphon/quant.h:31-90);
the byte offsets of the f16 scale fields are listed in F16_FIELDS.
"""
from __future__ import annotations

import numpy as np

from . import F16, F32, GEOM, Q2_K, Q3_K, Q4_0, Q4_K, Q5_0, Q5_K, Q6_K, Q8_0

# byte offsets of the f16 scale fields inside each block
F16_FIELDS = {Q4_0: (0,), Q5_0: (0,), Q8_0: (0,), Q2_K: (80, 82), Q3_K: (108,),
              Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208,)}


def _f16_uniform(rng, lo, hi, n):
    return rng.uniform(lo, hi, n).astype(np.float16).view(np.uint8).reshape(n, 2)


def make_weights(wtype: int, n_out: int, n_in: int, rng: np.random.Generator,
                 d_range=(1e-4, 4e-3), dmin_range=None) -> np.ndarray:
    """GGUF bytes of a [n_out x n_in] matrix; returns uint8 [n_out, row_bytes].

    Q6_K block scales are int8 uniform in [-32, 31] and Q8_0 quants uniform in
    [-127, 127] (the benchmark's stated distributions); all other quant and
    sub-scale bytes are uniform random. F16 and F32 weights are uniform in
    [-0.05, 0.05].
    """
    be, bb = GEOM[wtype]
    if wtype == F32:
        w = rng.uniform(-0.05, 0.05, n_out * n_in).astype(np.float32)
        return w.view(np.uint8).reshape(n_out, n_in * 4)
    if wtype == F16:
        w = rng.uniform(-0.05, 0.05, n_out * n_in).astype(np.float16)
        return w.view(np.uint8).reshape(n_out, n_in * 2)
    nblk = n_out * (n_in // be)
    b = rng.integers(0, 256, size=(nblk, bb), dtype=np.uint8)
    if wtype == Q6_K:
        b[:, 192:208] = rng.integers(-32, 32, size=(nblk, 16), dtype=np.int8).view(np.uint8)
    if wtype == Q8_0:
        b[:, 2:34] = rng.integers(-127, 128, size=(nblk, 32), dtype=np.int8).view(np.uint8)
    offs = F16_FIELDS[wtype]
    b[:, offs[0]:offs[0] + 2] = _f16_uniform(rng, *d_range, nblk)
    if len(offs) > 1:
        b[:, offs[1]:offs[1] + 2] = _f16_uniform(rng, *(dmin_range or d_range), nblk)
    return b.reshape(n_out, (n_in // be) * bb)


def make_activations(n: int, rng: np.random.Generator, m: int | None = None) -> np.ndarray:
    shape = (n,) if m is None else (m, n)
    return rng.standard_normal(shape).astype(np.float32)


# Benchmark configurations (matrix sets); each entry (name, type, n_out, n_in).
LLAMA3_8B_LAYER = [
    ("wq", Q4_K, 4096, 4096), ("wk", Q4_K, 1024, 4096), ("wv", Q6_K, 1024, 4096),
    ("wo", Q4_K, 4096, 4096), ("ffn_gate", Q4_K, 14336, 4096),
    ("ffn_up", Q4_K, 14336, 4096), ("ffn_down", Q6_K, 4096, 14336),
]

CONFIG0 = [("ffn_gate", Q4_K, 5632, 2048)]
# Q6_K 151936 x 896 cannot exist (896 is not a multiple of 256): the head runs
# at 151936 x 1024 in Q6_K, and in Q8_0 at the exact 151936 x 896 shape.
CONFIG1 = [("ffn_q8_0", Q8_0, 4864, 896), ("head_q6_K", Q6_K, 151936, 1024),
           ("head_q8_0", Q8_0, 151936, 896)]
CONFIG4_SHAPES = [("attn", 5120, 5120), ("kv", 1024, 5120), ("ffn_up", 27648, 5120),
                  ("ffn_down", 5120, 27648)]
CONFIG4_TYPES = [Q2_K, Q3_K, Q5_K, Q5_0, F16]
EXTRA_Q4_0 = [("q4_0_cfg0_shape", Q4_0, 5632, 2048)]
