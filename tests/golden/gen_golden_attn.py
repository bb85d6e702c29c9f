"""Write tests/golden/golden_attn_v1.npz from the compiled reference (oracle/_ref).

Decode attention over an f16 KV cache as the reference's attn_head computes
it (reference engine.c:90-147), composed in oracle/siq.py (Reference.attn_decode)
from the reference's own compiled f16 conversion, AVX2 f16 dot and softmax.
The fixtures are data only: seeded queries and caches, the shape of each
case, and the reference's scores, f16 probabilities and outputs.

Cases cover the dot's 32-element body with and without a tail (head dims
64, 80, 128), the softmax's 8-groups with and without a tail, position 0,
grouped-query heads, and score spreads wide enough to reach the exp
polynomial's scaled (|n| > 126) and saturated (|n| > 192) branches.

Run in a container where oracle/_ref is built:
    python tests/golden/gen_golden_attn.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import siq  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_attn_v1.npz")

# (n_head, n_head_kv, head_dim, n_ctx, pos, key scale)
CASES = [
    (8, 2, 64, 72, 70, 1.0),
    (4, 4, 80, 40, 32, 1.0),
    (4, 1, 128, 16, 0, 1.0),
    (6, 2, 64, 48, 47, 40.0),
    (2, 1, 128, 260, 257, 3.0),
]


def main():
    ref = siq.Reference.load()
    if ref is None:
        sys.exit("oracle/_ref is not built; run `make -C oracle ref` where /root/reference exists")
    assert ref.avx2, "the golden outputs follow the reference's AVX2 dispatch"
    rng = np.random.default_rng(20261201)
    data = {"cases": np.array(CASES, dtype=np.float64)}
    for i, (n_head, n_kv, hd, n_ctx, pos, kscale) in enumerate(CASES):
        q = rng.standard_normal(n_head * hd).astype(np.float32)
        k = (rng.standard_normal(n_kv * n_ctx * hd) * kscale).astype(np.float16).view(np.uint16)
        v = rng.standard_normal(n_kv * hd * n_ctx).astype(np.float16).view(np.uint16)
        kq = np.float32(1.0 / np.sqrt(np.float32(hd)))
        out, sc, pr = ref.attn_decode(q, k, v, n_head, n_kv, hd, n_ctx, pos, float(kq))
        data.update({f"q{i}": q, f"k{i}": k, f"v{i}": v, f"kq{i}": np.float32(kq),
                     f"out{i}": out, f"scores{i}": sc, f"probs{i}": pr})
    np.savez_compressed(OUT, **data)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
