"""The batched prefill (siphon_amd/host/si_prefill.c) against the reference
engine's token loop: one si_engine_forward per prompt token (reference
cmd_run.c:275-283, engine.c:288-398), both in one process.

The reference engine and model loader are compiled from the reference's own
sources into oracle/_ref (oracle/Makefile, target `engine`, a test-only
checker) and linked with the repository's prefill and hip adapter. The test
models are GGUF files written by tests/gguf_writer.py: two layers of a
llama (NORM RoPE, Q4_K_M-style types in layer 0, every other served type in
layer 1, an F16 norm, RoPE frequency factors) and a qwen2 (NEOX RoPE, q/k/v
biases), grouped-query attention (8 query heads on 2 KV heads).

CPU tests pin the prefill's per-row steps bit for bit: with the reference
CPU backend behind the gemm slot (one gemv per row), the prefill's last
logits, its whole KV cache and the decode steps after it are bit-identical
to the token loop's, for prompts shorter than a pass, over two passes of
SI_PREFILL_ROWS, and split over two prefill calls.

GPU tests put every layer on the hip backend (si_backend_hip_place at load,
the layers' gemm slot on the matrix cores) and check:
- every gemm call the prefill made, on its recorded inputs, against the
  oracle's per-row dots within the path's bar |gpu - ref| <= 1e-5 *
  sum|terms| + 1e-6 (every output);
- end to end, against the CPU token loop: every cached K and V value within
  4 f16 spacings of its head vector's largest magnitude, at most 1 % of
  them moved at all (the GEMMs round their f32 sums in another order, which
  moves an f16 rounding where a value sits near a rounding boundary, and
  attention passes such moves on to the next layer; a value near zero after
  cancellation can move by many of its own, much finer, spacings), and the
  last logits within 1e-4 of the largest logit.
"""
import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth
from siphon_amd.build import HIP_SO

from . import gguf_writer as gw

N_EMBD, N_HEAD, N_KV_HEAD, N_FF, N_VOCAB = 512, 8, 2, 1536, 1000
HEAD_DIM = N_EMBD // N_HEAD

LAYER_TYPES = [
    # layer 0: the Q4_K_M mix; layer 1: every other type the backend serves
    {"attn_q": sa.Q4_K, "attn_k": sa.Q4_K, "attn_v": sa.Q6_K, "attn_output": sa.Q4_K,
     "ffn_gate": sa.Q4_K, "ffn_up": sa.Q4_K, "ffn_down": sa.Q6_K},
    {"attn_q": sa.Q8_0, "attn_k": sa.Q4_0, "attn_v": sa.Q5_0, "attn_output": sa.F16,
     "ffn_gate": sa.Q2_K, "ffn_up": sa.Q3_K, "ffn_down": sa.Q5_K},
]
SHAPES = {"attn_q": (N_EMBD, N_EMBD), "attn_k": (N_KV_HEAD * HEAD_DIM, N_EMBD),
          "attn_v": (N_KV_HEAD * HEAD_DIM, N_EMBD), "attn_output": (N_EMBD, N_EMBD),
          "ffn_gate": (N_FF, N_EMBD), "ffn_up": (N_FF, N_EMBD), "ffn_down": (N_EMBD, N_FF)}


def _f32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint8)


def write_model(path, arch="llama", seed=7):
    """A two-layer model in GGUF; returns {tensor name: bytes}."""
    rng = np.random.default_rng(seed)
    kvs = [("general.architecture", gw.STRING, arch),
           (f"{arch}.block_count", gw.U32, 2),
           (f"{arch}.context_length", gw.U32, 4096),
           (f"{arch}.embedding_length", gw.U32, N_EMBD),
           (f"{arch}.feed_forward_length", gw.U32, N_FF),
           (f"{arch}.attention.head_count", gw.U32, N_HEAD),
           (f"{arch}.attention.head_count_kv", gw.U32, N_KV_HEAD),
           (f"{arch}.attention.layer_norm_rms_epsilon", gw.F32, 1e-5),
           (f"{arch}.rope.freq_base", gw.F32, 500000.0 if arch == "llama" else 1000000.0)]
    tensors, blobs = [], {}

    def add(name, wt, dims, data):
        blobs[name] = data
        tensors.append((name, wt, dims, data.reshape(-1)))

    add("token_embd.weight", sa.Q4_K, [N_EMBD, N_VOCAB],
        synth.make_weights(sa.Q4_K, N_VOCAB, N_EMBD, rng))
    add("output_norm.weight", sa.F32, [N_EMBD], _f32(1.0 + 0.1 * rng.standard_normal(N_EMBD)))
    add("output.weight", sa.Q6_K, [N_EMBD, N_VOCAB],
        synth.make_weights(sa.Q6_K, N_VOCAB, N_EMBD, rng, d_range=(1e-4, 2e-3)))
    if arch == "llama":
        # llama3-style frequency factors (RoPE divides each pair's angle)
        add("rope_freqs.weight", sa.F32, [HEAD_DIM // 2],
            _f32(np.linspace(1.0, 8.0, HEAD_DIM // 2)))
    for il, types in enumerate(LAYER_TYPES):
        norm = 1.0 + 0.1 * rng.standard_normal(N_EMBD)
        if il == 1 and arch == "llama":  # a norm the engine dequantizes (F16)
            add(f"blk.{il}.attn_norm.weight", sa.F16, [N_EMBD],
                np.ascontiguousarray(norm, np.float16).view(np.uint8))
        else:
            add(f"blk.{il}.attn_norm.weight", sa.F32, [N_EMBD], _f32(norm))
        add(f"blk.{il}.ffn_norm.weight", sa.F32, [N_EMBD],
            _f32(1.0 + 0.1 * rng.standard_normal(N_EMBD)))
        for name, wt in types.items():
            n_out, n_in = SHAPES[name]
            d_range = (1e-4, 2e-3) if wt == sa.Q6_K else (1e-4, 4e-3)
            add(f"blk.{il}.{name}.weight", wt, [n_in, n_out],
                synth.make_weights(wt, n_out, n_in, rng, d_range=d_range))
        if arch == "qwen2":
            for name in ("attn_q", "attn_k", "attn_v"):
                add(f"blk.{il}.{name}.bias", sa.F32, [SHAPES[name][0]],
                    _f32(0.5 * rng.standard_normal(SHAPES[name][0])))
    gw.write_gguf(str(path), kvs, tensors)
    return blobs


@pytest.fixture(scope="module")
def lib():
    from tests import engine_py
    import os
    if not os.path.exists(engine_py.SO):
        pytest.skip("oracle/_ref engine checker not built (needs /root/reference at build time)")
    return engine_py.RefEngineLib()


@pytest.fixture(scope="module", params=["llama", "qwen2"])
def model(request, lib, tmp_path_factory):
    path = tmp_path_factory.mktemp(request.param) / "model.gguf"
    write_model(path, request.param)
    m = lib.load(path)
    yield request.param, m
    lib.L.re_model_free(m)


def _tokens(n, seed=3):
    return np.random.default_rng(seed).integers(0, N_VOCAB, n, dtype=np.uint32)


def _bits(a):
    return a.view(np.uint32) if a.dtype == np.float32 else a


def test_mirror_layout_matches_reference(lib):
    """Every size and field offset the prefill and adapter assume (their
    mirror of model.h, engine.h and tensor.h plus the gemm slot) is the
    reference build's."""
    ref, mirror = lib.layouts()
    assert len(ref) == len(mirror) > 40
    assert ref == mirror


@pytest.mark.parametrize("n,split", [(37, None), (600, None), (50, 20)])
def test_prefill_cpu_bit_identical_to_token_loop(lib, model, n, split):
    """With the reference CPU backend behind the gemm slot, the prefill is
    the token loop: last logits, K and V caches and three decode steps
    afterwards bit for bit (600 tokens: two passes of 512 and 88 rows;
    split: two prefill calls, the second starting at position 20)."""
    arch, m = model
    toks = _tokens(n + 3)
    e_ref = lib.engine(m, 1024)
    e_pre = lib.engine(m, 1024)
    try:
        lib.L.re_layers_cpu(m)
        want = lib.forward_loop(e_ref, toks[:n])
        lib.L.re_layers_cpu_gemm(m)
        if split:
            assert lib.prefill(e_pre, toks[:split]) is not None, lib.errstr()
            assert lib.L.re_n_pos(e_pre) == split
            got = lib.prefill(e_pre, toks[split:n])
        else:
            got = lib.prefill(e_pre, toks[:n])
        assert got is not None, lib.errstr()
        assert lib.L.re_n_pos(e_pre) == lib.L.re_n_pos(e_ref) == n
        assert np.array_equal(_bits(got), _bits(want)), arch
        k0, v0 = lib.caches(e_ref, n)
        k1, v1 = lib.caches(e_pre, n)
        assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
        # decoding goes on from the same state
        lib.L.re_layers_cpu(m)
        for t in toks[n:]:
            a = lib.forward_loop(e_ref, [t])
            b = lib.forward_loop(e_pre, [t])
            assert np.array_equal(_bits(a), _bits(b))
    finally:
        lib.L.re_layers_cpu(m)
        lib.L.re_engine_free(e_ref)
        lib.L.re_engine_free(e_pre)


def test_prefill_without_gemm_slot(lib, model):
    """A layer backend with no gemm slot gets one gemv per row: same bits."""
    _, m = model
    toks = _tokens(21, seed=5)
    e_ref, e_pre = lib.engine(m, 64), lib.engine(m, 64)
    try:
        lib.L.re_layers_cpu(m)
        want = lib.forward_loop(e_ref, toks)
        lib.L.re_layers_cpu_nogemm(m)
        got = lib.prefill(e_pre, toks)
        assert got is not None and np.array_equal(_bits(got), _bits(want))
    finally:
        lib.L.re_layers_cpu(m)
        lib.L.re_engine_free(e_ref)
        lib.L.re_engine_free(e_pre)


def test_prefill_errors(lib, model):
    """Too long a prompt for the context, a token outside the vocabulary
    and an empty prompt: NULL with a message, nothing run."""
    _, m = model
    e = lib.engine(m, 16)
    try:
        lib.L.re_layers_cpu_gemm(m)
        assert lib.prefill(e, _tokens(17)) is None
        assert "context full" in lib.errstr()
        assert lib.L.re_n_pos(e) == 0
        bad = _tokens(4)
        bad[2] = N_VOCAB
        assert lib.prefill(e, bad) is None
        assert "vocabulary" in lib.errstr()
        assert lib.prefill(e, np.zeros(0, np.uint32)) is None
        assert lib.L.re_n_pos(e) == 0
        assert lib.prefill(e, _tokens(16)) is not None  # exactly fills the context
        assert lib.L.re_n_pos(e) == 16
    finally:
        lib.L.re_layers_cpu(m)
        lib.L.re_engine_free(e)


def _vector_ulps(a, b, axis):
    """|a - b| in units of the f16 spacing at the largest magnitude of each
    head vector (f16 bit patterns in; `axis` runs over the vector)."""
    fa = a.view(np.float16).astype(np.float64)
    fb = b.view(np.float16).astype(np.float64)
    top = np.max(np.abs(fa), axis=axis, keepdims=True).astype(np.float16)
    return np.abs(fa - fb) / np.spacing(top).astype(np.float64)


@pytest.mark.gpu
@pytest.mark.parametrize("n", [40, 600])
def test_prefill_hip_matches_token_loop(lib, oracle, model, n):
    """Every layer on the hip backend: each recorded gemm within the dot's
    bar against the oracle, and the end result against the CPU token loop
    (40 tokens: the small- and mid-M GEMMs; 600: passes of 512 and 88 rows,
    the M >= 384 Q4_K kernel)."""
    arch, m = model
    rc, be = lib.hip_open(HIP_SO)
    assert rc == 0, lib.errstr()
    toks = _tokens(n, seed=11)
    e_ref, e_pre = lib.engine(m, 1024), lib.engine(m, 1024)
    try:
        lib.L.re_layers_cpu(m)
        want = lib.forward_loop(e_ref, toks)
        lib.L.re_rec_clear()
        assert lib.L.re_layers_hip(m, be, 0, 1) == 0, lib.errstr()
        got = lib.prefill(e_pre, toks)
        assert got is not None, lib.errstr()
        calls = lib.recorded()
        assert len(calls) == 7 * 2 * (1 if n <= 512 else 2)
        for wt, n_in, n_out, M, data, X, Y in calls:
            import ctypes
            W = np.frombuffer(ctypes.string_at(data, n_out * (n_in // sa.GEOM[wt][0]) *
                                               sa.GEOM[wt][1]), np.uint8).reshape(n_out, -1)
            R, L1 = oracle.gemm(wt, W, n_out, n_in, X)
            err = np.abs(Y.astype(np.float64) - R)
            assert np.all(err <= 1e-5 * L1 + 1e-6), (arch, sa.NAMES[wt], M, float(np.max(err / L1)))
        k0, v0 = lib.caches(e_ref, n)
        k1, v1 = lib.caches(e_pre, n)
        ku, vu = _vector_ulps(k0, k1, 3), _vector_ulps(v0, v1, 2)
        moved = np.mean(np.concatenate([(k0 != k1).ravel(), (v0 != v1).ravel()]))
        print(f"{arch} n={n}: K max {ku.max():.2f}, V max {vu.max():.2f} ulps of the head "
              f"vector's largest value; {moved:.2e} of the cache moved; logits max |d| "
              f"{np.max(np.abs(got - want)):.3e} of {np.max(np.abs(want)):.3e}")
        assert ku.max() <= 4 and vu.max() <= 4 and moved <= 0.01
        assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want))
    finally:
        lib.L.re_layers_cpu(m)
        lib.L.re_rec_clear()
        lib.L.re_engine_free(e_ref)
        lib.L.re_engine_free(e_pre)
        lib.L.re_hip_close(be)
