"""Device-resident weights from an mmap'd GGUF file: the model loader's path
(reference gguf.c:282-408 si_gguf_open -> backend.c:144-176
si_tensor_from_gguf -> si_backend_hip_place) and the routed engine's calls
through each tensor's backend (engine.c:302-303, 317-378, 393-394 with the
embedding and head taken from m->tok_embd.be and m->output.be).

The file is written by tests/gguf_writer.py and opened by the reference's
own parser, compiled from its sources into oracle/_ref (a test-only
checker); the tensor views are the ones the reference loader makes.

CPU tests pin the writer and the view layout: every tensor's view points
into the mapping at the writer's offset, with the file's type, dimensions
and byte count, and the reference CPU backend's row_to_f32 and gemv on the
view agree with the oracle on the bytes written. GPU tests place the views
on the device and check gemv, gemm and row_to_f32 through the adapter
against the reference CPU backend on the same mmap.
"""
import ctypes

import numpy as np
import pytest

import siphon_amd as sa
from siphon_amd import synth
from siphon_amd.build import HIP_SO

from . import gguf_writer as gw
from .test_gpu_parity import assert_close

SI_OK, SI_EINVAL = 0, -5
N_EMBD, N_FF, N_KV, N_VOCAB = 512, 1536, 128, 1000

# a one-layer Llama-style Q4_K_M model, plus a second layer holding every
# other weight type the backend serves (ggml names; dims innermost first)
LAYOUT = [
    ("token_embd.weight", sa.Q4_K, N_VOCAB, N_EMBD),
    ("blk.0.attn_q.weight", sa.Q4_K, N_EMBD, N_EMBD),
    ("blk.0.attn_k.weight", sa.Q4_K, N_KV, N_EMBD),
    ("blk.0.attn_v.weight", sa.Q6_K, N_KV, N_EMBD),
    ("blk.0.attn_output.weight", sa.Q4_K, N_EMBD, N_EMBD),
    ("blk.0.ffn_gate.weight", sa.Q4_K, N_FF, N_EMBD),
    ("blk.0.ffn_up.weight", sa.Q4_K, N_FF, N_EMBD),
    ("blk.0.ffn_down.weight", sa.Q6_K, N_EMBD, N_FF),
    ("blk.1.attn_q.weight", sa.Q8_0, N_EMBD, N_EMBD),
    ("blk.1.attn_k.weight", sa.Q4_0, N_KV, N_EMBD),
    ("blk.1.attn_v.weight", sa.Q5_0, N_KV, N_EMBD),
    ("blk.1.attn_output.weight", sa.F16, N_EMBD, N_EMBD),
    ("blk.1.ffn_gate.weight", sa.Q2_K, N_FF, N_EMBD),
    ("blk.1.ffn_up.weight", sa.Q3_K, N_FF, N_EMBD),
    ("blk.1.ffn_down.weight", sa.Q5_K, N_EMBD, N_FF),
    ("blk.1.ffn_norm.weight", sa.F32, 1, N_EMBD),
    ("output.weight", sa.Q6_K, N_VOCAB, N_EMBD),
    ("output_norm.weight", sa.F32, 1, N_EMBD),
]


def _model_file(path, alignment=32, version=3, seed=11):
    rng = np.random.default_rng(seed)
    kvs = [("general.architecture", gw.STRING, "llama"),
           ("llama.embedding_length", gw.U32, N_EMBD),
           ("llama.feed_forward_length", gw.U32, N_FF),
           ("llama.block_count", gw.U32, 2),
           ("llama.attention.layer_norm_rms_epsilon", gw.F32, 1e-5),
           ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, [f"t{i}" for i in range(8)]))]
    if alignment != 32:
        kvs.append(("general.alignment", gw.U32, alignment))
    weights, tensors = {}, []
    for name, wt, n_out, n_in in LAYOUT:
        W = synth.make_weights(wt, n_out, n_in, rng)
        weights[name] = W
        dims = [n_in] if n_out == 1 else [n_in, n_out]
        tensors.append((name, wt, dims, W.reshape(-1)))
    offsets = gw.write_gguf(str(path), kvs, tensors, alignment=alignment, version=version)
    return weights, offsets


def _view(ref, g, name, be=None):
    from tests.host_py import SiTensor
    t = SiTensor()
    rc = ref.gguf_tensor(g, name, be, ctypes.addressof(t))
    assert rc == SI_OK, (name, rc)
    return t


@pytest.mark.parametrize("alignment,version", [(32, 3), (64, 3), (32, 2)])
def test_reference_loader_views(ref, oracle, tmp_path, alignment, version):
    """The reference parser opens the written file; each view is the
    loader's (type, dims, bytes, HOST, CPU backend) and points into the
    mapping at the writer's offset; the reference's row_to_f32 and gemv on
    the view agree with the oracle on the bytes written."""
    from tests.host_py import SI_LOC_HOST, SiTensor
    assert ref.tensor_size() == ctypes.sizeof(SiTensor)
    path = tmp_path / "model.gguf"
    weights, offsets = _model_file(path, alignment, version)
    g = ref.gguf_open(str(path))
    try:
        assert ref.gguf_alignment(g) == alignment
        rng = np.random.default_rng(5)
        for name, wt, n_out, n_in in LAYOUT:
            t = _view(ref, g, name)
            assert t.type == wt and t.loc == SI_LOC_HOST
            assert list(t.ne) == ([n_in, 0, 0, 0] if n_out == 1 else [n_in, n_out, 0, 0])
            assert t.n_bytes == weights[name].nbytes and t.n_elems == n_in * n_out
            assert ref.gguf_map_offset(g, t.data) == offsets[name]
            W = weights[name]
            for row in {0, n_out - 1}:
                got = ref.tensor_row(ctypes.addressof(t), row, n_in)
                want = oracle.dequant(wt, W[row], n_in)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, row)
            if n_out > 1:
                x = rng.standard_normal(n_in).astype(np.float32)
                y = ref.tensor_gemv(ctypes.addressof(t), x, n_out)
                want, l1 = oracle.gemv(wt, W, n_out, n_in, x)
                assert_close(y, want.astype(np.float64), l1, f"reference gemv on view {name}")
    finally:
        ref.gguf_close(g)


def test_reference_loader_rejects_truncated_file(ref, tmp_path):
    path = tmp_path / "cut.gguf"
    _model_file(path)
    data = path.read_bytes()
    path.write_bytes(data[:-4096])
    with pytest.raises(OSError, match="exceeds data section"):
        ref.gguf_open(str(path))


def test_harness_view_layout_matches_reference(ref):
    """The adapter's si_tensor (si_mirror.h) has the reference's size, so a
    view made by the reference loader is read field for field."""
    from tests import host_py
    assert host_py.Harness().tensor_size() == ref.tensor_size()


@pytest.fixture(scope="module")
def hip_backend():
    from tests import host_py
    h = host_py.Harness()
    rc, be = h.open(HIP_SO)
    if rc != 0:
        pytest.skip(f"no device: {h.errstr()}")
    yield h, be
    h.close(be)


@pytest.mark.gpu
def test_gguf_to_device_end_to_end(ref, oracle, hip_backend, tmp_path):
    """Load-time placement and the routed engine's calls:
    - views made with the hip backend assigned (si_tensor_from_gguf(g, t,
      be_hip, &view)); every 2-D weight but the embedding is placed
      (si_backend_hip_place): loc becomes SI_LOC_DEVICE, be the hip backend,
      data stays the mmap pointer; placing again uploads nothing;
    - gemv through each view's own backend matches the reference CPU
      backend on the same mmap (to the bar, against the oracle's sum of
      |terms|), and so does gemm at M = 5, row by row;
    - row_to_f32 through the views (the embedding lookup stays on the
      mmap'd rows) is bit-identical to the reference's."""
    from tests.host_py import SI_LOC_DEVICE, SI_LOC_HOST
    h, be = hip_backend
    path = tmp_path / "model.gguf"
    weights, offsets = _model_file(path, alignment=64)
    g = ref.gguf_open(str(path))
    try:
        n0, _ = h.weights(be)
        views = {name: _view(ref, g, name, be) for name, *_ in LAYOUT}
        placed = [name for name, wt, n_out, n_in in LAYOUT
                  if n_out > 1 and name != "token_embd.weight"]
        for name in placed:
            t = views[name]
            mmap_ptr = t.data
            assert h.place(be, t) == SI_OK, (name, h.errstr())
            assert t.loc == SI_LOC_DEVICE and t.be == be and t.data == mmap_ptr
            assert ref.gguf_map_offset(g, t.data) == offsets[name]
        n1, dev_bytes = h.weights(be)
        assert n1 == n0 + len(placed) and dev_bytes > 0
        for name in placed:
            assert h.place(be, views[name]) == SI_OK
        assert h.weights(be)[0] == n1, "placing a resident tensor again uploaded it again"
        assert views["token_embd.weight"].loc == SI_LOC_HOST

        rng = np.random.default_rng(9)
        for name, wt, n_out, n_in in LAYOUT:
            if name not in placed:
                continue
            t, W = views[name], weights[name]
            cpu_view = _view(ref, g, name)
            x = rng.standard_normal(n_in).astype(np.float32)
            y = np.full(n_out, np.nan, np.float32)
            assert h.tensor_gemv(t, x, y, n_out) == 0, (name, h.errstr())
            y_ref = ref.tensor_gemv(ctypes.addressof(cpu_view), x, n_out)
            _, l1 = oracle.gemv(wt, W, n_out, n_in, x)
            assert_close(y, y_ref.astype(np.float64), l1, f"gemv {name} vs reference cpu_gemv")
            X = rng.standard_normal((5, n_in)).astype(np.float32)
            Y = np.full((5, n_out), np.nan, np.float32)
            assert h.tensor_gemm(be, t, X, Y) == SI_OK, (name, h.errstr())
            for m in range(5):
                y_ref = ref.tensor_gemv(ctypes.addressof(cpu_view), X[m], n_out)
                _, l1 = oracle.gemv(wt, W, n_out, n_in, X[m])
                assert_close(Y[m], y_ref.astype(np.float64), l1, f"gemm {name} row {m}")
            for row in (0, n_out // 2, n_out - 1):
                got = np.full(n_in, np.nan, np.float32)
                assert h.tensor_row(t, row, got) == 0
                want = ref.tensor_row(ctypes.addressof(cpu_view), row, n_in)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, row)
        emb = views["token_embd.weight"]
        emb_cpu = _view(ref, g, "token_embd.weight")
        for tok in (0, 17, N_VOCAB - 1):
            got = np.full(N_EMBD, np.nan, np.float32)
            assert h.tensor_row(emb, tok, got) == 0
            want = ref.tensor_row(ctypes.addressof(emb_cpu), tok, N_EMBD)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), tok
    finally:
        ref.gguf_close(g)


@pytest.mark.gpu
def test_place_failure_leaves_view_untouched(ref, hip_backend, tmp_path):
    from tests.host_py import SI_LOC_HOST
    h, be = hip_backend
    path = tmp_path / "model.gguf"
    _model_file(path)
    g = ref.gguf_open(str(path))
    try:
        t = _view(ref, g, "blk.0.attn_q.weight")
        t.data = None
        cpu_be = t.be
        assert h.place(be, t) == SI_EINVAL
        assert t.loc == SI_LOC_HOST and t.be == cpu_be
        assert "bad arguments" in h.errstr()
    finally:
        ref.gguf_close(g)
