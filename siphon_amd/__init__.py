"""Python binding of libsiphon_hip.so (the C-ABI in include/sihip.h).

The product is the C-ABI library; this module is plumbing for tests and the
benchmark. It loads the in-tree build and raises if it is missing: there is
no CPU fallback behind it.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

from .build import HIP_SO

# ggml type ids (reference include/siphon/quant.h:103-119)
F32, F16, Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 2, 6, 8, 10, 11, 12, 13, 14, 15
GEOM = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34), Q2_K: (256, 84),
        Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210),
        Q8_K: (256, 292)}
PAIR = {F32: F32, F16: F16, Q4_0: Q8_0, Q5_0: Q8_0, Q8_0: Q8_0, Q2_K: Q8_K, Q3_K: Q8_K, Q4_K: Q8_K,
        Q5_K: Q8_K, Q6_K: Q8_K}
NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K",
         Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", Q8_K: "Q8_K"}
TYPES = {v: k for k, v in NAMES.items()}
# formats in the planar layout (every layout test runs over these); F32
# weights keep their rows as they are and have tests of their own
WEIGHT_TYPES = [Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, F16]

ABI_VERSION = 3


def row_bytes(wtype: int, n_in: int) -> int:
    be, bb = GEOM[wtype]
    return n_in // be * bb


class SihipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"sihip error {code}: {msg}")
        self.code = code


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_lib = None


def load_library(path: str = HIP_SO) -> ctypes.CDLL:
    """Load libsiphon_hip.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is missing: build it with `python -m siphon_amd.build` "
            "(there is no CPU fallback)")
    L = ctypes.CDLL(path)
    L.sihip_abi_version.restype = ctypes.c_int
    L.sihip_init.argtypes = [ctypes.c_int, ctypes.POINTER(_vp)]
    L.sihip_shutdown.argtypes = [_vp]
    L.sihip_shutdown.restype = None
    L.sihip_last_error.argtypes = [_vp]
    L.sihip_last_error.restype = ctypes.c_char_p
    L.sihip_set_option.argtypes = [_vp, ctypes.c_char_p, _i64]
    L.sihip_weight_upload.argtypes = [_vp, _u32, _u64, _u64, _vp, _u64, ctypes.POINTER(_vp)]
    L.sihip_weight_free.argtypes = [_vp, _vp]
    L.sihip_weight_device_bytes.argtypes = [_vp]
    L.sihip_weight_device_bytes.restype = _u64
    L.sihip_weight_tile_cols.argtypes = [_vp]
    L.sihip_weight_slice_rounds.argtypes = [_vp]
    L.sihip_weight_prepare_gemm.argtypes = [_vp, _vp]
    L.sihip_gemv.argtypes = [_vp, _vp, _vp, _vp, _i64]
    L.sihip_gemm.argtypes = [_vp, _vp, _vp, _i64, _vp]
    L.sihip_gemv_dev.argtypes = [_vp, _vp, _vp, _vp, _i64, _vp]
    L.sihip_dequant_row.argtypes = [_vp, _vp, _u64, _vp]
    L.sihip_dequant_rows_dev.argtypes = [_vp, _vp, _u64, _u64, _vp, _i64, _vp]
    L.sihip_probe_read_dev.argtypes = [_vp, _vp, _u64, _vp, _vp]
    L.sihip_attn_decode_dev.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                        ctypes.c_float, _vp, _vp, _vp, _vp]
    L.sihip_gemm_dev.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp]
    L.sihip_gemm_dev_noalloc.argtypes = [_vp, _vp, _vp, _i64, _vp, _vp]
    L.sihip_gemv_multi_dev.argtypes = [_vp, ctypes.c_int, ctypes.POINTER(_vp), _vp,
                                       ctypes.POINTER(_vp), _vp]
    L.sihip_gemm_multi_dev.argtypes = [_vp, ctypes.c_int, ctypes.POINTER(_vp), _vp, _i64,
                                       ctypes.POINTER(_vp), _vp]
    for fn in ("sihip_quantize_q8_K", "sihip_quantize_q8_0", "sihip_convert_f16"):
        getattr(L, fn).argtypes = [_vp, _vp, _vp, _i64]
    L.sihip_quantize_q8_K_rows.argtypes = [_vp, _vp, _i64, _i64, ctypes.c_int, _vp]
    L.sihip_vec_dot.argtypes = [_vp, _u32, ctypes.c_int, _vp, _vp, _vp]
    L.sihip_dev_alloc.argtypes = [_vp, _u64, ctypes.POINTER(_vp)]
    L.sihip_dev_free.argtypes = [_vp, _vp]
    L.sihip_memcpy_htod.argtypes = [_vp, _vp, _vp, _u64]
    L.sihip_memcpy_dtoh.argtypes = [_vp, _vp, _vp, _u64]
    L.sihip_synchronize.argtypes = [_vp]
    L.sihip_gemv_pair.argtypes = [_vp, _u32, _i64, _i64, _vp, _vp, _vp]
    if L.sihip_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {L.sihip_abi_version()} != {ABI_VERSION}")
    _lib = L
    return L


def load_library_at(path: str) -> ctypes.CDLL:
    """Load a specific build of the library (used to compare build variants)."""
    global _lib
    saved, _lib = _lib, None
    try:
        return load_library(path)
    finally:
        _lib = saved


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


class Weight:
    def __init__(self, dev: "Device", handle: int, wtype: int, n_out: int, n_in: int):
        self.dev, self.handle, self.type, self.n_out, self.n_in = dev, handle, wtype, n_out, n_in

    @property
    def device_bytes(self) -> int:
        return int(self.dev.L.sihip_weight_device_bytes(self.handle))

    @property
    def tile_cols(self) -> int:
        return int(self.dev.L.sihip_weight_tile_cols(self.handle))

    @property
    def slice_rounds(self) -> int:
        return int(self.dev.L.sihip_weight_slice_rounds(self.handle))

    @property
    def gguf_bytes(self) -> int:
        return self.n_out * row_bytes(self.type, self.n_in)

    def prepare_gemm(self):
        """Build the matrix-core GEMM copy now (Q4_K; no-op otherwise)."""
        self.dev._check(self.dev.L.sihip_weight_prepare_gemm(self.dev.ctx, self.handle))

    def free(self):
        if self.handle:
            self.dev.L.sihip_weight_free(self.dev.ctx, self.handle)
            self.handle = None


class Device:
    """One sihip context on HIP device `device`."""

    def __init__(self, device: int = 0, lib_path: str | None = None):
        self.L = load_library() if lib_path is None else load_library_at(lib_path)
        ctx = _vp()
        rc = self.L.sihip_init(device, ctypes.byref(ctx))
        if rc != 0:
            raise SihipError(rc, self.L.sihip_last_error(None).decode())
        self.ctx = ctx.value

    def _check(self, rc: int):
        if rc != 0:
            raise SihipError(rc, self.L.sihip_last_error(self.ctx).decode())

    def set_option(self, name: str, value: int):
        """A tuning knob of this context (sihip_set_option); -1 restores the
        built-in rule."""
        self._check(self.L.sihip_set_option(self.ctx, name.encode(), int(value)))

    def close(self):
        if self.ctx:
            self.L.sihip_shutdown(self.ctx)
            self.ctx = None

    def upload(self, wtype: int, n_out: int, n_in: int, blocks: np.ndarray) -> Weight:
        blocks = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
        h = _vp()
        self._check(self.L.sihip_weight_upload(self.ctx, wtype, n_out, n_in, _ptr(blocks),
                                               blocks.size, ctypes.byref(h)))
        return Weight(self, h.value, wtype, n_out, n_in)

    def gemv(self, w: Weight, x: np.ndarray, n_out: int | None = None) -> np.ndarray:
        n_out = w.n_out if n_out is None else n_out
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(n_out, dtype=np.float32)
        self._check(self.L.sihip_gemv(self.ctx, w.handle, _ptr(x), _ptr(y), n_out))
        return y

    def gemm(self, w: Weight, X: np.ndarray) -> np.ndarray:
        X = np.ascontiguousarray(X, dtype=np.float32)
        Y = np.zeros((X.shape[0], w.n_out), dtype=np.float32)
        self._check(self.L.sihip_gemm(self.ctx, w.handle, _ptr(X), X.shape[0], _ptr(Y)))
        return Y

    # device-pointer variants (pointers as ints, stream as int or None)
    def gemv_dev(self, w: Weight, x_ptr: int, y_ptr: int, n_out: int, stream: int | None = None):
        self._check(self.L.sihip_gemv_dev(self.ctx, w.handle, x_ptr, y_ptr, n_out, stream))

    def dequant_row(self, w: Weight, row: int) -> np.ndarray:
        out = np.zeros(w.n_in, dtype=np.float32)
        self._check(self.L.sihip_dequant_row(self.ctx, w.handle, row, _ptr(out)))
        return out

    def probe_read_dev(self, p: int, nbytes: int, sink_ptr: int, stream: int | None = None):
        self._check(self.L.sihip_probe_read_dev(self.ctx, p, nbytes, sink_ptr, stream))

    def dequant_rows_dev(self, w: Weight, row0: int, nrows: int, out_ptr: int, ldo: int,
                         stream: int | None = None):
        self._check(self.L.sihip_dequant_rows_dev(self.ctx, w.handle, row0, nrows, out_ptr, ldo,
                                                  stream))

    def attn_decode_dev(self, q_ptr: int, k_ptr: int, v_ptr: int, n_head: int, n_head_kv: int,
                        head_dim: int, n_ctx: int, pos: int, kq_scale: float, out_ptr: int,
                        scores_ptr: int | None = None, probs_ptr: int | None = None,
                        stream: int | None = None):
        self._check(self.L.sihip_attn_decode_dev(self.ctx, q_ptr, k_ptr, v_ptr, n_head, n_head_kv,
                                                 head_dim, n_ctx, pos, kq_scale, out_ptr,
                                                 scores_ptr, probs_ptr, stream))

    def gemm_dev(self, w: Weight, X_ptr: int, M: int, Y_ptr: int, stream: int | None = None):
        self._check(self.L.sihip_gemm_dev(self.ctx, w.handle, X_ptr, M, Y_ptr, stream))

    def gemm_dev_noalloc(self, w: Weight, X_ptr: int, M: int, Y_ptr: int,
                         stream: int | None = None):
        """gemm_dev on the library's static scratch: allocates nothing (the
        weight's GEMM copy must be prepared)."""
        self._check(self.L.sihip_gemm_dev_noalloc(self.ctx, w.handle, X_ptr, M, Y_ptr, stream))

    def gemv_multi_dev(self, ws, x_ptr: int, y_ptrs, stream: int | None = None):
        n = len(ws)
        wa = (_vp * n)(*[w.handle for w in ws])
        ya = (_vp * n)(*y_ptrs)
        self._check(self.L.sihip_gemv_multi_dev(self.ctx, n, wa, x_ptr, ya, stream))

    def gemm_multi_dev(self, ws, X_ptr: int, M: int, Y_ptrs, stream: int | None = None):
        n = len(ws)
        wa = (_vp * n)(*[w.handle for w in ws])
        ya = (_vp * n)(*Y_ptrs)
        self._check(self.L.sihip_gemm_multi_dev(self.ctx, n, wa, X_ptr, M, ya, stream))

    # device memory through the library's own HIP runtime (no torch needed)
    def alloc(self, nbytes: int) -> "DevBuf":
        p = _vp()
        self._check(self.L.sihip_dev_alloc(self.ctx, nbytes, ctypes.byref(p)))
        return DevBuf(self, p.value, nbytes)

    def to_device(self, a: np.ndarray) -> "DevBuf":
        a = np.ascontiguousarray(a)
        b = self.alloc(max(a.nbytes, 16))
        self._check(self.L.sihip_memcpy_htod(self.ctx, b.ptr, _ptr(a), a.nbytes))
        return b

    def synchronize(self):
        self._check(self.L.sihip_synchronize(self.ctx))

    def quantize(self, pair: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        be, bb = GEOM[pair]
        out = np.zeros(x.size // be * bb, dtype=np.uint8)
        if pair == F32:
            return x.view(np.uint8).copy()
        fn = {Q8_K: self.L.sihip_quantize_q8_K, Q8_0: self.L.sihip_quantize_q8_0,
              F16: self.L.sihip_convert_f16}[pair]
        self._check(fn(self.ctx, _ptr(x), _ptr(out), x.size))
        return out

    def quantize_gemm_rows(self, X: np.ndarray, bm: int) -> np.ndarray:
        """Rows of X through the matrix-core GEMMs' Q8_K activation records
        (m blocks of bm rows), returned as Q8_K blocks (292 B each)."""
        X = np.ascontiguousarray(X, dtype=np.float32)
        M, n_in = X.shape
        out = np.zeros(M * (n_in // 256) * 292, dtype=np.uint8)
        self._check(self.L.sihip_quantize_q8_K_rows(self.ctx, _ptr(X), M, n_in, bm, _ptr(out)))
        return out

    def vec_dot(self, wtype: int, n: int, w: np.ndarray, a: np.ndarray) -> float:
        s = np.zeros(1, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        a = np.ascontiguousarray(a, dtype=np.uint8)
        self._check(self.L.sihip_vec_dot(self.ctx, wtype, n, _ptr(s), _ptr(w), _ptr(a)))
        return float(s[0])

    def gemv_pair(self, wtype: int, n_rows: int, n_in: int, rows: np.ndarray,
                  xq: np.ndarray) -> np.ndarray:
        rows = np.ascontiguousarray(rows, dtype=np.uint8)
        xq = np.ascontiguousarray(xq, dtype=np.uint8)
        y = np.zeros(n_rows, dtype=np.float32)
        self._check(self.L.sihip_gemv_pair(self.ctx, wtype, n_rows, n_in, _ptr(rows), _ptr(xq),
                                           _ptr(y)))
        return y


class DevBuf:
    """A device allocation made through the library (sihip_dev_alloc)."""

    def __init__(self, dev: "Device", ptr: int, nbytes: int):
        self.dev, self.ptr, self.nbytes = dev, ptr, nbytes

    def to_host(self, dtype, count: int) -> np.ndarray:
        out = np.empty(count, dtype=dtype)
        assert out.nbytes <= self.nbytes
        self.dev._check(self.dev.L.sihip_memcpy_dtoh(self.dev.ctx, _ptr(out), self.ptr, out.nbytes))
        return out

    def fill(self, a: np.ndarray):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        self.dev._check(self.dev.L.sihip_memcpy_htod(self.dev.ctx, self.ptr, _ptr(a), a.nbytes))

    def free(self):
        if self.ptr:
            self.dev._check(self.dev.L.sihip_dev_free(self.dev.ctx, self.ptr))
            self.ptr = 0
