"""ctypes access to the CPU oracle (libsiq_oracle.so) and, when it was built,
the compiled reference checker (_ref/libsiphon_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, always as the checker, never as the thing
measured or shipped.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libsiq_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libsiphon_ref.so")

# ggml type ids and block geometry (reference quant.h:92-119)
F32, F16, Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 0, 1, 2, 6, 8, 10, 11, 12, 13, 14, 15
GEOM = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34),
        Q2_K: (256, 84), Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176),
        Q6_K: (256, 210), Q8_K: (256, 292)}
PAIR = {F32: F32, F16: F16, Q4_0: Q8_0, Q5_0: Q8_0, Q8_0: Q8_0, Q2_K: Q8_K, Q3_K: Q8_K,
        Q4_K: Q8_K, Q5_K: Q8_K, Q6_K: Q8_K}
NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q5_0: "Q5_0", Q8_0: "Q8_0", Q2_K: "Q2_K",
         Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K", Q6_K: "Q6_K", Q8_K: "Q8_K"}
WEIGHT_TYPES = [Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, F16]

# worker threads of the oracle's row loop: the CPUs this process may run on,
# at most 16 (the share of one GPU box)
LANES = max(1, min(16, len(os.sched_getaffinity(0))))

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_u32 = ctypes.c_uint32


def row_bytes(wtype: int, n: int) -> int:
    be, bb = GEOM[wtype]
    return n // be * bb


def pair_bytes(pair: int, n: int) -> int:
    be, bb = GEOM[pair]
    return n // be * bb


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def build_oracle() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "libsiq_oracle.so"], check=True)


def build_ref() -> bool:
    """Compile the reference checker when the reference tree is present."""
    if not os.path.isdir("/root/reference/src"):
        return False
    subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)
    return True


class Oracle:
    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            build_oracle()
        L = ctypes.CDLL(path)
        L.siq_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.siq_f16_to_f32.restype = ctypes.c_float
        L.siq_f32_to_f16.argtypes = [ctypes.c_float]
        L.siq_f32_to_f16.restype = ctypes.c_uint16
        for fn in ("siq_quantize_q8_K", "siq_quantize_q8_0", "siq_quantize_q8_0_scalar",
                   "siq_convert_f16"):
            getattr(L, fn).argtypes = [_vp, _vp, _i64]
            getattr(L, fn).restype = None
        L.siq_quantize_pair.argtypes = [_u32, _vp, _vp, _i64]
        L.siq_dequant_row.argtypes = [_u32, _vp, _vp, _i64]
        L.siq_vec_dot.argtypes = [_u32, _i64, _vp, _vp, _vp, _vp]
        L.siq_vec_dot_dequant.argtypes = [_u32, _i64, _vp, _vp, _vp, _vp]
        L.siq_gemv.argtypes = [_u32, _vp, _i64, _i64, _vp, _vp, _vp, ctypes.c_int]
        L.siq_gemm.argtypes = [_u32, _vp, _i64, _i64, _vp, _i64, _vp, _vp, ctypes.c_int]
        L.siq_expf_poly.argtypes = [ctypes.c_float]
        L.siq_expf_poly.restype = ctypes.c_float
        L.siq_softmax.argtypes = [_vp, _vp, _i64, ctypes.c_float]
        L.siq_softmax.restype = None
        L.siq_dot_f16_simd.argtypes = [_i64, _vp, _vp]
        L.siq_dot_f16_simd.restype = ctypes.c_float
        L.siq_attn_decode.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_float,
                                      _vp, _vp, _vp]
        self.L = L

    def f16_to_f32(self, h: int) -> float:
        return self.L.siq_f16_to_f32(h)

    def f32_to_f16(self, f: float) -> int:
        return self.L.siq_f32_to_f16(f)

    def quantize(self, pair: int, x: np.ndarray, scalar_q8_0: bool = False) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(pair_bytes(pair, x.size), dtype=np.uint8)
        if pair == Q8_0 and scalar_q8_0:
            self.L.siq_quantize_q8_0_scalar(_ptr(x), _ptr(out), x.size)
        else:
            assert self.L.siq_quantize_pair(pair, _ptr(x), _ptr(out), x.size)
        return out

    def dequant(self, wtype: int, w: np.ndarray, n: int) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.uint8)
        out = np.zeros(n, dtype=np.float32)
        assert self.L.siq_dequant_row(wtype, _ptr(w), _ptr(out), n)
        return out

    def vec_dot(self, wtype: int, n: int, w: np.ndarray, a: np.ndarray, dequant_form=False):
        w = np.ascontiguousarray(w, dtype=np.uint8)
        a = np.ascontiguousarray(a, dtype=np.uint8)
        d = ctypes.c_double()
        m = ctypes.c_double()
        fn = self.L.siq_vec_dot_dequant if dequant_form else self.L.siq_vec_dot
        assert fn(wtype, n, _ptr(w), _ptr(a), ctypes.byref(d), ctypes.byref(m))
        return d.value, m.value

    def gemv(self, wtype: int, W: np.ndarray, n_out: int, n_in: int, x: np.ndarray, lanes: int = LANES):
        W = np.ascontiguousarray(W, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(n_out, dtype=np.float32)
        l1 = np.zeros(n_out, dtype=np.float64)
        assert self.L.siq_gemv(wtype, _ptr(W), n_out, n_in, _ptr(x), _ptr(y), _ptr(l1), lanes)
        return y, l1

    def gemm(self, wtype: int, W: np.ndarray, n_out: int, n_in: int, X: np.ndarray, lanes: int = LANES):
        W = np.ascontiguousarray(W, dtype=np.uint8)
        X = np.ascontiguousarray(X, dtype=np.float32)
        M = X.shape[0]
        Y = np.zeros((M, n_out), dtype=np.float32)
        L1 = np.zeros((M, n_out), dtype=np.float64)
        assert self.L.siq_gemm(wtype, _ptr(W), n_out, n_in, _ptr(X), M, _ptr(Y), _ptr(L1), lanes)
        return Y, L1


    def expf_poly(self, x: np.ndarray) -> np.ndarray:
        return np.array([self.L.siq_expf_poly(float(v)) for v in np.asarray(x, np.float32)],
                        dtype=np.float32)

    def softmax(self, x: np.ndarray, max_: float) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros_like(x)
        self.L.siq_softmax(_ptr(y), _ptr(x), x.size, max_)
        return y

    def dot_f16(self, a: np.ndarray, b: np.ndarray) -> float:
        a = np.ascontiguousarray(a, dtype=np.uint16)
        b = np.ascontiguousarray(b, dtype=np.uint16)
        return self.L.siq_dot_f16_simd(a.size, _ptr(a), _ptr(b))

    def attn_decode(self, q, k, v, n_head, n_head_kv, hd, n_ctx, pos, kq_scale):
        """(out [n_head*hd] f32, scores [n_head][n_ctx] f32, probs16 [n_head][n_ctx] u16);
        entries past pos of a scores/probs row are zero."""
        q = np.ascontiguousarray(q, dtype=np.float32)
        k = np.ascontiguousarray(k, dtype=np.uint16)
        v = np.ascontiguousarray(v, dtype=np.uint16)
        out = np.zeros(n_head * hd, np.float32)
        sc = np.zeros((n_head, n_ctx), np.float32)
        pr = np.zeros((n_head, n_ctx), np.uint16)
        assert self.L.siq_attn_decode(_ptr(q), _ptr(k), _ptr(v), n_head, n_head_kv, hd, n_ctx,
                                      pos, kq_scale, _ptr(out), _ptr(sc), _ptr(pr))
        return out, sc, pr


class Reference:
    """The reference's own kernels (compiled from /root/reference/src by
    oracle/Makefile); None-returning loader when it was not built."""

    DOT_NAMES = {F16: "f16", Q4_0: "q4_0_q8_0", Q5_0: "q5_0_q8_0", Q8_0: "q8_0_q8_0",
                 Q2_K: "q2_K_q8_K", Q3_K: "q3_K_q8_K", Q4_K: "q4_K_q8_K",
                 Q5_K: "q5_K_q8_K", Q6_K: "q6_K_q8_K"}

    def __init__(self, path: str = REF_SO):
        L = ctypes.CDLL(path)
        L.ref_shim_impl.restype = ctypes.c_int
        L.si_f32_to_f16.argtypes = [ctypes.c_float]
        L.si_f32_to_f16.restype = ctypes.c_uint16
        L.si_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.si_f16_to_f32.restype = ctypes.c_float
        for fn in ("si_quant_row_q8_0", "si_quant_row_q8_K", "si_avx2_quant_row_q8_0"):
            getattr(L, fn).argtypes = [_vp, _vp, ctypes.c_int]
            getattr(L, fn).restype = None
        L.si_dequant_row.argtypes = [_u32, _vp, _vp, ctypes.c_int]
        L.si_dequant_row.restype = ctypes.c_bool
        for name in self.DOT_NAMES.values():
            for pre in ("si_dot_", "si_avx2_dot_"):
                f = getattr(L, pre + name)
                f.argtypes = [ctypes.c_int, _vp, _vp, _vp]
                f.restype = None
        L.ref_shim_gemv.argtypes = [_u32, _vp, _i64, _i64, _vp, _vp, ctypes.c_int, ctypes.c_int, _vp]
        L.ref_shim_gemv.restype = ctypes.c_int
        L.ref_shim_gguf_open.argtypes = [ctypes.c_char_p]
        L.ref_shim_gguf_open.restype = _vp
        L.ref_shim_gguf_close.argtypes = [_vp]
        L.ref_shim_errstr.restype = ctypes.c_char_p
        L.ref_shim_gguf_tensor.argtypes = [_vp, ctypes.c_char_p, _vp, _vp]
        L.ref_shim_gguf_map_offset.argtypes = [_vp, _vp]
        L.ref_shim_gguf_map_offset.restype = _i64
        L.ref_shim_gguf_alignment.argtypes = [_vp]
        L.ref_shim_gguf_alignment.restype = ctypes.c_uint64
        L.ref_shim_tensor_gemv.argtypes = [_vp, _vp, _vp, _i64, ctypes.c_int]
        L.ref_shim_tensor_row.argtypes = [_vp, ctypes.c_uint64, _vp]
        L.si_expf.argtypes = [ctypes.c_float]
        L.si_expf.restype = ctypes.c_float
        L.si_softmax.argtypes = [_vp, _vp, ctypes.c_int, ctypes.c_float]
        L.si_softmax.restype = None
        self.L = L
        self.avx2 = bool(L.ref_shim_impl())

    @staticmethod
    def load():
        if not os.path.exists(REF_SO):
            return None
        return Reference()

    def quant_q8_K(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(pair_bytes(Q8_K, x.size), dtype=np.uint8)
        self.L.si_quant_row_q8_K(_ptr(x), _ptr(out), x.size)
        return out

    def quant_q8_0(self, x: np.ndarray, simd: bool = True) -> np.ndarray:
        """simd=True: the AVX2 quantizer production dispatches to on x86.
        simd=False: the reference's dispatcher, which takes its scalar
        branch only in a process started with SI_SCALAR=1 (self.avx2 is
        then False)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(pair_bytes(Q8_0, x.size), dtype=np.uint8)
        if simd:
            self.L.si_avx2_quant_row_q8_0(_ptr(x), _ptr(out), x.size)
        else:
            assert not self.avx2, "scalar Q8_0 needs a process started with SI_SCALAR=1"
            self.L.si_quant_row_q8_0(_ptr(x), _ptr(out), x.size)
        return out

    def f16(self, x: np.ndarray) -> np.ndarray:
        return np.array([self.L.si_f32_to_f16(float(v)) for v in np.asarray(x, np.float32)],
                        dtype=np.uint16)

    def dequant(self, wtype: int, w: np.ndarray, n: int) -> np.ndarray:
        w = np.ascontiguousarray(w, dtype=np.uint8)
        out = np.zeros(n, dtype=np.float32)
        assert self.L.si_dequant_row(wtype, _ptr(w), _ptr(out), n)
        return out

    def dot(self, wtype: int, n: int, w: np.ndarray, a: np.ndarray, simd: bool = True) -> float:
        w = np.ascontiguousarray(w, dtype=np.uint8)
        a = np.ascontiguousarray(a, dtype=np.uint8)
        s = ctypes.c_float()
        f = getattr(self.L, ("si_avx2_dot_" if simd else "si_dot_") + self.DOT_NAMES[wtype])
        f(n, ctypes.byref(s), _ptr(w), _ptr(a))
        return s.value

    def expf(self, x: np.ndarray) -> np.ndarray:
        return np.array([self.L.si_expf(float(v)) for v in np.asarray(x, np.float32)],
                        dtype=np.float32)

    def softmax(self, x: np.ndarray, max_: float) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros_like(x)
        self.L.si_softmax(_ptr(y), _ptr(x), x.size, max_)
        return y

    def attn_decode(self, q, k, v, n_head, n_head_kv, hd, n_ctx, pos, kq_scale):
        """One layer's decode attention composed from the reference's own
        kernels in the steps of its attn_head (engine.c:90-147): f16 query,
        the dispatched f16 dot per cached position, the scale, the max, its
        softmax, f16 probabilities, the dispatched f16 dot per value row.
        Same return as Oracle.attn_decode."""
        q = np.asarray(q, np.float32)
        k = np.asarray(k, np.uint16).reshape(n_head_kv, n_ctx, hd)
        v = np.asarray(v, np.uint16).reshape(n_head_kv, hd, n_ctx)
        n, gqa = pos + 1, n_head // n_head_kv
        ks = np.float32(kq_scale)
        out = np.zeros(n_head * hd, np.float32)
        sc_all = np.zeros((n_head, n_ctx), np.float32)
        pr_all = np.zeros((n_head, n_ctx), np.uint16)
        for h in range(n_head):
            hk = h // gqa
            q16 = self.f16(q[h * hd:(h + 1) * hd])
            q8 = q16.view(np.uint8)
            sc = np.array([self.dot(F16, hd, k[hk, j].view(np.uint8), q8, simd=self.avx2)
                           for j in range(n)], np.float32) * ks
            mx = np.float32(-np.inf)
            for s in sc:
                if s > mx:
                    mx = s
            pr16 = self.f16(self.softmax(sc, float(mx)))
            p8 = pr16.view(np.uint8)
            out[h * hd:(h + 1) * hd] = [
                self.dot(F16, n, np.ascontiguousarray(v[hk, c, :n]).view(np.uint8), p8,
                         simd=self.avx2) for c in range(hd)]
            sc_all[h, :n] = sc
            pr_all[h, :n] = pr16
        return out, sc_all, pr_all

    # GGUF container through the reference parser; tensor views are
    # si_tensor structs at caller-owned addresses (t_addr)
    def gguf_open(self, path: str) -> int:
        g = self.L.ref_shim_gguf_open(path.encode())
        if not g:
            raise OSError(f"reference si_gguf_open({path}): {self.L.ref_shim_errstr().decode()}")
        return g

    def gguf_close(self, g: int) -> None:
        self.L.ref_shim_gguf_close(g)

    def gguf_tensor(self, g: int, name: str, be: int | None, t_addr: int) -> int:
        return self.L.ref_shim_gguf_tensor(g, name.encode(), be, t_addr)

    def gguf_map_offset(self, g: int, p: int) -> int:
        return self.L.ref_shim_gguf_map_offset(g, p)

    def gguf_alignment(self, g: int) -> int:
        return self.L.ref_shim_gguf_alignment(g)

    def tensor_size(self) -> int:
        return self.L.ref_shim_tensor_size()

    def tensor_gemv(self, t_addr: int, x: np.ndarray, n_out: int, lanes: int = LANES):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(n_out, dtype=np.float32)
        self.L.ref_shim_tensor_gemv(t_addr, _ptr(x), _ptr(y), n_out, lanes)
        return y

    def tensor_row(self, t_addr: int, row: int, n: int):
        out = np.zeros(n, dtype=np.float32)
        self.L.ref_shim_tensor_row(t_addr, row, _ptr(out))
        return out

    def gemv_timed(self, wtype: int, W: np.ndarray, n_out: int, n_in: int, x: np.ndarray,
                   lanes: int, reps: int):
        W = np.ascontiguousarray(W, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros(n_out, dtype=np.float32)
        secs = np.zeros(reps, dtype=np.float64)
        rc = self.L.ref_shim_gemv(wtype, _ptr(W), n_out, n_in, _ptr(x), _ptr(y), lanes, reps,
                                  _ptr(secs))
        assert rc == 0
        return y, secs
