"""ctypes access to the "hip" si_backend adapter through its test harness
(tests/host: the adapter plus stand-ins for the Siphon functions it calls)."""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "host")
SO = os.path.join(HERE, "libsi_harness.so")


SI_LOC_NONE, SI_LOC_HOST, SI_LOC_DEVICE = 0, 1, 2


class SiTensor(ctypes.Structure):
    """si_tensor (reference include/siphon/tensor.h:33-41)."""
    _fields_ = [("type", ctypes.c_uint32), ("ne", ctypes.c_uint64 * 4),
                ("n_elems", ctypes.c_uint64), ("n_bytes", ctypes.c_uint64),
                ("data", ctypes.c_void_p), ("loc", ctypes.c_int), ("be", ctypes.c_void_p)]


class Harness:
    def __init__(self):
        subprocess.run(["make", "-s", "-C", HERE], check=True)
        L = ctypes.CDLL(SO)
        vp, u32, u64, i64 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int64
        L.th_errstr.restype = ctypes.c_char_p
        L.th_open.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(vp)]
        L.th_close.argtypes = [vp]
        L.th_name.argtypes = [vp]
        L.th_name.restype = ctypes.c_char_p
        L.th_gemv.argtypes = [vp, u32, u64, u64, vp, u64, vp, vp, i64]
        L.th_gemm.argtypes = [vp, u32, u64, u64, vp, u64, vp, i64, vp]
        L.th_cpu.restype = vp
        L.th_vtable_gemm.argtypes = [vp, u32, u64, u64, vp, u64, vp, i64, vp]
        L.th_row_to_f32.argtypes = [vp, u32, u64, u64, vp, u64, u64, vp]
        L.th_weights.argtypes = [vp, ctypes.POINTER(u64)]
        L.th_upload.argtypes = [vp, u32, u64, u64, vp, u64]
        tp = ctypes.POINTER(SiTensor)
        L.th_place.argtypes = [vp, tp]
        L.th_tensor_gemv.argtypes = [tp, vp, vp, i64]
        L.th_tensor_row.argtypes = [tp, u64, vp]
        L.th_tensor_gemm.argtypes = [vp, tp, vp, i64, vp]
        self.L = L

    def errstr(self) -> str:
        return self.L.th_errstr().decode()

    def open(self, path, device=0):
        be = ctypes.c_void_p()
        rc = self.L.th_open(path.encode() if path else None, device, ctypes.byref(be))
        return rc, be.value

    def close(self, be):
        self.L.th_close(be)

    def name(self, be):
        return self.L.th_name(be).decode()

    def gemv(self, be, wt, n_out, n_in, W, x, y, n):
        return self.L.th_gemv(be, wt, n_out, n_in, W.ctypes.data, W.nbytes, x.ctypes.data,
                              y.ctypes.data, n)

    def gemm(self, be, wt, n_out, n_in, W, X, Y):
        return self.L.th_gemm(be, wt, n_out, n_in, W.ctypes.data, W.nbytes, X.ctypes.data,
                              X.shape[0], Y.ctypes.data)

    def cpu(self):
        """The harness's CPU backend (oracle dots, gemm slot = one gemv per row)."""
        return self.L.th_cpu()

    def vtable_gemm(self, be, wt, n_out, n_in, W, X, Y):
        """be->gemm through the vtable slot."""
        return self.L.th_vtable_gemm(be, wt, n_out, n_in, W.ctypes.data, W.nbytes, X.ctypes.data,
                                     X.shape[0], Y.ctypes.data)

    def row_to_f32(self, be, wt, n_out, n_in, W, row, out):
        return self.L.th_row_to_f32(be, wt, n_out, n_in, W.ctypes.data, W.nbytes, row,
                                    out.ctypes.data)

    def upload(self, be, wt, n_out, n_in, W):
        return self.L.th_upload(be, wt, n_out, n_in, W.ctypes.data, W.nbytes)

    def weights(self, be):
        b = ctypes.c_uint64()
        n = self.L.th_weights(be, ctypes.byref(b))
        return n, b.value

    def tensor_size(self) -> int:
        return self.L.th_tensor_size()

    def place(self, be, t: SiTensor) -> int:
        return self.L.th_place(be, ctypes.byref(t))

    def tensor_gemv(self, t: SiTensor, x, y, n) -> int:
        return self.L.th_tensor_gemv(ctypes.byref(t), x.ctypes.data, y.ctypes.data, n)

    def tensor_row(self, t: SiTensor, row, out) -> int:
        return self.L.th_tensor_row(ctypes.byref(t), row, out.ctypes.data)

    def tensor_gemm(self, be, t: SiTensor, X, Y) -> int:
        return self.L.th_tensor_gemm(be, ctypes.byref(t), X.ctypes.data, X.shape[0], Y.ctypes.data)
