"""ctypes access to the host emulation of the matvec kernel (tests/emu)."""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "emu")
SO = os.path.join(HERE, "libsiphon_emu.so")


class Emulator:
    def __init__(self):
        # make rebuilds only when emu.cpp or the kernel headers it compiles changed
        subprocess.run(["make", "-s", "-C", HERE], check=True)
        L = ctypes.CDLL(SO)
        vp = ctypes.c_void_p
        L.emu_gemv_pair.argtypes = [ctypes.c_uint32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                    ctypes.c_int64, vp, vp, vp]
        L.emu_layout_bytes.argtypes = [ctypes.c_uint32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
        L.emu_layout_bytes.restype = ctypes.c_int64
        L.emu_repack.argtypes = [ctypes.c_uint32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, vp, vp]
        L.emu_dequant.argtypes = [ctypes.c_uint32, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                  vp, vp]
        self.L = L

    def gemv_pair(self, wtype, n_out, n_in, G, rows, xq, slice_elems=None):
        """slice_elems: column slice length the library applies at upload
        (None: SIHIP_SPLIT_ELEMS, which the library reads once at
        sihip_init, else the default)."""
        if slice_elems is None:
            slice_elems = int(os.environ.get("SIHIP_SPLIT_ELEMS", "-1"))
        rows = np.ascontiguousarray(rows, dtype=np.uint8)
        xq = np.ascontiguousarray(xq, dtype=np.uint8)
        y = np.zeros(n_out, dtype=np.float32)
        rc = self.L.emu_gemv_pair(wtype, n_out, n_in, G, slice_elems, rows.ctypes.data,
                                  xq.ctypes.data, y.ctypes.data)
        assert rc == 0
        return y

    def repack(self, wtype, n_out, n_in, G, rows):
        nb = self.L.emu_layout_bytes(wtype, n_out, n_in, G)
        assert nb > 0
        out = np.zeros(nb, dtype=np.uint8)
        rows = np.ascontiguousarray(rows, dtype=np.uint8)
        assert self.L.emu_repack(wtype, n_out, n_in, G, rows.ctypes.data, out.ctypes.data) == 0
        return out

    def dequant(self, wtype, n_out, n_in, G, rows):
        """Every row's weight values through the planar layout."""
        rows = np.ascontiguousarray(rows, dtype=np.uint8)
        out = np.zeros((n_out, n_in), dtype=np.float32)
        assert self.L.emu_dequant(wtype, n_out, n_in, G, rows.ctypes.data, out.ctypes.data) == 0
        return out
