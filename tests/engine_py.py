"""ctypes access to the reference engine checker (oracle/_ref/
libsiphon_engine_ref.so, built by oracle/Makefile target `engine` from the
reference's own engine.c, model.c and what they link, together with this
repository's batched prefill and hip adapter). TEST INFRASTRUCTURE ONLY."""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SO = os.path.join(ROOT, "oracle", "_ref", "libsiphon_engine_ref.so")


class RefEngineLib:
    def __init__(self, path: str = SO):
        L = ctypes.CDLL(path)
        vp, i64, u32p = ctypes.c_void_p, ctypes.c_int64, ctypes.POINTER(ctypes.c_uint32)
        fp = ctypes.POINTER(ctypes.c_float)
        L.re_errstr.restype = ctypes.c_char_p
        L.re_model_load.argtypes = [ctypes.c_char_p]
        L.re_model_load.restype = vp
        L.re_model_free.argtypes = [vp]
        L.re_engine_create.argtypes = [vp, i64, ctypes.c_int]
        L.re_engine_create.restype = vp
        L.re_engine_free.argtypes = [vp]
        L.re_engine_reset.argtypes = [vp]
        L.re_n_pos.argtypes = [vp]
        L.re_n_pos.restype = i64
        L.re_dims.argtypes = [vp, ctypes.POINTER(i64)]
        L.re_k_cache.argtypes = [vp]
        L.re_k_cache.restype = vp
        L.re_v_cache.argtypes = [vp]
        L.re_v_cache.restype = vp
        L.re_forward_loop.argtypes = [vp, u32p, i64]
        L.re_forward_loop.restype = fp
        L.re_prefill.argtypes = [vp, u32p, i64]
        L.re_prefill.restype = fp
        for f in ("re_layers_cpu", "re_layers_cpu_gemm", "re_layers_cpu_nogemm"):
            getattr(L, f).argtypes = [vp]
        L.re_hip_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(vp)]
        L.re_hip_close.argtypes = [vp]
        L.re_layers_hip.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int]
        L.re_rec_get.argtypes = [ctypes.c_int, ctypes.POINTER(vp), ctypes.POINTER(i64),
                                 ctypes.POINTER(fp), ctypes.POINTER(fp)]
        L.re_layout.argtypes = [ctypes.POINTER(i64)]
        L.re_mirror_layout.argtypes = [ctypes.POINTER(i64)]
        self.L = L

    def errstr(self) -> str:
        return self.L.re_errstr().decode()

    def layouts(self):
        a, b = (ctypes.c_int64 * 64)(), (ctypes.c_int64 * 64)()
        na, nb = self.L.re_layout(a), self.L.re_mirror_layout(b)
        return list(a[:na]), list(b[:nb])

    def load(self, path):
        m = self.L.re_model_load(str(path).encode())
        if not m:
            raise OSError(self.errstr())
        return m

    def engine(self, model, n_ctx, threads=2):
        e = self.L.re_engine_create(model, n_ctx, threads)
        if not e:
            raise OSError(self.errstr())
        return e

    def dims(self, e):
        d = (ctypes.c_int64 * 9)()
        self.L.re_dims(e, d)
        keys = ("n_layer", "n_head", "n_head_kv", "head_dim", "n_ctx", "n_vocab", "n_embd",
                "n_ff", "arch")
        return dict(zip(keys, list(d)))

    def _logits(self, p, e):
        if not p:
            return None
        return np.ctypeslib.as_array(p, shape=(self.dims(e)["n_vocab"],)).copy()

    def forward_loop(self, e, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        p = self.L.re_forward_loop(e, t.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), t.size)
        return self._logits(p, e)

    def prefill(self, e, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        p = self.L.re_prefill(e, t.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), t.size)
        return self._logits(p, e)

    def caches(self, e, n_pos):
        """K [n_layer][n_kv][n_pos][hd] and V [n_layer][n_kv][hd][n_pos] as
        f16 bit patterns (the written positions only)."""
        d = self.dims(e)
        shape_k = (d["n_layer"], d["n_head_kv"], d["n_ctx"], d["head_dim"])
        shape_v = (d["n_layer"], d["n_head_kv"], d["head_dim"], d["n_ctx"])
        k = np.ctypeslib.as_array(ctypes.cast(self.L.re_k_cache(e), ctypes.POINTER(ctypes.c_uint16)),
                                  shape=shape_k)[:, :, :n_pos, :].copy()
        v = np.ctypeslib.as_array(ctypes.cast(self.L.re_v_cache(e), ctypes.POINTER(ctypes.c_uint16)),
                                  shape=shape_v)[:, :, :, :n_pos].copy()
        return k, v

    def hip_open(self, lib):
        be = ctypes.c_void_p()
        rc = self.L.re_hip_open(lib.encode(), ctypes.byref(be))
        return rc, be.value

    def recorded(self):
        """[(weight bytes, type, n_in, n_out, X, Y)] of every recorded gemm."""
        out = []
        for i in range(self.L.re_rec_count()):
            data, meta = ctypes.c_void_p(), (ctypes.c_int64 * 4)()
            X, Y = ctypes.POINTER(ctypes.c_float)(), ctypes.POINTER(ctypes.c_float)()
            self.L.re_rec_get(i, ctypes.byref(data), meta, ctypes.byref(X), ctypes.byref(Y))
            wt, n_in, n_out, M = list(meta)
            out.append((wt, n_in, n_out, M, data.value,
                        np.ctypeslib.as_array(X, shape=(M, n_in)).copy(),
                        np.ctypeslib.as_array(Y, shape=(M, n_out)).copy()))
        return out
