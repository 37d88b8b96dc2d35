"""Python wrapper of the engine API (eva_open .. eva_close of include/xtag_eva.h, mirroring src/engine/eva.h)."""
import ctypes as C

import numpy as np

from .lib import lib

EVA_NBUF = 8
EVA_IN = 1024 * 592
EVA_SPARSE24 = 1


class EvaStruct(C.Structure):
    """The caller-allocated `eva` struct of include/xtag_eva.h."""
    _fields_ = [("nt", C.c_uint32), ("ntp", C.c_uint32), ("nt0", C.c_uint32), ("nb", C.c_uint32),
                ("hpn", C.c_void_p * EVA_NBUF), ("hout", C.c_void_p * EVA_NBUF), ("impl", C.c_void_p)]


class Engine:
    """eva_open_ex .. eva_close. Errors raise RuntimeError (the C calls print "eva: ..." to stderr).
    sparse: 2:4-prune the layer GEMM weights at bring-up and run them on the sparse matrix cores (EVA_SPARSE24)."""

    def __init__(self, weights, device=0, nb=8, extra=0, sparse=False):
        self.e = EvaStruct()
        self.ref = C.byref(self.e)
        flags = EVA_SPARSE24 if sparse else 0
        if lib.eva_open_ex(self.ref, str(weights).encode(), device, None, 0, extra, nb, flags) != 0:
            raise RuntimeError("eva_open failed")
        self.open = True

    @property
    def nt(self):
        return self.e.nt

    @property
    def nb(self):
        return self.e.nb

    def ready(self):
        if lib.eva_ready(self.ref) != 0:
            raise RuntimeError("eva bring-up failed")

    def submit(self, buf, inputs):
        """inputs: fp16 array [n][1024][592] (n <= nb)."""
        x = np.ascontiguousarray(inputs, dtype=np.float16)
        n = x.shape[0]
        ptrs = (C.c_void_p * max(n, 1))(*[x.ctypes.data + i * EVA_IN * 2 for i in range(n)])
        if lib.eva_submit(self.ref, buf, ptrs, n) != 0:
            raise RuntimeError("eva_submit failed")
        self._keep = x
        return n

    def wait(self, buf, n):
        p = lib.eva_wait(self.ref, buf)
        if not p:
            raise RuntimeError("eva_wait failed")
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (n * self.nt,)).reshape(n, self.nt).copy()

    def hpn(self, buf, n):
        p = self.e.hpn[buf]
        if not p:
            return None
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint16)), (n * 1024,)).reshape(n, 1024).copy()

    def query(self, buf):
        return lib.eva_query(self.ref, buf)

    def head_put(self, j, w16, bias):
        w = np.ascontiguousarray(w16, dtype=np.float16)
        if lib.eva_head_put(self.ref, j, w.ctypes.data, C.c_float(bias)) != 0:
            raise RuntimeError("eva_head_put failed")

    def head_get(self):
        w = np.empty((self.e.nt0, 1024), np.float16)
        b = np.empty(self.e.nt0, np.float32)
        if lib.eva_head_get(self.ref, w.ctypes.data, b.ctypes.data) != 0:
            raise RuntimeError("eva_head_get failed")
        return w, b

    # resident-input path
    def dev_input(self):
        return lib.eva_dev_input(self.ref)

    def dev_output(self):
        return lib.eva_dev_output(self.ref)

    def stream(self):
        return lib.eva_stream_handle(self.ref)

    def run(self):
        if lib.eva_run(self.ref) != 0:
            raise RuntimeError("eva_run failed")

    def sync(self):
        if lib.eva_sync(self.ref) != 0:
            raise RuntimeError("eva_sync failed")

    def profile(self):
        """eva_profile: GPU ms per op kind of one direct (non-graph) forward, summed over the layers."""
        ms = (C.c_double * 9)()
        if lib.eva_profile(self.ref, ms) != 0:
            raise RuntimeError("eva_profile failed")
        return {lib.eva_profile_opname(i).decode(): ms[i] for i in range(9)}

    def close(self):
        if self.open:
            lib.eva_close(self.ref)
            self.open = False

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


PX_NBUF = 4
PX_IN = 5184 * 592


class PxStruct(C.Structure):
    """The caller-allocated `px` struct of include/xtag_eva.h."""
    _fields_ = [("nt", C.c_uint32), ("ntp", C.c_uint32), ("nb", C.c_uint32), ("hout", C.c_void_p * PX_NBUF),
                ("impl", C.c_void_p)]


class PxEngine:
    """px_open_nb .. px_close (the PixAI tagger engine, src/engine/px.h). Errors raise RuntimeError."""

    def __init__(self, weights, device=0, nb=4):
        self.p = PxStruct()
        self.ref = C.byref(self.p)
        if lib.px_open_nb(self.ref, str(weights).encode(), device, None, 0, nb) != 0:
            raise RuntimeError("px_open failed")
        self.open = True

    @property
    def nt(self):
        return self.p.nt

    @property
    def nb(self):
        return self.p.nb

    def ready(self):
        if lib.px_ready(self.ref) != 0:
            raise RuntimeError("px bring-up failed")

    def submit(self, buf, inputs):
        """inputs: fp16 array [n][5184][592] window-major patch operands (n <= nb)."""
        x = np.ascontiguousarray(inputs, dtype=np.float16)
        n = x.shape[0]
        ptrs = (C.c_void_p * max(n, 1))(*[x.ctypes.data + i * PX_IN * 2 for i in range(n)])
        if lib.px_submit(self.ref, buf, ptrs, n) != 0:
            raise RuntimeError("px_submit failed")
        self._keep = x
        return n

    def wait(self, buf, n):
        p = lib.px_wait(self.ref, buf)
        if not p:
            raise RuntimeError("px_wait failed")
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (n * self.nt,)).reshape(n, self.nt).copy()

    def query(self, buf):
        return lib.px_query(self.ref, buf)

    def dev_input(self):
        return lib.px_dev_input(self.ref)

    def dev_output(self):
        return lib.px_dev_output(self.ref)

    def stream(self):
        return lib.px_stream_handle(self.ref)

    def run(self):
        if lib.px_run(self.ref) != 0:
            raise RuntimeError("px_run failed")

    def sync(self):
        if lib.px_sync(self.ref) != 0:
            raise RuntimeError("px_sync failed")

    def close(self):
        if self.open:
            lib.px_close(self.ref)
            self.open = False

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
