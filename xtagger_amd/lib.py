"""ctypes binding of libxtag_eva.so (declared in include/xtag_eva.h). Raises ImportError if it is not built."""
import ctypes as C
import os

from . import LIB_PATH

if not os.path.exists(LIB_PATH):
    raise ImportError(f"{LIB_PATH} is not built: run `make -C xtagger_amd/csrc` (or __graft_entry__.build())")

lib = C.CDLL(LIB_PATH)

_p, _i, _u32, _f = C.c_void_p, C.c_int, C.c_uint32, C.c_float

_SIGS = {
    "eva_k_quant_act": (_i, [_p, _i, _i, _i, _i, _p, _i, _p, _i, _p]),
    "eva_k_quant_w": (_i, [_p, _i, _i, _p, _p, _p]),
    "eva_k_e4m3_bits": (_i, [_u32, _u32, _p, _p]),
    "eva_k_gemm": (_i, [_p, _i, _p, _i, _p, _p, _i, _i, _i, _p, _i, _i, _p]),
}

for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


def ptr(t):
    """Device (or host) address of a torch tensor or numpy array, or None."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return C.c_void_p(t.data_ptr())
    return C.c_void_p(t.ctypes.data)


def check(rc, what):
    if rc != 0:
        raise RuntimeError(f"{what} failed (see stderr)")
