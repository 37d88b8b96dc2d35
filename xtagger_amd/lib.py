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
    "eva_k_scale_bits": (_i, [_u32, _u32, _i, _p, _p]),
    "eva_k_gemm": (_i, [_p, _i, _p, _i, _p, _p, _i, _i, _i, _p, _i, _i, _p]),
    "eva_k_ln": (_i, [_p, _p, _p, _p, _p, _i, _i, _p]),
    "eva_k_qkv": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _p, _i, _p]),
    "eva_k_flash": (_i, [_p, _p, _p, _p, _p, _i, _i, _p, _p]),
    "eva_k_flash_seq": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _p, _p]),
    "eva_k_oproj": (_i, [_p, _p, _i, _p, _p, _p, _i, _p]),
    "px_k_qkv": (_i, [_p, _p, _i, _p, _p, _p, _p, _i, _p, _p, _p, _i, _p]),
    "px_k_proj": (_i, [_p, _p, _i, _p, _p, _p, _p, _i, _p]),
    "px_k_fc1": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _p, _i, _p]),
    "px_k_fc2": (_i, [_p, _p, _i, _p, _p, _p, _p, _i, _p]),
    "px_probe_gelu": (_i, [_p, _p, _i, _p]),
    "px_k_pe": (_i, [_p, _p, _p, _i, _p]),
    "px_k_pembed": (_i, [_p, _p, _i, _p, _p, _i, _p]),
    "px_k_hln": (_i, [_p, _p, _p, _p, _i, _p, _p, _p, _i, _p]),
    "px_k_hstat": (_i, [_p, _p, _i, _i, _p]),
    "px_k_hpool": (_i, [_p, _p, _p, _p, _p, _i, _i, _p]),
    "px_k_hproj": (_i, [_p, _i, _p, _p, _i, _p]),
    "eva_k_fc1": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _i, _p]),
    "eva_k_fc2": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _p, _i, _p]),
    "eva_k_head": (_i, [_p, _p, _i, _p, _p, _i, _p, _p, _i, _i, _p]),
    "eva_k_pe": (_i, [_p, _p, _p, _p, _i, _p]),
    "eva_k_pool": (_i, [_p, _p, _i, _p]),
    "eva_k_lnh": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _p]),
    "eva_k_prep_w": (_i, [_p, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p]),
    "eva_k_fold_cd": (_i, [_p, _p, _p, _i, _p, _p, _p, _p]),
    "eva_k_prune24": (_i, [_p, _i, _i, _p]),
    "eva_k_pack24": (_i, [_p, _i, _i, _p, _p, _p, _p]),
    "eva_k_gemm_sp": (_i, [_p, _i, _p, _i, _p, _p, _p, _i, _i, _i, _p, _i, _i, _p]),
    "eva_k_qkv_sp": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _p, _p, _i, _p]),
    "eva_k_oproj_sp": (_i, [_p, _p, _i, _p, _p, _p, _p, _i, _p]),
    "eva_k_fc1_sp": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _p, _i, _p]),
    "eva_k_fc1_rs": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _p, _i, _p]),
    "eva_k_fc1_rs_sp": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _p, _p, _i, _p]),
    "eva_k_prep_w8": (_i, [_p, _i, _i, _i, _i, _i, _i, _f, _p, _p, _p]),
    "eva_k_fold_c_rs": (_i, [_p, _p, _p, _p, _p]),
    "eva_k_fc2_sp": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _p, _p, _i, _p]),
    "eva_open": (_i, [_p, C.c_char_p, _i, _p, C.c_size_t, _u32]),
    "eva_open_nb": (_i, [_p, C.c_char_p, _i, _p, C.c_size_t, _u32, _u32]),
    "eva_open_ex": (_i, [_p, C.c_char_p, _i, _p, C.c_size_t, _u32, _u32, _u32]),
    "eva_ready": (_i, [_p]),
    "eva_poll": (_i, [_p]),
    "eva_submit": (_i, [_p, _u32, _p, _u32]),
    "eva_query": (_i, [_p, _u32]),
    "eva_wait": (_p, [_p, _u32]),
    "eva_head_put": (_i, [_p, _u32, _p, _f]),
    "eva_head_get": (_i, [_p, _p, _p]),
    "eva_close": (None, [_p]),
    "px_open": (_i, [_p, C.c_char_p, _i, _p, C.c_size_t]),
    "px_open_nb": (_i, [_p, C.c_char_p, _i, _p, C.c_size_t, _u32]),
    "px_ready": (_i, [_p]),
    "px_poll": (_i, [_p]),
    "px_submit": (_i, [_p, _u32, _p, _u32]),
    "px_query": (_i, [_p, _u32]),
    "px_wait": (_p, [_p, _u32]),
    "px_close": (None, [_p]),
    "px_dev_input": (_p, [_p]),
    "px_run": (_i, [_p]),
    "px_dev_output": (_p, [_p]),
    "px_stream_handle": (_p, [_p]),
    "px_sync": (_i, [_p]),
    "eva_dev_input": (_p, [_p]),
    "eva_run": (_i, [_p]),
    "eva_dev_output": (_p, [_p]),
    "eva_stream_handle": (_p, [_p]),
    "eva_sync": (_i, [_p]),
    "eva_profile": (_i, [_p, _p]),
    "eva_profile_opname": (C.c_char_p, [_i]),
    "eva_img_over_white": (_i, [_p, C.c_size_t, _u32, _u32, _p]),
    "eva_img_pyramid_bytes": (C.c_size_t, [_u32, _u32, _u32]),
    "eva_img_pyramid": (_i, [_p, _p, C.c_size_t, _u32, _p]),
    "eva_img_prep_bytes": (C.c_size_t, [_u32, _u32]),
    "eva_img_prep": (_i, [_p, _u32, _u32, _u32, _u32, _u32, _p, C.c_size_t, _p, _p]),
    "eva_img_prep_static": (_i, [_p, _u32, _u32, _u32, _u32, _u32, _p, _p]),
    "eva_probe_mfma_fp8": (_i, [_i, _i, _p, _p]),
    "eva_probe_copy": (_i, [_p, _p, C.c_size_t, _p]),
    "eva_probe_lds": (_i, [_i, _i, _p, _p]),
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


class EvaPyr(C.Structure):
    """eva_pyr of include/xtag_eva.h: device RGBX levels of an image (pi_pyr, src/core/procimg.h:468-472)."""
    _fields_ = [("lv", C.c_void_p * 12), ("ls", C.c_size_t * 12), ("lw", C.c_uint32 * 12), ("lh", C.c_uint32 * 12),
                ("nlv", C.c_uint32)]
