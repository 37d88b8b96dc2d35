"""ctypes binding of liboracle.so, the CPU restatement of the reference path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
product (xtagger_amd/).
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SO = os.path.join(HERE, "liboracle.so")


def build():
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE], check=True)


if not os.path.exists(SO):
    build()
lib = C.CDLL(SO)

_p, _i, _u32, _f, _u8, _u16 = C.c_void_p, C.c_int, C.c_uint32, C.c_float, C.c_uint8, C.c_uint16
_SIGS = {
    "xo_e4m3_encode": (_u8, [_f]),
    "xo_e4m3_decode": (_f, [_u8]),
    "xo_e4m3_encode_bits": (None, [_u32, _u32, _p, _i]),
    "xo_e4m3_encode_n": (None, [_p, C.c_size_t, _p]),
    "xo_f32_to_bf16": (_u16, [_f]),
    "xo_bf16_to_f32": (_f, [_u16]),
    "xo_f32_to_f16": (_u16, [_f]),
    "xo_f16_to_f32": (_f, [_u16]),
    "xo_block_scale": (_f, [_f]),
    "xo_quant_act": (None, [_p, _i, _i, _i, _p, _i, _p, _i]),
    "xo_quant_w": (None, [_p, _i, _i, _p, _p]),
    "xo_gemm_bs_f64_rows": (None, [_p, _i, _p, _i, _p, _p, _i, _i, _p, _i, _p]),
    "xo_gemm_bs_f32": (None, [_p, _i, _p, _i, _p, _p, _i, _i, _i, _i, _p, _p, _i, _i, _i]),
    "xo_max_threads": (_i, []),
    "xo_ln_quant": (None, [_p, _p, _p, _i, _p, _p, _i, _p]),
    "xo_lcg_frand": (None, [_p, C.c_size_t, _p]),
    "xo_lcg_e4m3": (None, [_p, C.c_size_t, _p]),
}
for _n, (_r, _a) in _SIGS.items():
    _fn = getattr(lib, _n)
    _fn.restype = _r
    _fn.argtypes = _a


def _ptr(a):
    return None if a is None else C.c_void_p(a.ctypes.data)


def _c(a, dt):
    a = np.ascontiguousarray(a, dtype=dt)
    return a


def e4m3_encode_bits(first, count, threads=0):
    out = np.empty(count, np.uint8)
    lib.xo_e4m3_encode_bits(first, count, _ptr(out), threads)
    return out


def e4m3_encode(x):
    """fp32 array -> E4M3 bytes (via the bit-pattern encoder, vectorised)."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint8)
    lib.xo_e4m3_encode_n(_ptr(x), x.size, _ptr(out))
    return out


E4M3_LUT = np.array([lib.xo_e4m3_decode(i) for i in range(256)], np.float32)


def e4m3_decode(q):
    return E4M3_LUT[np.asarray(q, np.uint8)]


def quant_act(x, lds=None):
    """x fp32 [M][K] -> (q uint8 [M][K], s fp32 [K/128][lds])."""
    x = _c(x, np.float32)
    M, K = x.shape
    lds = lds or M
    q = np.empty((M, K), np.uint8)
    s = np.zeros((K // 128, lds), np.float32)
    lib.xo_quant_act(_ptr(x), M, K, K, _ptr(q), K, _ptr(s), lds)
    return q, s


def quant_w(w):
    """w fp32 [N][K] -> (q uint8 [ceil(N/128)*128][K], s fp32 [ceil(N/128)][K/128])."""
    w = _c(w, np.float32)
    N, K = w.shape
    NB = (N + 127) // 128
    q = np.empty((NB * 128, K), np.uint8)
    s = np.empty((NB, K // 128), np.float32)
    lib.xo_quant_w(_ptr(w), N, K, _ptr(q), _ptr(s))
    return q, s


def gemm_f64_rows(qa, sa, qw, sw, N, rows):
    qa = _c(qa, np.uint8)
    sa = _c(sa, np.float32)
    qw = _c(qw, np.uint8)
    sw = _c(sw, np.float32)
    rows = _c(rows, np.int32)
    K = qa.shape[1]
    out = np.empty((rows.size, N), np.float64)
    lib.xo_gemm_bs_f64_rows(_ptr(qa), K, _ptr(sa), sa.shape[1], _ptr(qw), _ptr(sw), N, K, _ptr(rows), rows.size,
                            _ptr(out))
    return out


def gemm_f32(qa, sa, qw, sw, N, m0=0, m1=None, threads=0, avx2=1, want_bf16=False):
    qa = _c(qa, np.uint8)
    sa = _c(sa, np.float32)
    qw = _c(qw, np.uint8)
    sw = _c(sw, np.float32)
    M, K = qa.shape
    m1 = M if m1 is None else m1
    cf = np.zeros((M, N), np.float32)
    cb = np.zeros((M, N), np.uint16) if want_bf16 else None
    lib.xo_gemm_bs_f32(_ptr(qa), K, _ptr(sa), sa.shape[1], _ptr(qw), _ptr(sw), N, K, m0, m1, _ptr(cf), _ptr(cb), N,
                       threads, avx2)
    return (cf, cb) if want_bf16 else cf


def ln_quant(x16, g, b, lds=None):
    """x fp16 bits uint16 [M][1024] -> (q [M][1024], s [8][lds], y fp32 [M][1024])."""
    x16 = _c(x16, np.uint16)
    M = x16.shape[0]
    lds = lds or M
    q = np.empty((M, 1024), np.uint8)
    s = np.zeros((8, lds), np.float32)
    y = np.empty((M, 1024), np.float32)
    lib.xo_ln_quant(_ptr(x16), _ptr(_c(g, np.float32)), _ptr(_c(b, np.float32)), M, _ptr(q), _ptr(s), lds, _ptr(y))
    return q, s, y


def max_threads():
    return lib.xo_max_threads()


class Lcg:
    """kcheck.c:21-22 generator with state in C (fast bulk draws)."""

    def __init__(self, seed=12345):
        self.rs = np.array([seed], np.uint32)

    def frand(self, n):
        out = np.empty(n, np.float32)
        lib.xo_lcg_frand(_ptr(self.rs), n, _ptr(out))
        return out

    def e4m3(self, n):
        out = np.empty(n, np.uint8)
        lib.xo_lcg_e4m3(_ptr(self.rs), n, _ptr(out))
        return out
