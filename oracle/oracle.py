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
    "xo_img_over_white": (None, [_p, C.c_size_t, _p, C.c_size_t, _u32, _u32]),
    "xo_img_half": (None, [_p, C.c_size_t, _p, C.c_size_t, _u32, _u32]),
    "xo_img_levels": (_u32, [_u32, _u32, _u32, _p, _p]),
    "xo_img_level": (_u32, [_u32, _u32, _u32]),
    "xo_img_lsrc": (None, [_u32, _p, _p, _p, _p, _p, _p]),
    "xo_img_mt": (_u32, [_u32, _u32]),
    "xo_img_axis": (None, [_u32, _u32, _u32, _u32, _u32, _f, _f, _p, _p, _p, _p]),
    "xo_img_prep": (None, [_p, C.c_size_t, _u32, _u32, _u32, _p]),
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
    "xo_gemm_rr_f64_rows": (None, [_p, _i, _p, _i, _p, _p, _i, _i, _i, _p, _i, _p]),
    "xo_gemm_bs_f32": (None, [_p, _i, _p, _i, _p, _p, _i, _i, _i, _i, _p, _p, _i, _i, _i]),
    "xo_max_threads": (_i, []),
    "xo_ln_quant": (None, [_p, _p, _p, _i, _p, _p, _i, _p]),
    "xo_qkv_epi": (None, [_p, _i, _p, _p, _p, _p]),
    "xo_attention": (None, [_p, _p, _p, _i, _p, _i]),
    "xo_attention_seq": (None, [_p, _p, _p, _i, _i, _i, _i, _p, _i]),
    "xo_fc1_epi": (None, [_p, _i, _p, _p]),
    "xo_fc2_epi": (None, [_p, _i, _p, _p, _p, _p]),
    "xo_oproj_epi": (None, [_p, _i, _p]),
    "xo_px_qkv_epi": (None, [_p, _i, _i, _p, _p, _p, _p, _p]),
    "xo_px_res_epi": (None, [_p, _i, _p, _p]),
    "xo_px_fc1_epi": (None, [_p, _i, _p, _p, _p]),
    "xo_px_hln": (None, [_p, _i, _i, _p, _p, _p, _p, _p, _p]),
    "xo_px_pe": (None, [_p, _p, _i, _p]),
    "xo_px_pembed": (None, [_p, _i, _i, _p, _p, _p, _p]),
    "xo_px_hsoft": (None, [_p, _i, _i, _p]),
    "xo_px_hpool_hv": (None, [_p, _p, _i, _i, _p, _p]),
    "xo_embed": (None, [_p, _p, _p, _i, _p]),
    "xo_pool": (None, [_p, _i, _p]),
    "xo_lnh": (None, [_p, _p, _p, _i, _p, _p, _p, _i]),
    "xo_fold_w2": (None, [_p, _i, _p, _p, _p, _p]),
    "xo_fold_c": (None, [_p, _p, _p]),
    "xo_forward": (_i, [_p, _p, _i, _i, _p, _p, _i]),
    "xo_prune24": (None, [_p, _i, _i, _i]),
    "xo_pack24": (_i, [_p, _i, _i, _p, _p]),
    "xo_lcg_frand": (None, [_p, C.c_size_t, _p]),
    "xo_lcg_e4m3": (None, [_p, C.c_size_t, _p]),
}
for _n, (_r, _a) in _SIGS.items():
    _fn = getattr(lib, _n)
    _fn.restype = _r
    _fn.argtypes = _a


_LIVE = []   # arrays whose addresses were handed out for the C call in progress


def _ptr(a):
    """Address of a numpy array; the array is kept alive until the next _done() (so temporaries made by _c() inline
    in a call's argument list cannot be freed before the C function reads them)."""
    if a is None:
        return None
    _LIVE.append(a)
    return C.c_void_p(a.ctypes.data)


def _done():
    _LIVE.clear()


def _c(a, dt):
    a = np.ascontiguousarray(a, dtype=dt)
    return a


def e4m3_encode_bits(first, count, threads=0):
    _done()
    out = np.empty(count, np.uint8)
    lib.xo_e4m3_encode_bits(first, count, _ptr(out), threads)
    return out


def e4m3_encode(x):
    """fp32 array -> E4M3 bytes (via the bit-pattern encoder, vectorised)."""
    _done()
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint8)
    lib.xo_e4m3_encode_n(_ptr(x), x.size, _ptr(out))
    return out


E4M3_LUT = np.array([lib.xo_e4m3_decode(i) for i in range(256)], np.float32)


def e4m3_decode(q):
    _done()
    return E4M3_LUT[np.asarray(q, np.uint8)]


def quant_act(x, lds=None):
    """x fp32 [M][K] -> (q uint8 [M][K], s fp32 [K/128][lds])."""
    _done()
    x = _c(x, np.float32)
    M, K = x.shape
    lds = lds or M
    q = np.empty((M, K), np.uint8)
    s = np.zeros((K // 128, lds), np.float32)
    lib.xo_quant_act(_ptr(x), M, K, K, _ptr(q), K, _ptr(s), lds)
    return q, s


def quant_w(w):
    """w fp32 [N][K] -> (q uint8 [ceil(N/128)*128][K], s fp32 [ceil(N/128)][K/128])."""
    _done()
    w = _c(w, np.float32)
    N, K = w.shape
    NB = (N + 127) // 128
    q = np.empty((NB * 128, K), np.uint8)
    s = np.empty((NB, K // 128), np.float32)
    lib.xo_quant_w(_ptr(w), N, K, _ptr(q), _ptr(s))
    return q, s


def gemm_f64_rows(qa, sa, qw, sw, N, rows):
    _done()
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


def gemm_rr_f64_rows(qa, sa, qw, sw, N, rows):
    """fp64 rows of the head GEMM whose weight rows carry their own 1x128 scales: qw [N][K] E4M3, sw [K/128][ldw]."""
    _done()
    qa = _c(qa, np.uint8)
    sa = _c(sa, np.float32)
    qw = _c(qw, np.uint8)
    sw = _c(sw, np.float32)
    rows = _c(rows, np.int32)
    out = np.empty((len(rows), N), np.float64)
    lib.xo_gemm_rr_f64_rows(_ptr(qa), qa.shape[1], _ptr(sa), sa.shape[1], _ptr(qw), _ptr(sw), sw.shape[1], N,
                            qa.shape[1], _ptr(rows), len(rows), _ptr(out))
    return out


def head_pack(hw16):
    """The head's fp16 rows [nt][1024] -> (q [nt][1024] E4M3, s [8][nt]): every row packed with its own 1x128 scales."""
    return quant_act(np.asarray(hw16).astype(np.float32))


def gemm_f32(qa, sa, qw, sw, N, m0=0, m1=None, threads=0, avx2=1, want_bf16=False):
    _done()
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
    _done()
    x16 = _c(x16, np.uint16)
    M = x16.shape[0]
    lds = lds or M
    q = np.empty((M, 1024), np.uint8)
    s = np.zeros((8, lds), np.float32)
    y = np.empty((M, 1024), np.float32)
    lib.xo_ln_quant(_ptr(x16), _ptr(_c(g, np.float32)), _ptr(_c(b, np.float32)), M, _ptr(q), _ptr(s), lds, _ptr(y))
    return q, s, y


def max_threads():
    _done()
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


# ---------------------------------------------------------------- EVA02-L pieces
TP = 1088


def qkv_epi(acc, nb, cs):
    _done()
    acc = _c(acc, np.float32)
    q = np.zeros((nb, 16, TP, 64), np.uint16)
    k = np.zeros((nb, 16, TP, 64), np.uint16)
    vt = np.zeros((nb, 16, 64, TP), np.uint16)
    lib.xo_qkv_epi(_ptr(acc), nb, _ptr(_c(cs, np.float32)), _ptr(q), _ptr(k), _ptr(vt))
    return q, k, vt


def attention(q, k, vt, nb, threads=0):
    _done()
    o = np.empty((nb * 1025, 1024), np.float64)
    lib.xo_attention(_ptr(_c(q, np.uint16)), _ptr(_c(k, np.uint16)), _ptr(_c(vt, np.uint16)), nb, _ptr(o), threads)
    return o


def attention_seq(q, k, vt, nseq, T, TP, qstep=1, threads=0):
    """fp64 softmax attention of nseq sequences of T tokens (padded to TP) -> o [nseq * T][1024] (rows t % qstep != 0
    are NaN)."""
    o = np.full((nseq * T, 1024), np.nan)
    lib.xo_attention_seq(_ptr(np.ascontiguousarray(q)), _ptr(np.ascontiguousarray(k)), _ptr(np.ascontiguousarray(vt)),
                         nseq, T, TP, qstep, _ptr(o), threads)
    return o


def fc1_epi(acc):
    _done()
    acc = _c(acc, np.float32)
    M = acc.shape[0]
    h = np.empty((M, 2816), np.float32)
    stat = np.empty((22, M, 2), np.float32)
    lib.xo_fc1_epi(_ptr(acc), M, _ptr(h), _ptr(stat))
    return h, stat


def fc2_epi(acc, stat, c, d, x16):
    _done()
    acc = _c(acc, np.float32)
    x = _c(x16, np.uint16).copy()
    lib.xo_fc2_epi(_ptr(acc), acc.shape[0], _ptr(_c(stat, np.float32)), _ptr(_c(c, np.float32)),
                   _ptr(_c(d, np.float32)), _ptr(x))
    return x


def oproj_epi(acc, x16):
    _done()
    acc = _c(acc, np.float32)
    x = _c(x16, np.uint16).copy()
    lib.xo_oproj_epi(_ptr(acc), acc.shape[0], _ptr(x))
    return x


def px_qkv_epi(acc, L, bias, cs):
    """PixAI qkv epilogue: acc [M][3072] natural order -> q, k [M/L][16][L][64], vt [M/L][16][64][L] bf16 bits."""
    _done()
    acc = _c(acc, np.float32)
    M = acc.shape[0]
    S = M // L
    q = np.zeros((S, 16, L, 64), np.uint16)
    k = np.zeros((S, 16, L, 64), np.uint16)
    vt = np.zeros((S, 16, 64, L), np.uint16)
    lib.xo_px_qkv_epi(_ptr(acc), M, L, _ptr(_c(bias, np.float32)), _ptr(_c(cs, np.float32)), _ptr(q), _ptr(k),
                      _ptr(vt))
    return q, k, vt


def px_res_epi(acc, bias, x16):
    _done()
    acc = _c(acc, np.float32)
    x = _c(x16, np.uint16).copy()
    lib.xo_px_res_epi(_ptr(acc), acc.shape[0], _ptr(_c(bias, np.float32)), _ptr(x))
    return x


def px_fc1_epi(acc, bias, rs=None):
    _done()
    acc = _c(acc, np.float32)
    h = np.empty((acc.shape[0], 4736), np.float32)
    lib.xo_px_fc1_epi(_ptr(acc), acc.shape[0], _ptr(_c(bias, np.float32)),
                      None if rs is None else _ptr(_c(rs, np.float32)), _ptr(h))
    return h


def px_pe(in16, pe16):
    _done()
    in16 = _c(in16, np.uint16)
    x = np.empty((in16.shape[0], 1024), np.uint16)
    lib.xo_px_pe(_ptr(in16), _ptr(_c(pe16, np.uint16)), in16.shape[0], _ptr(x))
    return x


def px_pembed(x16, T, pos, g, b):
    _done()
    x16 = _c(x16, np.uint16)
    y = np.empty_like(x16)
    lib.xo_px_pembed(_ptr(x16), x16.shape[0], T, _ptr(_c(pos, np.float32)), _ptr(_c(g, np.float32)),
                     _ptr(_c(b, np.float32)), _ptr(y))
    return y


def px_hln(x16, T, g, b, hpos16, U):
    """PixAI pool head keys / scores: (y fp16 bits [M][1024], s float64 [M][16])."""
    _done()
    x16 = _c(x16, np.uint16)
    M = x16.shape[0]
    y = np.empty((M, 1024), np.uint16)
    s = np.empty((M, 16), np.float64)
    lib.xo_px_hln(_ptr(x16), M, T, _ptr(_c(g, np.float32)), _ptr(_c(b, np.float32)), _ptr(_c(hpos16, np.uint16)),
                  _ptr(_c(U, np.float32)), _ptr(y), _ptr(s))
    return y, s


def px_hsoft(s, nb, T):
    _done()
    P = np.empty((nb, 16, T), np.float64)
    lib.xo_px_hsoft(_ptr(_c(s, np.float32)), nb, T, _ptr(P))
    return P


def px_hpool_hv(P16, y16, nb, T, wv16):
    _done()
    o = np.empty((nb, 1024), np.float64)
    lib.xo_px_hpool_hv(_ptr(_c(P16, np.uint16)), _ptr(_c(y16, np.uint16)), nb, T, _ptr(_c(wv16, np.uint16)), _ptr(o))
    return o


def embed(inp16, pe16, pos, nb):
    _done()
    x = np.zeros((nb * 1025, 1024), np.uint16)
    lib.xo_embed(_ptr(_c(inp16, np.uint16)), _ptr(_c(pe16, np.uint16)), _ptr(_c(pos, np.float32)), nb, _ptr(x))
    return x


def pool(x16, nb):
    _done()
    p = np.empty((nb, 1024), np.float32)
    lib.xo_pool(_ptr(_c(x16, np.uint16)), nb, _ptr(p))
    return p


def lnh(p, g, b, lds=None):
    _done()
    p = _c(p, np.float32)
    nb = p.shape[0]
    lds = lds or nb
    pn = np.empty((nb, 1024), np.uint16)
    q = np.empty((nb, 1024), np.uint8)
    s = np.zeros((8, lds), np.float32)
    lib.xo_lnh(_ptr(p), _ptr(_c(g, np.float32)), _ptr(_c(b, np.float32)), nb, _ptr(pn), _ptr(q), _ptr(s), lds)
    return pn, q, s


def fold_w2(w2_16, gamma, beta):
    _done()
    w2 = _c(w2_16, np.uint16)
    wt = np.empty((1024, 2816), np.float32)
    d = np.empty(1024, np.float32)
    lib.xo_fold_w2(_ptr(w2), w2.shape[1], _ptr(_c(gamma, np.float32)), _ptr(_c(beta, np.float32)), _ptr(wt), _ptr(d))
    return wt, d


def fold_c(q, s):
    _done()
    c = np.empty(1024, np.float32)
    lib.xo_fold_c(_ptr(_c(q, np.uint8)), _ptr(_c(s, np.float32)), _ptr(c))
    return c


class _Model(C.Structure):
    _fields_ = [("pe", C.c_void_p), ("pos", C.c_void_p), ("cs", C.c_void_p),
                ("ln1w", C.c_void_p * 24), ("ln1b", C.c_void_p * 24), ("ln2w", C.c_void_p * 24),
                ("ln2b", C.c_void_p * 24), ("mlnw", C.c_void_p * 24), ("mlnb", C.c_void_p * 24),
                ("wqkv", C.c_void_p * 24), ("wo", C.c_void_p * 24), ("w12", C.c_void_p * 24), ("w2", C.c_void_p * 24),
                ("fnw", C.c_void_p), ("fnb", C.c_void_p), ("hw", C.c_void_p), ("hb", C.c_void_p), ("nt", C.c_int),
                ("sparse", C.c_int)]


def prune24(q, wanda=False):
    """2:4 pruning of E4M3 weights q [N][K] along K (a copy; see xo_prune24)."""
    _done()
    q = np.array(q, dtype=np.uint8, order="C", copy=True)
    lib.xo_prune24(_ptr(q), q.shape[0], q.shape[1], 1 if wanda else 0)
    return q


def pack24(q):
    """Compressed 2:4 layout (vals [N/16][K/128][64][16] u8, idx [N/16][K/128][64] u32) of pruned E4M3 q [N][K]."""
    _done()
    q = np.ascontiguousarray(q, dtype=np.uint8)
    N, K = q.shape
    vals = np.empty((N // 16, K // 128, 64, 16), np.uint8)
    idx = np.empty((N // 16, K // 128, 64), np.uint32)
    if lib.xo_pack24(_ptr(q), N, K, _ptr(vals), _ptr(idx)) != 0:
        raise ValueError("a group of 4 holds more than 2 nonzero bytes")
    return vals, idx


def forward(m, inp16, nl=24, threads=0, sparse=False):
    """Full oracle forward from model tensors m (xtagger_amd.blob layout) on fp16 inputs [nb][1024][592];
    sparse: the layer GEMM weights are 2:4-pruned (magnitude) after packing."""
    _done()
    keep = []

    def P(a, dt):
        a = np.ascontiguousarray(a, dtype=dt)
        keep.append(a)
        return a.ctypes.data

    md = _Model()
    md.pe, md.pos, md.cs = P(m["pe"].view(np.uint16), np.uint16), P(m["pos"], np.float32), P(m["rope"], np.float32)
    for i, L in enumerate(m["layers"][:nl]):
        md.ln1w[i], md.ln1b[i] = P(L["ln1w"], np.float32), P(L["ln1b"], np.float32)
        md.ln2w[i], md.ln2b[i] = P(L["ln2w"], np.float32), P(L["ln2b"], np.float32)
        md.mlnw[i], md.mlnb[i] = P(L["mlnw"], np.float32), P(L["mlnb"], np.float32)
        md.wqkv[i], md.wo[i] = P(L["wqkv"].view(np.uint16), np.uint16), P(L["wo"].view(np.uint16), np.uint16)
        md.w12[i], md.w2[i] = P(L["w12"].view(np.uint16), np.uint16), P(L["w2"].view(np.uint16), np.uint16)
    md.fnw, md.fnb = P(m["fnw"], np.float32), P(m["fnb"], np.float32)
    md.hw, md.hb = P(m["hw"].view(np.uint16), np.uint16), P(m["hb"], np.float32)
    md.nt = m["nt"]
    md.sparse = 1 if sparse else 0
    x = np.ascontiguousarray(inp16, dtype=np.float16).view(np.uint16)
    nb = x.shape[0]
    out = np.empty((nb, m["nt"]), np.float32)
    pn = np.empty((nb, 1024), np.uint16)
    lib.xo_forward(C.byref(md), _ptr(x), nb, nl, _ptr(out), _ptr(pn), threads)
    return out, pn


# ---- patch-operand producer (src/core/procimg.h; xt_img.c) ----
def img_over_white(rgba):
    """RGBA uint8 [h][w][4] -> RGBX over white (pi_row_rgbx with alpha)."""
    rgba = np.ascontiguousarray(rgba, np.uint8)
    h, w = rgba.shape[:2]
    out = np.empty_like(rgba)
    lib.xo_img_over_white(_ptr(out), w * 4, _ptr(rgba), w * 4, w, h)
    return out


def img_pyramid(rgbx, S=448):
    """Levels 0.. of pi_pyramid: a list of RGBX uint8 [lh][lw][4] arrays (level 0 is the input)."""
    rgbx = np.ascontiguousarray(rgbx, np.uint8)
    h, w = rgbx.shape[:2]
    lw, lh = np.zeros(12, np.uint32), np.zeros(12, np.uint32)
    n = lib.xo_img_levels(w, h, S, _ptr(lw), _ptr(lh))
    lv = [rgbx]
    for L in range(1, n):
        d = np.empty((int(lh[L]), int(lw[L]), 4), np.uint8)
        s = lv[L - 1]
        lib.xo_img_half(_ptr(d), int(lw[L]) * 4, _ptr(s), s.shape[1] * 4, int(lw[L]), int(lh[L]))
        lv.append(d)
    return lv


def img_prep(levels, x0, y0, cw, ch, S=448):
    """pi_prep of the level-0 rect (x0, y0, cw, ch): the level choice, the rect on that level, the resample (or the
    identity at side == S) -> fp16 bits [(S/14)^2][592]. Also returns (level, x0, y0, cw, ch) on that level."""
    lw = np.array([l.shape[1] for l in levels] + [0] * (12 - len(levels)), np.uint32)
    lh = np.array([l.shape[0] for l in levels] + [0] * (12 - len(levels)), np.uint32)
    L = lib.xo_img_level(len(levels), max(cw, ch), S)
    r = [C.c_uint32(v) for v in (x0, y0, cw, ch)]
    lib.xo_img_lsrc(L, _ptr(lw), _ptr(lh), C.byref(r[0]), C.byref(r[1]), C.byref(r[2]), C.byref(r[3]))
    x0, y0, cw, ch = (v.value for v in r)
    src = levels[L]
    out = np.empty(((S // 14) ** 2, 592), np.uint16)
    lib.xo_img_prep(C.c_void_p(src.ctypes.data + (y0 * src.shape[1] + x0) * 4), src.shape[1] * 4, cw, ch, S, _ptr(out))
    return out, (L, x0, y0, cw, ch)


def img_axis(S, side, off, length, sc, add):
    """pi_axis: weights [S][mt], first tap s [S], taps n [S], constant k [S]."""
    mt = lib.xo_img_mt(side, S)
    w = np.zeros((S, mt), np.float32)
    s, n = np.zeros(S, np.int32), np.zeros(S, np.int32)
    k = np.zeros(S, np.float32)
    lib.xo_img_axis(S, side, off, length, mt, sc, add, _ptr(w), _ptr(s), _ptr(n), _ptr(k))
    return w, s, n, k
