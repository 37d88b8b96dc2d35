"""GPU parity of the EVA02-L layer kernels (LayerNorm, qkv + RoPE, attention, out-projection, fc1 + SwiGLU, fc2 +
folded LN, patch embed, pool, final LN, head, weight preparation) against the oracle, through the C-ABI.

Bit-exact where the kernel's arithmetic is restated in the oracle step for step (LayerNorm, pool, final LN, weight
packing, fold terms, attention output packing given the kernel's fp32 output). Where a fused epilogue follows a
block-scaled GEMM, the oracle applies the same epilogue to the fp64 product of the same packed operands, and the
check is a tolerance: the matrix core's summation differs from fp64 by ~1e-5 relative, which can move a value across
one bf16 / fp16 / E4M3 rounding boundary.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

T, D, TP, HIDP = 1025, 1024, 1088, 2816


def _say(*a):
    print(*a, flush=True)


def _st():
    return torch.cuda.current_stream().cuda_stream


def _ok(rc, what):
    assert rc == 0, f"{what} returned {rc}"
    torch.cuda.synchronize()


_KEEP = []                                                   # device copies stay alive until the test ends


@pytest.fixture(autouse=True)
def _release_device_copies():
    yield
    _KEEP.clear()


def _d(a, dev):
    t = a.to(dev) if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    _KEEP.append(t)
    return t


def _ulp_diff_f16(a, b):
    a = a.view(np.int16).astype(np.int32)
    b = b.view(np.int16).astype(np.int32)
    a = np.where(a < 0, -32768 - a, a)
    b = np.where(b < 0, -32768 - b, b)
    return np.abs(a - b)


def _ulp_diff_bf16(a, b):
    return _ulp_diff_f16(a, b)  # same ordering trick on 16-bit sign-magnitude patterns


def _bf16_f32(u16):
    return (np.asarray(u16, np.uint32) << 16).view(np.float32)


def _f16_f32(u16):
    return np.asarray(u16, np.uint16).view(np.float16).astype(np.float32)


def _check_close(name, got, ref, scale, unit):
    """|got - ref| <= unit * |ref| + 2e-4 * scale: one rounding unit of the output type (2^-7 bf16, 2^-10 fp16) plus
    the GEMM summation difference (the matrix core vs fp64, ~1e-5 of the terms), which dominates where terms cancel."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    bound = unit * np.abs(ref) + 2e-4 * scale
    worst = float((err / bound).max())
    _say(f"  {name}: worst err / bound {worst:.3f}, elements differing {np.mean(err > 0):.2e}")
    assert worst <= 1.0, name


def _packed_act(orc, M, K, seed, scale=1.0):
    r = np.random.default_rng(seed)
    x = (r.standard_normal((M, K)) * scale).astype(np.float32)
    q, s = orc.quant_act(x)
    return x, q, s


def _packed_w(orc, N, K, seed, std=0.02):
    r = np.random.default_rng(seed)
    w = (r.standard_normal((N, K)) * std).astype(np.float32)
    q, s = orc.quant_w(w)
    return w, q, s


# ---------------------------------------------------------------- LayerNorm / pool / final LN: bit-exact
@pytest.mark.parametrize("M", [1025, 37, 1, 6145, 14000])
def test_ln_bitexact(dev, xt, orc, M):
    """k_ln against the oracle, bytes and scales. Above 4 x 6 x (CUs) rows the resident grid's waves take several rows
    each (M = 6145: one wave a second row on a 256-CU part; 14000: two or three rows a wave)."""
    _say(f"k_ln M={M}")
    r = np.random.default_rng(M)
    x = (r.standard_normal((M, D)) * 2 + 0.3).astype(np.float16)
    x[0, :] = 1.0                                            # constant row: variance 0
    g = (1 + 0.1 * r.standard_normal(D)).astype(np.float32)
    b = (0.02 * r.standard_normal(D)).astype(np.float32)
    lds = M + 5
    d_q = torch.zeros((M, D), dtype=torch.uint8, device=dev)
    d_s = torch.zeros((8, lds), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_ln(xt.ptr(_d(x, dev)), xt.ptr(_d(g, dev)), xt.ptr(_d(b, dev)), xt.ptr(d_q), xt.ptr(d_s), M, lds,
                        _st()), "eva_k_ln")
    q, s, _ = orc.ln_quant(x.view(np.uint16), g, b, lds=lds)
    assert (d_q.cpu().numpy() == q).all()
    assert (d_s.cpu().numpy() == s).all()


def test_pool_lnh_bitexact(dev, xt, orc):
    nb = 3
    _say("k_pool + k_lnh")
    r = np.random.default_rng(9)
    x = (r.standard_normal((nb * T, D)) * 3).astype(np.float16)
    g = (1 + 0.1 * r.standard_normal(D)).astype(np.float32)
    b = (0.02 * r.standard_normal(D)).astype(np.float32)
    d_p = torch.zeros((nb, D), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_pool(xt.ptr(_d(x, dev)), xt.ptr(d_p), nb, _st()), "eva_k_pool")
    p = orc.pool(x.view(np.uint16), nb)
    assert (d_p.cpu().numpy() == p).all()
    d_pn = torch.zeros((nb, D), dtype=torch.int16, device=dev)
    d_q = torch.zeros((nb, D), dtype=torch.uint8, device=dev)
    d_s = torch.zeros((8, 4), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_lnh(xt.ptr(d_p), xt.ptr(_d(g, dev)), xt.ptr(_d(b, dev)), xt.ptr(d_pn), xt.ptr(d_q), xt.ptr(d_s),
                         nb, 4, _st()), "eva_k_lnh")
    pn, q, s = orc.lnh(p, g, b, lds=4)
    assert (d_pn.cpu().numpy().view(np.uint16) == pn).all()
    assert (d_q.cpu().numpy() == q).all()
    assert (d_s.cpu().numpy() == s).all()


# ---------------------------------------------------------------- weight preparation: bit-exact
def test_prep_qkv_pair_split_bitexact(dev, xt, orc):
    _say("eva_k_prep_w qkv")
    r = np.random.default_rng(11)
    w16 = (r.standard_normal((3 * D, D)) * 0.02).astype(np.float16)
    d_q = torch.zeros((3 * D, D), dtype=torch.uint8, device=dev)
    d_s = torch.zeros((24, 8), dtype=torch.float32, device=dev)
    scratch = torch.empty((3 * D, D), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_prep_w(xt.ptr(_d(w16, dev)), D, 3 * D, D, 3 * D, D, 1, None, xt.ptr(scratch), xt.ptr(d_q),
                            xt.ptr(d_s), _st()), "eva_k_prep_w")
    q, s = orc.quant_w(w16.astype(np.float32))               # natural order
    # the split only permutes rows inside each 64-row head of q and k: same scales, permuted codes
    assert (d_s.cpu().numpy() == s).all()
    perm = np.arange(3 * D)
    for h in range(32):
        for pc in range(64):
            j, i = pc >> 4, pc & 15
            perm[h * 64 + pc] = h * 64 + 4 * i + j         # column tile j, lane i: dim 4 i + j
    assert (d_q.cpu().numpy() == q[perm]).all()


def test_prep_w8_v3_bitexact(dev, xt, orc):
    """eva_k_prep_w8: the v3 blob's E4M3 bytes with one scale per tensor (export_eva.py:64-66) into the kernels'
    layout: qkv rows quad-split as eva_k_prep_w's perm 1, W12 and W~2 zero-padded to 2816 units; every block scale is
    the tensor's. eva_k_fold_c_rs: c = sum_k dec(q) s rs against float64."""
    _say("eva_k_prep_w8 + eva_k_fold_c_rs")
    r = np.random.default_rng(13)
    perm = np.arange(3 * D)
    for h in range(32):
        for pc in range(64):
            j, i = pc >> 4, pc & 15
            perm[h * 64 + pc] = h * 64 + 4 * i + j         # column tile j, lane i: dim 4 i + j
    q = r.integers(0, 256, (3 * D, D)).astype(np.uint8)
    q[(q & 0x7F) == 0x7F] = 0                                 # no NaN codes in a blob
    d_q = torch.zeros((3 * D, D), dtype=torch.uint8, device=dev)
    d_s = torch.zeros((24, 8), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_prep_w8(xt.ptr(_d(q, dev)), D, 3 * D, D, 3 * D, D, 1, 0.0123, xt.ptr(d_q), xt.ptr(d_s), _st()),
        "prep_w8 qkv")
    assert (d_q.cpu().numpy() == q[perm]).all() and (d_s.cpu().numpy() == np.float32(0.0123)).all()
    w2 = r.integers(0, 0x7F, (D, 2736)).astype(np.uint8) | (r.integers(0, 2, (D, 2736)).astype(np.uint8) << 7)
    w2[:, 2730:] = 0
    d_q2 = torch.full((D, HIDP), 0xAB, dtype=torch.uint8, device=dev)
    d_s2 = torch.zeros((8, 22), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_prep_w8(xt.ptr(_d(w2, dev)), 2736, D, 2730, D, HIDP, 0, 3e-4, xt.ptr(d_q2), xt.ptr(d_s2), _st()),
        "prep_w8 w2")
    ref = np.zeros((D, HIDP), np.uint8)
    ref[:, :2730] = w2[:, :2730]
    assert (d_q2.cpu().numpy() == ref).all() and (d_s2.cpu().numpy() == np.float32(3e-4)).all()
    rs = np.zeros(HIDP, np.float32)
    rs[:2730] = np.exp(r.uniform(-3, 3, 2730))
    d_c = torch.zeros(D, dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_fold_c_rs(xt.ptr(d_q2), xt.ptr(d_s2), xt.ptr(_d(rs, dev)), xt.ptr(d_c), _st()), "fold_c_rs")
    dec = orc.e4m3_decode(ref).astype(np.float64) * np.float64(np.float32(3e-4))
    c64 = dec @ rs.astype(np.float64)
    terms = np.abs(dec) @ rs.astype(np.float64)
    assert (np.abs(d_c.cpu().numpy() - c64) <= 1e-5 * terms).all()


def test_prep_fc_fold_bitexact(dev, xt, orc):
    _say("eva_k_prep_w w12 / w2 fold + eva_k_fold_cd")
    r = np.random.default_rng(12)
    w12 = (r.standard_normal((2 * 2736, D)) * 0.02).astype(np.float16)
    d_q = torch.zeros((2 * HIDP, D), dtype=torch.uint8, device=dev)
    d_s = torch.zeros((44, 8), dtype=torch.float32, device=dev)
    scratch = torch.empty((2 * HIDP, D), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_prep_w(xt.ptr(_d(w12, dev)), D, 2 * 2736, D, 2 * HIDP, D, 0, None, xt.ptr(scratch), xt.ptr(d_q),
                            xt.ptr(d_s), _st()), "prep w12")
    wpad = np.zeros((2 * HIDP, D), np.float32)
    wpad[:2 * 2736] = w12.astype(np.float32)
    q, s = orc.quant_w(wpad)
    assert (d_q.cpu().numpy() == q).all() and (d_s.cpu().numpy() == s).all()

    w2 = np.zeros((D, 2736), np.float16)
    w2[:, :2730] = (r.standard_normal((D, 2730)) * 0.02).astype(np.float16)
    gamma = np.zeros(2736, np.float32)
    beta = np.zeros(2736, np.float32)
    gamma[:2730] = 1 + 0.1 * r.standard_normal(2730)
    beta[:2730] = 0.02 * r.standard_normal(2730)
    d_q2 = torch.zeros((D, HIDP), dtype=torch.uint8, device=dev)
    d_s2 = torch.zeros((8, 22), dtype=torch.float32, device=dev)
    d_w2, d_gamma, d_beta = _d(w2, dev), _d(gamma, dev), _d(beta, dev)
    _ok(xt.lib.eva_k_prep_w(xt.ptr(d_w2), 2736, D, 2730, D, HIDP, 0, xt.ptr(d_gamma), xt.ptr(scratch), xt.ptr(d_q2),
                            xt.ptr(d_s2), _st()), "prep w2")
    wt, dref = orc.fold_w2(w2.view(np.uint16), gamma, beta)
    q2, s2 = orc.quant_w(wt)
    assert (d_q2.cpu().numpy() == q2).all() and (d_s2.cpu().numpy() == s2).all()
    d_c = torch.zeros(D, dtype=torch.float32, device=dev)
    d_dd = torch.zeros(D, dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_fold_cd(xt.ptr(d_q2), xt.ptr(d_s2), xt.ptr(d_w2), 2736, xt.ptr(d_beta), xt.ptr(d_c), xt.ptr(d_dd),
                             _st()), "fold_cd")
    cref = orc.fold_c(q2, s2)
    assert (d_c.cpu().numpy() == cref).all()
    assert (d_dd.cpu().numpy() == dref).all()
    # the fold identity: LN(h) W2^T = rstd (h W~^T - mean c) + d with unpacked W~ (export_eva.py:101-104)
    h = r.standard_normal((4, 2730)).astype(np.float64) * 0.3
    mu, var = h.mean(1, keepdims=True), h.var(1, keepdims=True)
    ln = (h - mu) / np.sqrt(var + 1e-6) * gamma[:2730] + beta[:2730]
    w2d = w2[:, :2730].astype(np.float64)
    lhs = ln @ w2d.T
    wtd = wt[:, :2730].astype(np.float64)
    rhs = (h @ wtd.T - mu * wtd.sum(1)) / np.sqrt(var + 1e-6) + w2d @ beta[:2730].astype(np.float64)
    assert np.allclose(lhs, rhs, rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- fused GEMM epilogues
def _acc_ref(orc, qa, sa, qw, sw, N):
    return orc.gemm_f64_rows(qa, sa, qw, sw, N, np.arange(qa.shape[0])).astype(np.float32)


def test_qkv_rope_layouts(dev, xt, orc):
    nb = 2
    M = nb * T
    _say("k_qkv")
    _, qa, sa = _packed_act(orc, M, D, 21)
    r = np.random.default_rng(22)
    w16 = (r.standard_normal((3 * D, D)) * 0.02).astype(np.float16)
    ang = r.random((1024, 32)) * 6.28
    cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    d_wq = torch.zeros((3 * D, D), dtype=torch.uint8, device=dev)
    d_ws = torch.zeros((24, 8), dtype=torch.float32, device=dev)
    scratch = torch.empty((3 * D, D), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_prep_w(xt.ptr(_d(w16, dev)), D, 3 * D, D, 3 * D, D, 1, None, xt.ptr(scratch), xt.ptr(d_wq),
                            xt.ptr(d_ws), _st()), "prep")
    kw = [torch.zeros((nb, 16, TP, 64), dtype=torch.int16, device=dev) for _ in range(2)]
    d_vt = torch.zeros((nb, 16, 64, TP), dtype=torch.int16, device=dev)
    _ok(xt.lib.eva_k_qkv(xt.ptr(_d(qa, dev)), xt.ptr(_d(sa, dev)), M, xt.ptr(d_wq), xt.ptr(d_ws), xt.ptr(_d(cs, dev)),
                         xt.ptr(kw[0]), xt.ptr(kw[1]), xt.ptr(d_vt), M, _st()), "eva_k_qkv")
    qw, sw = orc.quant_w(w16.astype(np.float32))
    acc = _acc_ref(orc, qa, sa, qw, sw, 3 * D)
    q, k, vt = orc.qkv_epi(acc, nb, cs)
    scale = np.abs(acc).max()
    for name, got, ref in (("q", kw[0], q), ("k", kw[1], k), ("vt", d_vt, vt)):
        g = got.cpu().numpy().view(np.uint16)
        _check_close(name, _bf16_f32(g), _bf16_f32(ref), scale, 2.0 ** -7)
    # padded rows untouched
    assert (kw[0].cpu().numpy()[:, :, T:] == 0).all() and (d_vt.cpu().numpy()[:, :, :, T:] == 0).all()


def _attn_inputs(nb, seed):
    r = np.random.default_rng(seed)
    q = np.zeros((nb, 16, TP, 64), np.float32)
    k = np.zeros((nb, 16, TP, 64), np.float32)
    vt = np.zeros((nb, 16, 64, TP), np.float32)
    q[:, :, :T] = r.standard_normal((nb, 16, T, 64)) * 0.6
    k[:, :, :T] = r.standard_normal((nb, 16, T, 64)) * 0.6
    vt[:, :, :, :T] = r.standard_normal((nb, 16, 64, T))
    q[0, 3, 5] *= 12.0                                        # peaked rows far above their first key tile
    k[0, 3, 700] = q[0, 3, 5]                                 # raise the offset
    q[0, 7, 100] *= 12.0                                      # ... one whose maximum is the last key, which the
    k[0, 7, T - 1] = q[0, 7, 100]                             # kernel adds after the 16 tiles of 64 keys
    q[0, 9, T - 1] *= 12.0                                    # and the last query, alone in its query block
    k[0, 9, 3] = q[0, 9, T - 1]
    b = nb - 1
    q[b, 2, 50] *= 12.0                                       # a peak in an odd key tile (the loop's second stage)
    k[b, 2, 750] = q[b, 2, 50]
    q[b, 5, 10] *= 12.0                                       # a first key tile far below the row's other scores
    k[b, 5, :64] = -2.0 * q[b, 5, 10]
    k[b, 6, 500] = 20.0 * q[b, 6, 40]                         # an ordinary first tile, then one key 2^460 above it
    # the last query (its block's only one: the key tiles are split over four waves per head and merged)
    q[b, 11, T - 1] *= 12.0                                   # its maximum in a tile of the third wave
    k[b, 11, 900] = q[b, 11, T - 1]
    q[b, 13, T - 1] *= 12.0                                   # its maximum at the last key, added after the tiles
    k[b, 13, T - 1] = q[b, 13, T - 1]
    q[b, 14, T - 1] *= 8.0                                    # every tile of the second wave far below the rest
    for kt in (1, 5, 9, 13):
        k[b, 14, 64 * kt:64 * kt + 64] = -2.0 * q[b, 14, T - 1]
    bf = lambda a: torch.from_numpy(a).to(torch.bfloat16)
    return bf(q), bf(k), bf(vt)


def test_flash_parity(dev, xt, orc):
    nb = 2
    M = nb * T
    _say("k_flash")
    q, k, vt = _attn_inputs(nb, 31)
    lds = M + 7
    d_o8 = torch.zeros((M, D), dtype=torch.uint8, device=dev)
    d_os = torch.zeros((8, lds), dtype=torch.float32, device=dev)
    d_o32 = torch.zeros((M, D), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_flash(xt.ptr(_d(q, dev)), xt.ptr(_d(k, dev)), xt.ptr(_d(vt, dev)), xt.ptr(d_o8), xt.ptr(d_os), lds,
                           nb, xt.ptr(d_o32), _st()), "eva_k_flash")
    ref = orc.attention(q.view(torch.int16).numpy(), k.view(torch.int16).numpy(), vt.view(torch.int16).numpy(), nb)
    _say("  flash vs fp64 softmax:")
    o = d_o32.cpu().numpy().astype(np.float64)
    err = np.abs(o - ref)
    rel = err.max() / np.abs(ref).max()
    _say(f"  o32 max err / max|ref| {rel:.3g}, normwise {np.linalg.norm(o - ref) / np.linalg.norm(ref):.3g}")
    # P enters the PV product in bf16 (relative 2^-9 per weight)
    assert rel <= 4e-3
    assert np.linalg.norm(o - ref) <= 2e-3 * np.linalg.norm(ref)
    # packing of the kernel's own fp32 output is bit-exact
    q8, s8 = orc.quant_act(d_o32.cpu().numpy(), lds=lds)
    assert (d_o8.cpu().numpy() == q8).all()
    assert (d_os.cpu().numpy()[:, :M] == s8[:, :M]).all()
    # same kernel without the fp32 side output
    d_o8b = torch.zeros_like(d_o8)
    _ok(xt.lib.eva_k_flash(xt.ptr(_d(q, dev)), xt.ptr(_d(k, dev)), xt.ptr(_d(vt, dev)), xt.ptr(d_o8b), xt.ptr(d_os), lds,
                           nb, None, _st()), "eva_k_flash")
    assert torch.equal(d_o8b, d_o8)


def test_flash_row_sums_and_permutation(dev, xt, orc):
    """Invariants: V = ones gives o = 1 exactly for every query; permuting keys (with V) leaves o unchanged."""
    nb = 1
    q, k, vt = _attn_inputs(nb, 41)
    vt1 = torch.zeros_like(vt)
    vt1[:, :, :, :T] = 1.0
    d_o8 = torch.zeros((T, D), dtype=torch.uint8, device=dev)
    d_os = torch.zeros((8, T), dtype=torch.float32, device=dev)
    d_o32 = torch.zeros((T, D), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_flash(xt.ptr(_d(q, dev)), xt.ptr(_d(k, dev)), xt.ptr(_d(vt1, dev)), xt.ptr(d_o8), xt.ptr(d_os), T,
                           nb, xt.ptr(d_o32), _st()), "flash ones")
    o = d_o32.cpu().numpy()
    # l sums the same bf16 weights the PV product uses: rows of a V of ones come out 1 up to fp32 summation order
    assert np.abs(o - 1.0).max() <= 1e-5
    perm = np.random.default_rng(5).permutation(T)
    kp, vp = k.clone(), vt.clone()
    kp[:, :, :T] = k[:, :, perm]
    vp[:, :, :, :T] = vt[:, :, :, perm]
    d_o32b = torch.zeros_like(d_o32)
    _ok(xt.lib.eva_k_flash(xt.ptr(_d(q, dev)), xt.ptr(_d(kp, dev)), xt.ptr(_d(vp, dev)), xt.ptr(d_o8), xt.ptr(d_os), T,
                           nb, xt.ptr(d_o32b), _st()), "flash perm")
    _ok(xt.lib.eva_k_flash(xt.ptr(_d(q, dev)), xt.ptr(_d(k, dev)), xt.ptr(_d(vt, dev)), xt.ptr(d_o8), xt.ptr(d_os), T,
                           nb, xt.ptr(d_o32), _st()), "flash")
    a, b = d_o32.cpu().numpy(), d_o32b.cpu().numpy()
    assert np.abs(a - b).max() <= 4e-3 * np.abs(a).max()


@pytest.mark.parametrize("nseq,T,qstep", [(18, 576, 1), (1, 5184, 41), (3, 200, 1), (2, 129, 1), (2, 385, 1)])
def test_flash_seq_parity(dev, xt, orc, nseq, T, qstep):
    """Sequences of T tokens: the PixAI windows (9 per image x 2 images, L = 576) and its global attention (L = 5184,
    every 41st query checked against fp64), a length that is not a multiple of 64 (masked keys), and lengths 128 n + 1
    whose last query block holds one query, with key tiles that do not split evenly over four waves (2 and 6 tiles)."""
    TPad = (T + 63) // 64 * 64
    _say(f"k_flash_seq nseq={nseq} T={T}")
    r = np.random.default_rng(T)
    qf = np.zeros((nseq, 16, TPad, 64), np.float32)
    kf = np.zeros_like(qf)
    vf = np.zeros((nseq, 16, 64, TPad), np.float32)
    qf[:, :, :T] = r.standard_normal((nseq, 16, T, 64)) * 0.6
    kf[:, :, :T] = r.standard_normal((nseq, 16, T, 64)) * 0.6
    vf[..., :T] = r.standard_normal((nseq, 16, 64, T))
    bf = lambda a: torch.from_numpy(a).to(torch.bfloat16)
    q, k, vt = bf(qf), bf(kf), bf(vf)
    M = nseq * T
    lds = M + 5
    d_o8 = torch.zeros((M, D), dtype=torch.uint8, device=dev)
    d_os = torch.zeros((8, lds), dtype=torch.float32, device=dev)
    d_o32 = torch.zeros((M, D), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_flash_seq(xt.ptr(_d(q, dev)), xt.ptr(_d(k, dev)), xt.ptr(_d(vt, dev)), xt.ptr(d_o8), xt.ptr(d_os),
                               lds, nseq, T, TPad, xt.ptr(d_o32), _st()), "eva_k_flash_seq")
    ref = orc.attention_seq(q.view(torch.int16).numpy(), k.view(torch.int16).numpy(), vt.view(torch.int16).numpy(),
                            nseq, T, TPad, qstep)
    rows = np.arange(M)[(np.arange(M) % T) % qstep == 0]
    o = d_o32.cpu().numpy().astype(np.float64)[rows]
    ref = ref[rows]
    rel = np.abs(o - ref).max() / np.abs(ref).max()
    _say(f"  o32 max err / max|ref| {rel:.3g}")
    assert rel <= 4e-3
    assert np.linalg.norm(o - ref) <= 2e-3 * np.linalg.norm(ref)
    q8, s8 = orc.quant_act(d_o32.cpu().numpy(), lds=lds)     # output packing of the kernel's own fp32 output
    assert (d_o8.cpu().numpy() == q8).all()
    assert (d_os.cpu().numpy()[:, :M] == s8[:, :M]).all()


def test_oproj_residual(dev, xt, orc):
    M = 2 * T
    _say("k_oproj")
    _, qa, sa = _packed_act(orc, M, D, 51)
    _, qw, sw = _packed_w(orc, D, D, 52)
    x = (np.random.default_rng(53).standard_normal((M, D)) * 2).astype(np.float16)
    d_x = _d(x, dev)
    _ok(xt.lib.eva_k_oproj(xt.ptr(_d(qa, dev)), xt.ptr(_d(sa, dev)), M, xt.ptr(_d(qw, dev)), xt.ptr(_d(sw, dev)),
                           xt.ptr(d_x), M, _st()), "eva_k_oproj")
    acc = _acc_ref(orc, qa, sa, qw, sw, D)
    ref = orc.oproj_epi(acc, x.view(np.uint16))
    _check_close("x", _f16_f32(d_x.cpu().numpy().view(np.uint16)), _f16_f32(ref), np.abs(acc).max(), 2.0 ** -10)


@pytest.mark.parametrize("with_rs", [False, True])
def test_fc1_swiglu_pack(dev, xt, orc, with_rs):
    """k_fc1 against the oracle's epilogue on the fp64 product; with_rs: eva_k_fc1_rs, the v3 blob's per-unit
    multiplier rs (eva_kernels.cu:258-264): the packed operand is h rs, the row sums stay over h."""
    M = 2 * T
    _say(f"k_fc1 (rs: {with_rs})")
    _, qa, sa = _packed_act(orc, M, D, 61)
    r = np.random.default_rng(62)
    w = (r.standard_normal((2 * HIDP, D)) * 0.02).astype(np.float32)
    units = np.arange(HIDP)
    pad = units[units >= 2730]                                # pad units have zero g and x rows, as in the blob
    w[32 * (pad // 16) + pad % 16] = 0
    w[32 * (pad // 16) + 16 + pad % 16] = 0
    qw, sw = orc.quant_w(w)
    lds = M + 3
    sa_l = np.zeros((8, lds), np.float32)
    sa_l[:, :M] = sa
    d_m8 = torch.zeros((M, HIDP), dtype=torch.uint8, device=dev)
    d_ms = torch.zeros((22, lds), dtype=torch.float32, device=dev)
    d_st = torch.zeros((22, lds, 2), dtype=torch.float32, device=dev)
    rs = np.exp(r.uniform(-2, 2, HIDP)).astype(np.float32)   # multipliers over e^-2 .. e^2, as 1 / (adq s~) spread
    if with_rs:
        _ok(xt.lib.eva_k_fc1_rs(xt.ptr(_d(qa, dev)), xt.ptr(_d(sa_l, dev)), lds, xt.ptr(_d(qw, dev)),
                                xt.ptr(_d(sw, dev)), xt.ptr(d_m8), xt.ptr(d_ms), xt.ptr(d_st), xt.ptr(_d(rs, dev)), M,
                                _st()), "eva_k_fc1_rs")
    else:
        _ok(xt.lib.eva_k_fc1(xt.ptr(_d(qa, dev)), xt.ptr(_d(sa_l, dev)), lds, xt.ptr(_d(qw, dev)), xt.ptr(_d(sw, dev)),
                             xt.ptr(d_m8), xt.ptr(d_ms), xt.ptr(d_st), M, _st()), "eva_k_fc1")
    h, stat = orc.fc1_epi(_acc_ref(orc, qa, sa, qw, sw, 2 * HIDP))
    hq = (h * rs[None, :]).astype(np.float32) if with_rs else h   # one fp32 rounding, as the kernel's multiply
    q, s = orc.quant_act(hq)
    ms = d_ms.cpu().numpy()[:, :M]
    # each block scale is one GEMM-fed maximum over 128 units; with multipliers spread over e^+-2 that maximum is a
    # single unit's h rs, which carries the matrix core's summation error relative to its own terms (~1e-4)
    assert np.abs(ms / s - 1).max() < (5e-4 if with_rs else 1e-4)
    m8 = d_m8.cpu().numpy()
    same = m8 == q
    _say(f"  E4M3 codes differing: {np.mean(~same):.2e}")
    assert np.mean(~same) < 2e-3
    dq = orc.e4m3_decode(m8) * np.repeat(ms.T, 128, 1)
    assert np.abs(dq - hq).max() <= 2.0 ** -3 * np.abs(hq).max() + 1e-6
    st = d_st.cpu().numpy()[:, :M]
    assert np.abs(st[..., 0] - stat[..., 0]).max() <= 1e-4 * np.abs(stat[..., 1]).max() ** 0.5 + 1e-5
    assert np.abs(st[..., 1] / np.maximum(stat[..., 1], 1e-12) - 1).max() < 1e-4
    assert (m8[:, 2730:] == 0).all()                          # pad units of h are exactly zero


def test_fc2_folded_ln(dev, xt, orc):
    M = 2 * T
    _say("k_fc2")
    r = np.random.default_rng(71)
    h = (r.standard_normal((M, HIDP)) * 0.3).astype(np.float32)
    h[:, 2730:] = 0
    qa, sa = orc.quant_act(h)
    stat = np.stack([h.reshape(M, 22, 128).sum(2).T, (h.astype(np.float64) ** 2).reshape(M, 22, 128).sum(2).T], -1)
    stat = stat.astype(np.float32)
    _, qw, sw = _packed_w(orc, D, HIDP, 72)
    c = (r.standard_normal(D) * 0.5).astype(np.float32)
    d = (r.standard_normal(D) * 0.1).astype(np.float32)
    x = (r.standard_normal((M, D)) * 2).astype(np.float16)
    d_x = _d(x, dev)
    _ok(xt.lib.eva_k_fc2(xt.ptr(_d(qa, dev)), xt.ptr(_d(sa, dev)), M, xt.ptr(_d(qw, dev)), xt.ptr(_d(sw, dev)),
                         xt.ptr(_d(stat, dev)), xt.ptr(_d(c, dev)), xt.ptr(_d(d, dev)), xt.ptr(d_x), M, _st()),
        "eva_k_fc2")
    acc = _acc_ref(orc, qa, sa, qw, sw, D)
    ref = orc.fc2_epi(acc, stat, c, d, x.view(np.uint16))
    S, Q = stat[..., 0].sum(0), stat[..., 1].sum(0)
    mean = S / 2730.0
    rstd = 1.0 / np.sqrt(np.maximum(Q / 2730.0 - mean ** 2, 0) + 1e-6)
    scale = np.abs(rstd[:, None] * acc).max()
    _check_close("x", _f16_f32(d_x.cpu().numpy().view(np.uint16)), _f16_f32(ref), scale, 2.0 ** -10)


@pytest.mark.parametrize("nb,nt", [(32, 10861), (64, 13461), (1, 300), (128, 1000), (37, 64)])
def test_head_sigmoid(dev, xt, orc, nb, nt):
    _say(f"k_head nb={nb} nt={nt}")
    _, qa, sa = _packed_act(orc, nb, D, 81)
    r = np.random.default_rng(82)
    w16 = (r.standard_normal((nt, D)) * 0.05).astype(np.float16)
    w16[::97] *= 30                                           # rows of very different size: each has its own scales
    ldw = nt + 19
    d_w16 = _d(w16, dev)
    d_qw = torch.zeros((nt, D), dtype=torch.uint8, device=dev)
    d_sw = torch.full((8, ldw), np.nan, dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_quant_act(xt.ptr(d_w16), 2, D, nt, D, xt.ptr(d_qw), D, xt.ptr(d_sw), ldw, _st()), "pack head")
    qw, sw = orc.head_pack(w16)
    assert (d_qw.cpu().numpy() == qw).all() and (d_sw.cpu().numpy()[:, :nt] == sw).all()   # fp16 packing bit-exact
    hb = (np.random.default_rng(83).standard_normal(nt) * 0.1).astype(np.float32)
    d_out = torch.zeros((nb, nt), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_head(xt.ptr(_d(qa, dev)), xt.ptr(_d(sa, dev)), nb, xt.ptr(d_qw), xt.ptr(d_sw), ldw,
                          xt.ptr(_d(hb, dev)), xt.ptr(d_out), nb, nt, _st()), "eva_k_head")
    logit = orc.gemm_rr_f64_rows(qa, sa, qw, sw, nt, np.arange(nb))
    ref = 1.0 / (1.0 + np.exp(-(logit + hb)))
    err = np.abs(d_out.cpu().numpy() - ref)
    # the matrix core's fp32 sums sit within ~1e-5 of the terms of fp64; sigmoid' <= 1/4. The x30 rows have terms
    # ~1500, the others ~50 (sigmoid within 1e-4 there, as the forward's head)
    lut = orc.E4M3_LUT.astype(np.float64)
    terms = (np.abs(lut[qa]) * np.repeat(sa.T, 128, 1)) @ (np.abs(lut[qw]) * np.repeat(sw.T, 128, 1)).T
    big = np.zeros(nt, bool)
    big[::97] = True
    _say(f"  sigmoid max |err| {err[:, ~big].max():.2e} (ordinary rows), {err[:, big].max():.2e} (x30 rows)")
    assert err[:, ~big].max() < 1e-4
    assert (err <= 0.25 * 2e-5 * terms + 1e-6).all()


def test_patch_embed(dev, xt, orc):
    nb = 2
    _say("k_pe")
    from xtagger_amd import blob
    r = np.random.default_rng(91)
    inp = blob.synth_inputs(nb, seed=92)
    pe = np.zeros((D, 592), np.float16)
    pe[:, :588] = (r.standard_normal((D, 588)) * 0.02).astype(np.float16)
    pos = (r.standard_normal((T, D)) * 0.02).astype(np.float32)
    d_x = torch.zeros((nb * T, D), dtype=torch.int16, device=dev)
    _ok(xt.lib.eva_k_pe(xt.ptr(_d(inp, dev)), xt.ptr(_d(pe, dev)), xt.ptr(_d(pos, dev)), xt.ptr(d_x), nb, _st()),
        "eva_k_pe")
    ref = orc.embed(inp.view(np.uint16), pe.view(np.uint16), pos, nb)
    got = d_x.cpu().numpy().view(np.uint16)
    _check_close("x", _f16_f32(got), _f16_f32(ref), np.abs(_f16_f32(ref)).max(), 2.0 ** -10)
    assert (got[::T] == ref[::T]).all()                      # cls rows are pos[0] exactly


@pytest.mark.parametrize("tail", [1, 8, 17, 32, 33, 64])
def test_partial_row_tile_bit_identical(dev, xt, orc, tail):
    """A last row tile with `tail` rows below M (its waves run only the 16-row tiles that hold such rows) gives its
    rows bit for bit what a whole tile gives them: oproj and fc1 over M = 2048 + tail rows against the same rows of an
    M = 2304 run (nine whole tiles)."""
    MF, MT = 2304, 2048 + tail
    _say(f"partial row tile of {tail} rows")
    _, qa, sa = _packed_act(orc, MF, D, 71)
    _, qw, sw = _packed_w(orc, D, D, 72)
    x = (np.random.default_rng(73).standard_normal((MF, D)) * 2).astype(np.float16)
    d_a, d_sa, d_w, d_sw = _d(qa, dev), _d(sa, dev), _d(qw, dev), _d(sw, dev)
    outs = []
    for rows in (MF, MT):
        d_x = _d(x, dev)
        _ok(xt.lib.eva_k_oproj(xt.ptr(d_a), xt.ptr(d_sa), MF, xt.ptr(d_w), xt.ptr(d_sw), xt.ptr(d_x), rows, _st()),
            "eva_k_oproj")
        outs.append(d_x.cpu().numpy())
    assert np.array_equal(outs[0][:MT], outs[1][:MT])
    assert np.array_equal(outs[1][MT:], x[MT:])               # rows past M untouched
    r = np.random.default_rng(74)
    w12 = (r.standard_normal((2 * HIDP, D)) * 0.02).astype(np.float32)
    units = np.arange(HIDP)
    pad = units[units >= 2730]
    w12[32 * (pad // 16) + pad % 16] = 0
    w12[32 * (pad // 16) + 16 + pad % 16] = 0
    qw1, sw1 = orc.quant_w(w12)
    d_w1, d_sw1 = _d(qw1, dev), _d(sw1, dev)
    res = []
    for rows in (MF, MT):
        m8 = torch.zeros((MF, HIDP), dtype=torch.uint8, device=dev)
        ms = torch.zeros((22, MF), dtype=torch.float32, device=dev)
        st = torch.zeros((22, MF, 2), dtype=torch.float32, device=dev)
        _ok(xt.lib.eva_k_fc1(xt.ptr(d_a), xt.ptr(d_sa), MF, xt.ptr(d_w1), xt.ptr(d_sw1), xt.ptr(m8), xt.ptr(ms),
                             xt.ptr(st), rows, _st()), "eva_k_fc1")
        res.append((m8.cpu().numpy(), ms.cpu().numpy(), st.cpu().numpy()))
    (a8, as_, ast), (b8, bs, bst) = res
    assert np.array_equal(a8[:MT], b8[:MT]) and np.array_equal(as_[:, :MT], bs[:, :MT])
    assert np.array_equal(ast[:, :MT], bst[:, :MT])


@pytest.mark.parametrize("tail", [8, 32])
def test_partial_row_tile_bit_identical_fc2(dev, xt, orc, tail):
    """fc2 (its row statistics and column terms staged while the first operands load) over M = 2048 + tail rows
    against the same rows of a nine-tile run."""
    MF, MT = 2304, 2048 + tail
    r = np.random.default_rng(81)
    h = (r.standard_normal((MF, HIDP)) * 0.3).astype(np.float32)
    h[:, 2730:] = 0
    qa, sa = orc.quant_act(h)
    stat = np.stack([h.reshape(MF, 22, 128).sum(2).T, (h.astype(np.float64) ** 2).reshape(MF, 22, 128).sum(2).T], -1)
    stat = stat.astype(np.float32)
    _, qw, sw = _packed_w(orc, D, HIDP, 82)
    c = (r.standard_normal(D) * 0.5).astype(np.float32)
    d = (r.standard_normal(D) * 0.1).astype(np.float32)
    x = (r.standard_normal((MF, D)) * 2).astype(np.float16)
    args = [_d(t, dev) for t in (qa, sa, qw, sw, stat, c, d)]
    outs = []
    for rows in (MF, MT):
        d_x = _d(x, dev)
        _ok(xt.lib.eva_k_fc2(*(xt.ptr(t) for t in args[:2]), MF, *(xt.ptr(t) for t in args[2:]), xt.ptr(d_x), rows,
                             _st()), "eva_k_fc2")
        outs.append(d_x.cpu().numpy())
    bad = np.flatnonzero((outs[0][:MT] != outs[1][:MT]).any(1))
    assert bad.size == 0, f"rows differing: {bad.tolist()[:40]}"


@pytest.mark.parametrize("nb", [2, 17, 32])
def test_partial_row_tile_bit_identical_qkv(dev, xt, orc, nb):
    """qkv over nb images (1025 nb rows: a last row tile of nb rows) against the same images inside an nb + 1 run,
    where their rows sit in whole tiles."""
    _say(f"k_qkv partial row tile, nb={nb}")
    r = np.random.default_rng(91)
    w16 = (r.standard_normal((3 * D, D)) * 0.02).astype(np.float16)
    ang = r.random((1024, 32)) * 6.28
    cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    d_wq = torch.zeros((3 * D, D), dtype=torch.uint8, device=dev)
    d_ws = torch.zeros((24, 8), dtype=torch.float32, device=dev)
    scratch = torch.empty((3 * D, D), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_prep_w(xt.ptr(_d(w16, dev)), D, 3 * D, D, 3 * D, D, 1, None, xt.ptr(scratch), xt.ptr(d_wq),
                            xt.ptr(d_ws), _st()), "prep")
    MF = (nb + 1) * T
    _, qa, sa = _packed_act(orc, MF, D, 92)
    d_a, d_sa, d_cs = _d(qa, dev), _d(sa, dev), _d(cs, dev)
    outs = []
    for n in (nb + 1, nb):
        kw = [torch.zeros((n, 16, TP, 64), dtype=torch.int16, device=dev) for _ in range(2)]
        d_vt = torch.zeros((n, 16, 64, TP), dtype=torch.int16, device=dev)
        _ok(xt.lib.eva_k_qkv(xt.ptr(d_a), xt.ptr(d_sa), MF, xt.ptr(d_wq), xt.ptr(d_ws), xt.ptr(d_cs), xt.ptr(kw[0]),
                             xt.ptr(kw[1]), xt.ptr(d_vt), n * T, _st()), "eva_k_qkv")
        outs.append([t.cpu().numpy()[:nb] for t in (kw[0], kw[1], d_vt)])
    for name, a, b in zip(("q", "k", "vt"), *outs):
        diff = a != b
        toks = np.flatnonzero(diff.any(axis=(0, 1, 3) if name != "vt" else (0, 1, 2)))
        imgs = np.flatnonzero(diff.reshape(nb, -1).any(1))
        assert not diff.any(), f"{name}: images {imgs.tolist()}, tokens {toks.tolist()[:40]}"
