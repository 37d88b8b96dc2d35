"""Pins the oracle's layer functions (oracle/xt_oracle.c) against independent float64 formulations before they are
trusted as the checker of the attention, SwiGLU, folded-MLP, embedding, pooling, final-LayerNorm and forward kernels.

Each test recomputes the function from its definition with numpy / scipy in float64 and compares; the inputs are
chosen so that the plausible mistakes fail: padding keys hold large values (a read past T changes every output),
the cls row holds a large value (pooling it shifts the mean), the SwiGLU hidden mean is far from zero (a 2816 instead
of 2730 denominator, or a lost mean term, moves every output), g and x differ in scale (swapping them changes h),
and the forward is composed from numpy primitives, not from the oracle's C functions.

Reference semantics: attention flash8 (src/engine/kern_common.cuh:403-543: softmax in the exp2 domain over the T
real keys); SwiGLU and its row partials k_fc1 (src/engine/eva_kernels.cu:211-279, g / x interleave
src/tools/export_eva.py:60-62); folded MLP LayerNorm k_fc2 (eva_kernels.cu:286-334, export_eva.py:101-104,
117-119); embedding k_pe + k_embed (eva_kernels.cu:21-33, 126-130); pool and final LN k_pool / k_lnh
(eva_kernels.cu:402-431, kern_common.cuh:188-192); the forward order eva_forward (src/engine/eva.h:227-310).
"""
import numpy as np
import pytest
import torch
from scipy.special import softmax

LN2 = float(np.log(2.0))


def bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def bf16_val(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def f16_val(b):
    return np.asarray(b, np.uint16).view(np.float16).astype(np.float64)


def f16_ulp(v):
    """One fp16 unit in the last place at |v| (normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -14)))
    return 2.0 ** (e - 10)


# ---------------------------------------------------------------- attention
def _attn_inputs(nseq, T, TP, seed):
    r = np.random.default_rng(seed)
    q = r.standard_normal((nseq, 16, TP, 64)) * 0.7
    k = r.standard_normal((nseq, 16, TP, 64)) * 0.7
    vt = r.standard_normal((nseq, 16, 64, TP))
    # padding rows past T: huge scores and values, so any use of them changes every output row
    q[:, :, T:], k[:, :, T:], vt[..., T:] = 30.0, 30.0, 1000.0
    return bf16_bits(q), bf16_bits(k), bf16_bits(vt)


def _attn_ref(q, k, vt, T):
    Q, K = bf16_val(q)[:, :, :T], bf16_val(k)[:, :, :T]
    V = np.swapaxes(bf16_val(vt)[..., :T], -1, -2)
    s = Q @ np.swapaxes(K, -1, -2)                       # log2-domain scores (q carries log2(e)/8)
    p = softmax(s * LN2, axis=-1)                         # 2^s normalised == softmax of s ln 2
    o = p @ V                                             # [nseq][16][T][64]
    return np.transpose(o, (0, 2, 1, 3)).reshape(-1, 1024)


@pytest.mark.parametrize("nseq,T,TP,qstep", [(2, 200, 256, 1), (1, 576, 576, 7)])
def test_attention_seq_vs_scipy_softmax(orc, nseq, T, TP, qstep):
    q, k, vt = _attn_inputs(nseq, T, TP, T)
    o = orc.attention_seq(q, k, vt, nseq, T, TP, qstep=qstep)
    ref = _attn_ref(q, k, vt, T)
    rows = np.arange(nseq * T)
    rows = rows[(rows % T) % qstep == 0]
    err = np.abs(o[rows] - ref[rows]).max()
    assert err <= 1e-10, err
    assert np.isnan(o[(np.arange(nseq * T) % T) % qstep != 0]).all()


def test_attention_t1025_vs_scipy_softmax(orc):
    # the wd shape: T = 1025 real keys in TP = 1088 rows; the attention() wrapper's constants
    q, k, vt = _attn_inputs(1, 1025, 1088, 11)
    o = orc.attention(q, k, vt, 1)
    ref = _attn_ref(q, k, vt, 1025)
    assert np.abs(o - ref).max() <= 1e-10


def test_attention_rows_sum_to_one_and_key_permutation(orc):
    T, TP = 300, 320
    q, k, vt = _attn_inputs(1, T, TP, 5)
    ones = vt.copy()
    ones[..., :T] = bf16_bits(np.ones(1))[0]
    o = orc.attention_seq(q, k, ones, 1, T, TP)
    assert np.abs(o - 1.0).max() <= 1e-12
    perm = np.random.default_rng(0).permutation(T)
    k2, v2 = k.copy(), vt.copy()
    k2[:, :, :T] = k[:, :, perm]
    v2[..., :T] = vt[..., perm]
    o1 = orc.attention_seq(q, k, vt, 1, T, TP)
    o2 = orc.attention_seq(q, k2, v2, 1, T, TP)
    assert np.abs(o1 - o2).max() <= 1e-12


# ---------------------------------------------------------------- SwiGLU epilogue
def _fc1_acc(M, seed):
    """fc1 accumulators [M][5632]: 16-unit chunks [g c | x c]; g wide (it reaches the exp over- and underflow
    ranges), x narrower with an offset; the pad units 2730.. are zero (their weight rows are)."""
    r = np.random.default_rng(seed)
    g = (r.standard_normal((M, 2816)) * 3.0).astype(np.float32)
    x = (r.standard_normal((M, 2816)) * 0.5 + 0.2).astype(np.float32)
    g[:, :4] = np.array([-120.0, -89.0, 89.0, 120.0], np.float32)
    g[:, 2730:] = 0
    x[:, 2730:] = 0
    return np.stack([g.reshape(M, 176, 16), x.reshape(M, 176, 16)], 2).reshape(M, 5632)


def test_fc1_epi_vs_float64(orc):
    M = 37
    acc = _fc1_acc(M, 1)
    h, stat = orc.fc1_epi(acc)
    a = acc.astype(np.float64).reshape(M, 176, 2, 16)
    g, x = a[:, :, 0].reshape(M, 2816), a[:, :, 1].reshape(M, 2816)
    with np.errstate(over="ignore"):
        ref = x * g / (1.0 + np.exp(-g))                    # silu(g) x, exact sigmoid
    scale = np.abs(ref).max()
    assert np.abs(h - ref).max() <= 2e-7 * scale
    assert (h[:, 2730:] == 0).all()
    # the swapped form silu(x) g is far from it: the interleave is pinned
    swapped = g * x / (1.0 + np.exp(-x))
    assert np.abs(swapped - ref).max() > 0.1 * scale
    hb = h.astype(np.float64).reshape(M, 22, 128)
    S, Q = hb.sum(-1).T, (hb * hb).sum(-1).T                 # [22][M], sums of the unpacked fp32 h
    assert np.abs(stat[..., 0] - S).max() <= 1e-5 * np.abs(hb).sum(-1).max()
    assert np.abs(stat[..., 1] - Q).max() <= 1e-5 * (hb * hb).sum(-1).max()


# ---------------------------------------------------------------- folded MLP LayerNorm + fc2
def test_fold_and_fc2_epi_vs_unfolded_layernorm(orc):
    r = np.random.default_rng(2)
    M, HID = 29, 2730
    w2 = np.zeros((1024, 2736), np.float32)
    w2[:, :HID] = r.standard_normal((1024, HID)) * 0.02
    w2_16 = w2.astype(np.float16)
    gamma = np.zeros(2736, np.float32)
    beta = np.zeros(2736, np.float32)
    gamma[:HID] = 1 + r.standard_normal(HID) * 0.1
    beta[:HID] = r.standard_normal(HID) * 0.05
    wt, d = orc.fold_w2(w2_16.view(np.uint16), gamma, beta)
    w2f = w2_16.astype(np.float64)
    # W~ = W2 diag(gamma): one fp32 rounding of each product; pads zero; d = W2 beta
    assert (wt[:, :HID] == (w2_16[:, :HID].astype(np.float32) * gamma[:HID])).all()
    assert (wt[:, HID:] == 0).all()
    dref = w2f[:, :HID] @ beta[:HID].astype(np.float64)
    assert np.abs(d - dref).max() <= 1e-5 * np.abs(w2f[:, :HID] * beta[:HID]).sum(1).max()
    # c = W~ 1 from the packed (dequantized) W~
    qw, sw = orc.quant_w(wt)
    lut = orc.E4M3_LUT.astype(np.float64)
    wdq = lut[qw] * np.repeat(np.repeat(sw.astype(np.float64), 128, 0), 128, 1)[:1024, :2816]
    c = orc.fold_c(qw, sw)
    assert np.abs(c - wdq.sum(1)).max() <= 1e-5 * np.abs(wdq).sum(1).max()
    # fc2 epilogue on acc = h . W~dq^T equals the unfolded LN(h) over the 2730 real units through the same W~dq
    h = np.zeros((M, 2816), np.float32)
    h[:, :HID] = r.standard_normal((M, HID)) * 0.8 + 0.6    # a mean far from zero
    hb = h.astype(np.float64).reshape(M, 22, 128)
    stat = np.stack([hb.sum(-1).T, (hb * hb).sum(-1).T], -1).astype(np.float32)
    acc = (h.astype(np.float64) @ wdq.T).astype(np.float32)
    x16 = (r.standard_normal((M, 1024)) * 2).astype(np.float16)
    got = f16_val(orc.fc2_epi(acc, stat, c, d, x16.view(np.uint16)))
    hh = h[:, :HID].astype(np.float64)
    mu, var = hh.mean(1, keepdims=True), hh.var(1, keepdims=True)
    y = (hh - mu) / np.sqrt(var + 1e-6)
    ref = x16.astype(np.float64) + y @ wdq[:, :HID].T + dref
    err = np.abs(got - ref)
    assert (err <= f16_ulp(ref) + 2e-4 * np.abs(y @ wdq[:, :HID].T).max()).all(), err.max()
    # a 2816-unit mean / variance would be visibly off
    mu2 = h.astype(np.float64).mean(1, keepdims=True)
    assert np.abs((mu2 - mu) * wdq.sum(1)).max() > 1e-2


# ---------------------------------------------------------------- embedding, pooling, final LayerNorm
def test_embed_vs_float64(orc):
    r = np.random.default_rng(3)
    nb = 2
    inp = np.zeros((nb, 1024, 592), np.float16)
    inp[..., :588] = r.uniform(-1, 1, (nb, 1024, 588))
    pe = np.zeros((1024, 592), np.float16)
    pe[:, :588] = r.standard_normal((1024, 588)) * 0.05
    pos = (r.standard_normal((1025, 1024)) * 0.1).astype(np.float32)
    x = f16_val(orc.embed(inp.view(np.uint16), pe.view(np.uint16), pos, nb)).reshape(nb, 1025, 1024)
    dot = inp.astype(np.float64) @ pe.astype(np.float64).T
    ref = dot + pos[1:].astype(np.float64)
    err = np.abs(x[:, 1:] - ref)
    # the dot is rounded to fp32, dot + pos to fp32, then to fp16: half an fp16 ulp of the result plus half an fp32
    # ulp of the dot and of the sum (the dot's rounding survives a cancelling pos)
    assert (err <= f16_ulp(ref) * 0.5 + 2.0 ** -24 * (np.abs(dot) + np.abs(ref)) * 1.01 + 1e-12).all(), err.max()
    assert (err <= f16_ulp(ref)).all()
    assert (x[:, 0] == pos[0].astype(np.float16).astype(np.float64)).all()


def test_pool_vs_float64(orc):
    r = np.random.default_rng(4)
    nb = 3
    x = (r.standard_normal((nb, 1025, 1024)) * 2 + 0.5).astype(np.float16)
    x[:, 0] = 1000.0                                       # cls: must not enter the mean
    p = orc.pool(x.reshape(-1, 1024).view(np.uint16), nb)
    ref = x[:, 1:].astype(np.float64).mean(1)
    assert np.abs(p - ref).max() <= 1e-5


def test_lnh_vs_float64(orc):
    r = np.random.default_rng(5)
    nb = 5
    p = (r.standard_normal((nb, 1024)) * 3 + 0.7).astype(np.float32)
    g = (1 + r.standard_normal(1024) * 0.1).astype(np.float32)
    b = (r.standard_normal(1024) * 0.05).astype(np.float32)
    pn, q, s = orc.lnh(p, g, b)
    pf = p.astype(np.float64)
    ref = (pf - pf.mean(1, keepdims=True)) / np.sqrt(pf.var(1, keepdims=True) + 1e-6) * g + b
    err = np.abs(f16_val(pn) - ref)
    assert (err <= f16_ulp(ref) * 0.5 + 1e-6).all(), err.max()
    # the head input is the 1x128 packing of the fp16 values
    q2, s2 = orc.quant_act(f16_val(pn).astype(np.float32))
    assert (q == q2).all() and (s == s2).all()


# ---------------------------------------------------------------- the head GEMM with per-row weight scales
def test_head_gemm_rr_vs_numpy(orc):
    r = np.random.default_rng(6)
    nb, nt = 7, 333
    x = (r.standard_normal((nb, 1024)) * 2).astype(np.float32)
    w = (r.standard_normal((nt, 1024)) * 0.05).astype(np.float16)
    w[::13] *= 50                                          # rows of very different size
    qa, sa = orc.quant_act(x)
    qw, sw = orc.head_pack(w)
    lut = orc.E4M3_LUT.astype(np.float64)
    A = lut[qa] * np.repeat(sa.T.astype(np.float64), 128, 1)
    W = lut[qw] * np.repeat(sw.T.astype(np.float64), 128, 1)
    ref = A @ W.T
    got = orc.gemm_rr_f64_rows(qa, sa, qw, sw, nt, np.arange(nb))
    assert np.abs(got - ref).max() <= 1e-12 * (np.abs(A) @ np.abs(W).T).max()
    # each row's packing depends on that row alone: scaling one row leaves every other row's codes and scales
    w2 = w.copy()
    w2[5] *= 7
    qw2, sw2 = orc.head_pack(w2)
    keep = np.arange(nt) != 5
    assert (qw2[keep] == qw[keep]).all() and (sw2[:, keep] == sw[:, keep]).all()
    # and the packing is the 1x128 packing of the fp16 values, within E4M3 resolution of them
    err = np.abs(W - w.astype(np.float64))
    assert (err <= 2.0 ** -4 * np.repeat(sw.T.astype(np.float64), 128, 1) * 448).all()


# ---------------------------------------------------------------- the forward, composed in float64
def _f64_forward(orc, m, inp16, nl):
    """eva_forward's order (eva.h:227-310) from numpy float64 primitives. The storage formats the design fixes are
    kept: fp16 residual stream, E4M3 1x128 / 128x128 packing at every GEMM input (the oracle's pinned packers),
    bf16 q / k / v, fp32 SwiGLU h with its LayerNorm folded as k_fc2 computes it."""
    lut = orc.E4M3_LUT.astype(np.float64)
    nb = inp16.shape[0]
    T, M = 1025, nb * 1025

    def act(x):                                          # E4M3 1x128 round trip of a float array [M][K]
        q, s = orc.quant_act(np.asarray(x, np.float32))
        return lut[q] * np.repeat(s.T.astype(np.float64), 128, 1)[: q.shape[0]]

    def wt(w):                                           # E4M3 128x128 round trip of weights [N][K]
        q, s = orc.quant_w(np.asarray(w, np.float32))
        return lut[q] * np.repeat(np.repeat(s.astype(np.float64), 128, 0), 128, 1)[: q.shape[0], : q.shape[1]]

    def ln(x, g, b, eps=1e-6):
        mu, var = x.mean(-1, keepdims=True), x.var(-1, keepdims=True)
        return (x - mu) / np.sqrt(var + eps) * g + b

    f16 = lambda v: np.asarray(v).astype(np.float16).astype(np.float64)
    bf16 = lambda v: bf16_val(bf16_bits(v))
    x = np.empty((nb, T, 1024))
    pe = m["pe"].astype(np.float64)
    for b in range(nb):
        x[b, 0] = m["pos"][0]
        x[b, 1:] = inp16[b].astype(np.float64) @ pe.T + m["pos"][1:]
    x = f16(x).reshape(M, 1024)
    cs = m["rope"].astype(np.float64)
    for L in m["layers"][:nl]:
        a = act(ln(x, L["ln1w"], L["ln1b"]))
        y = (a @ wt(L["wqkv"].astype(np.float32)).T).reshape(nb, T, 3, 16, 32, 2)
        for part in (0, 1):                               # RoPE on pairs (2i, 2i + 1) of q and k, patch tokens only
            f0, f1 = y[:, 1:, part, :, :, 0].copy(), y[:, 1:, part, :, :, 1].copy()
            c, s = cs[None, :, None, :, 0], cs[None, :, None, :, 1]
            y[:, 1:, part, :, :, 0] = f0 * c - f1 * s
            y[:, 1:, part, :, :, 1] = f1 * c + f0 * s
        y = bf16(y).reshape(nb, T, 3, 16, 64)
        qh, kh, vh = (np.transpose(y[:, :, i], (0, 2, 1, 3)) for i in range(3))
        p = softmax(qh @ np.swapaxes(kh, -1, -2) * LN2, axis=-1)
        o = np.transpose(p @ vh, (0, 2, 1, 3)).reshape(M, 1024)
        x = f16(x + act(o) @ wt(L["wo"].astype(np.float32)).T)
        a = act(ln(x, L["ln2w"], L["ln2b"]))
        w12 = np.zeros((5632, 1024), np.float32)
        w12[:5472] = L["w12"]
        acc = (a @ wt(w12).T).reshape(M, 176, 2, 16)
        g, xv = acc[:, :, 0].reshape(M, 2816), acc[:, :, 1].reshape(M, 2816)
        h = (xv * g / (1.0 + np.exp(-g))).astype(np.float32).astype(np.float64)
        hq = act(h)
        mu, var = h[:, :2730].mean(1, keepdims=True), h[:, :2730].var(1, keepdims=True)
        wtl = np.zeros((1024, 2816), np.float32)
        wtl[:, :2730] = L["w2"][:, :2730].astype(np.float32) * L["mlnw"][:2730]
        wdq = wt(wtl)
        d = L["w2"][:, :2730].astype(np.float64) @ L["mlnb"][:2730].astype(np.float64)
        x = f16(x + (hq - mu) / np.sqrt(var + 1e-6) @ wdq.T + d)
    pool = x.reshape(nb, T, 1024)[:, 1:].mean(1)
    pn = f16(ln(pool, m["fnw"], m["fnb"]))
    nt = m["nt"]
    logit = act(pn) @ act(m["hw"][:nt]).T + m["hb"][:nt]     # head rows packed 1x128, each with its own scales
    return 1.0 / (1.0 + np.exp(-logit)), pn


def _sequenced_forward(orc, m, inp16, nl, sparse=False):
    """eva_forward's launch order (src/engine/eva.h:227-310) as a Python sequence of the oracle's primitives, each pinned
    above or in test_oracle.py: which tensor feeds which GEMM, which LayerNorm parameters serve which site, where the
    residual, the fold terms and the head bias enter."""
    nb, M = inp16.shape[0], inp16.shape[0] * 1025
    f32 = lambda a: np.asarray(a, np.float32)
    x = orc.embed(inp16.view(np.uint16), m["pe"].view(np.uint16), m["pos"], nb)

    def gemm(a8, s8, w, lda=1024):
        q, s = orc.quant_w(f32(w))
        if sparse:
            q = orc.prune24(q)
        return orc.gemm_f32(a8, s8, q, s, q.shape[0], threads=0, avx2=1), (q, s)

    for L in m["layers"][:nl]:
        h8, hs, _ = orc.ln_quant(x, L["ln1w"], L["ln1b"])
        acc, _ = gemm(h8, hs, L["wqkv"])
        q, k, vt = orc.qkv_epi(acc, nb, m["rope"])
        o = orc.attention(q, k, vt, nb)
        a8, as_ = orc.quant_act(o.astype(np.float32))
        acc, _ = gemm(a8, as_, L["wo"])
        x = orc.oproj_epi(acc, x)
        h8, hs, _ = orc.ln_quant(x, L["ln2w"], L["ln2b"])
        w12 = np.zeros((5632, 1024), np.float32)
        w12[:5472] = L["w12"]
        acc, _ = gemm(h8, hs, w12)
        h, stat = orc.fc1_epi(acc)
        m8, ms = orc.quant_act(h)
        wt, d = orc.fold_w2(L["w2"].view(np.uint16), L["mlnw"], L["mlnb"])
        acc, (q2, s2) = gemm(m8, ms, wt)
        x = orc.fc2_epi(acc, stat, orc.fold_c(q2, s2), d, x)
    p = orc.pool(x, nb)
    pn, pq, ps = orc.lnh(p, m["fnw"], m["fnb"])
    nt = m["nt"]
    qh, sh = orc.head_pack(m["hw"][:nt])
    logit = orc.gemm_rr_f64_rows(pq, ps, qh, sh, nt, np.arange(nb)).astype(np.float32)
    return (1.0 / (1.0 + np.exp(-(logit + m["hb"][:nt])))).astype(np.float32), pn


@pytest.mark.parametrize("sparse", [False, True])
def test_forward_equals_sequenced_primitives(orc, sparse):
    from xtagger_amd import blob
    nl, nt = 2, 600
    m = blob.synth_model(seed=31, nt=nt, nl=nl, head_std=0.05)
    r = np.random.default_rng(32)
    inp = np.zeros((1, 1024, 592), np.float16)
    inp[..., :588] = r.uniform(-1, 1, (1, 1024, 588))
    out, pn = orc.forward(m, inp, nl=nl, sparse=sparse)
    ref, pn_ref = _sequenced_forward(orc, m, inp, nl, sparse)
    assert (pn == pn_ref).all()
    assert np.abs(out - ref).max() <= 1e-6   # the sigmoid through libm expf (oracle) or numpy's exp


def test_forward_vs_float64_composition(orc):
    # coarse check of the same order from numpy float64 primitives: free running, the two differ by the noise of
    # E4M3 requantization after differently rounded sums (the oracle against itself, scalar vs AVX2 sums, differs
    # by 6.7e-4 in the head input and 5.6e-3 in sigmoid after one layer; this composition rounds every step
    # differently and sits at 6.3e-3 / 2.3e-2)
    from xtagger_amd import blob
    nl, nt = 1, 600
    m = blob.synth_model(seed=21, nt=nt, nl=nl, head_std=0.05)
    r = np.random.default_rng(22)
    inp = np.zeros((1, 1024, 592), np.float16)
    inp[..., :588] = r.uniform(-1, 1, (1, 1024, 588))
    out, pn = orc.forward(m, inp, nl=nl)
    ref, pn_ref = _f64_forward(orc, m, inp, nl)
    assert np.abs(f16_val(pn) - pn_ref).max() <= 0.02 * np.abs(pn_ref).max()
    assert np.abs(out - ref).max() <= 0.06
    top = lambda v: set(np.argsort(-v[0])[:50])
    assert len(top(out) & top(ref)) >= 45
