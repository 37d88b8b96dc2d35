"""Pins the oracle's PixAI (ViTDet-L) block epilogues (oracle/xt_oracle.c xo_px_*, px_kernels.cu) on the CPU.

Each check uses a formulation independent of the oracle's loops: RoPE as a complex multiplication in float64 with the
layouts built by numpy reshapes, GELU against torch's exact-erf GELU in float64 and the identity gelu(u) - gelu(-u) = u,
and the residual update against the wd model's out-projection epilogue (bias zero) and closed forms.
"""
import numpy as np
import torch


def _bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _bf16_f32(u16):
    return (np.asarray(u16, np.uint32) << 16).view(np.float32)


def test_px_qkv_epi_rope_as_complex_product(orc):
    """px_kernels.cu:84-98: (f0, f1) of pair i at token t rotates by the angle whose (cos, sin) is cs[t % L][i], i.e.
    (f0 + i f1) (c + i s); layouts q / k [S][16][L][64], vt [S][16][64][L] from reshapes."""
    L, S = 64, 3
    M = L * S
    r = np.random.default_rng(5)
    acc = (r.standard_normal((M, 3072)) * 2).astype(np.float32)
    bias = r.standard_normal(3072).astype(np.float32)
    ang = r.random((L, 32)) * 6.28
    cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    q, k, vt = orc.px_qkv_epi(acc, L, bias, cs)
    f = (acc + bias).astype(np.float64)                                  # the bias add is one fp32 rounding
    rot = (cs[..., 0] + 1j * cs[..., 1]).astype(np.complex128)           # [L][32]
    for part, got in ((0, q), (1, k)):
        z = f[:, part * 1024:(part + 1) * 1024].reshape(S, L, 16, 32, 2)
        z = (z[..., 0] + 1j * z[..., 1]) * rot[None, :, None, :]
        ref = np.stack([z.real, z.imag], -1).reshape(S, L, 16, 64).transpose(0, 2, 1, 3)
        g = _bf16_f32(got).astype(np.float64)
        # one fp32 rounding of each product and sum, then bf16: within one bf16 unit of the float64 rotation
        assert np.all(np.abs(g - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-6 * np.abs(f).max())
    vref = f[:, 2048:].reshape(S, L, 16, 64).transpose(0, 2, 3, 1)
    assert (vt == _bf16_bits(vref.astype(np.float32))).all()


def test_px_qkv_epi_identity_rotation_is_bias_add(orc):
    L, S = 128, 2
    r = np.random.default_rng(6)
    acc = r.standard_normal((L * S, 3072)).astype(np.float32)
    bias = r.standard_normal(3072).astype(np.float32)
    cs = np.zeros((L, 32, 2), np.float32)
    cs[..., 0] = 1.0
    q, k, _ = orc.px_qkv_epi(acc, L, bias, cs)
    f = acc + bias
    assert (q == _bf16_bits(f[:, :1024].reshape(S, L, 16, 64).transpose(0, 2, 1, 3))).all()
    assert (k == _bf16_bits(f[:, 1024:2048].reshape(S, L, 16, 64).transpose(0, 2, 1, 3))).all()


def test_px_qkv_epi_matches_wd_epilogue_on_shifted_table(orc):
    """With L = 1025, table row 0 the identity and rows 1.. the wd table, the PixAI epilogue at zero bias equals the wd
    epilogue (eva_kernels.cu:74-79, table row t - 1 for patch tokens, cls unrotated) on the unpadded rows."""
    nb = 2
    r = np.random.default_rng(7)
    acc = r.standard_normal((nb * 1025, 3072)).astype(np.float32)
    ang = r.random((1024, 32)) * 6.28
    cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    cs_px = np.concatenate([np.stack([np.ones((1, 32)), np.zeros((1, 32))], -1).astype(np.float32), cs])
    q, k, vt = orc.px_qkv_epi(acc, 1025, np.zeros(3072, np.float32), cs_px)
    qw, kw, vtw = orc.qkv_epi(acc, nb, cs)
    assert (q == qw[:, :, :1025]).all() and (k == kw[:, :, :1025]).all() and (vt == vtw[..., :1025]).all()


def test_px_fc1_epi_gelu_vs_torch_and_odd_identity(orc):
    r = np.random.default_rng(8)
    M = 6
    acc = (r.standard_normal((M, 4736)) * 3).astype(np.float32)
    acc[0, :8] = [0.0, -0.0, 1e-30, -1e-30, 12.0, -12.0, 40.0, -40.0]
    bias = (r.standard_normal(4736) * 0.5).astype(np.float32)
    h = orc.px_fc1_epi(acc, bias)
    u = (acc + bias).astype(np.float64)
    ref = torch.nn.functional.gelu(torch.from_numpy(u), approximate="none").numpy()
    assert np.all(np.abs(h - ref) <= 4 * 2.0 ** -24 * np.abs(u) + 1e-30)
    # gelu(u) - gelu(-u) = u (Phi(u) + Phi(-u) = 1): with bias zero, feeding acc and -acc
    z = np.zeros(4736, np.float32)
    hp, hn = orc.px_fc1_epi(acc, z), orc.px_fc1_epi(-acc, z)
    assert np.all(np.abs((hp.astype(np.float64) - hn) - acc) <= 4 * 2.0 ** -24 * np.abs(acc) + 1e-30)
    # the per-unit multiplier scales each column once
    rs = (r.random(4736) + 0.5).astype(np.float32)
    assert (orc.px_fc1_epi(acc, bias, rs) == (h * rs).astype(np.float32)).all()


def test_px_res_epi_reduces_to_oproj_and_closed_form(orc):
    r = np.random.default_rng(9)
    M = 40
    acc = r.standard_normal((M, 1024)).astype(np.float32)
    x = (r.standard_normal((M, 1024)) * 2).astype(np.float16).view(np.uint16)
    assert (orc.px_res_epi(acc, np.zeros(1024, np.float32), x) == orc.oproj_epi(acc, x)).all()
    bias = r.standard_normal(1024).astype(np.float32)
    got = orc.px_res_epi(np.zeros_like(acc), bias, x).view(np.float16)
    ref = (x.view(np.float16).astype(np.float32) + bias).astype(np.float16)
    assert (got == ref).all()


def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16)


def test_px_hln_vs_float64_layernorm(orc):
    """k_phln + k_phscore (px_kernels.cu:344-400): y = f16(LN_1e-5(x) g + b + hpos[m % T]) within one fp16 rounding of
    the float64 formula, a constant row gives b + hpos, and s = U y of the fp16 y (numpy matmul)."""
    r = np.random.default_rng(10)
    T, M = 48, 96
    x = _f16(r.standard_normal((M, 1024)) * 2 + 0.5)
    x[5] = np.float16(1.25)
    g = (1 + 0.1 * r.standard_normal(1024)).astype(np.float32)
    b = (0.1 * r.standard_normal(1024)).astype(np.float32)
    hpos = _f16(r.standard_normal((T, 1024)) * 0.2)
    U = (r.standard_normal((16, 1024)) * 0.05).astype(np.float32)
    y, s = orc.px_hln(x.view(np.uint16), T, g, b, hpos.view(np.uint16), U)
    xf = x.astype(np.float64)
    mean = xf.mean(1, keepdims=True)
    var = ((xf - mean) ** 2).mean(1, keepdims=True)
    ref = (xf - mean) / np.sqrt(var + 1e-5) * g + b + hpos[np.arange(M) % T].astype(np.float64)
    yf = y.view(np.float16).astype(np.float64)
    assert np.all(np.abs(yf - ref) <= 2.0 ** -10 * np.abs(ref) + 2.0 ** -24 + 1e-6 * np.abs(ref).max())
    assert (y.view(np.float16)[5] == _f16(b + hpos[5].astype(np.float32))).all()
    assert np.allclose(s, yf @ U.astype(np.float64).T, rtol=1e-12, atol=1e-12)


def test_px_hsoft_vs_softmax(orc):
    from scipy.special import softmax
    r = np.random.default_rng(11)
    nb, T = 2, 300
    s = (np.round(r.standard_normal((nb * T, 16)) * 4 * 1024) / 1024).astype(np.float32)   # s + 3 stays exact
    P = orc.px_hsoft(s, nb, T)
    ref = softmax(s.astype(np.float64).reshape(nb, T, 16) * np.log(2.0), axis=1).transpose(0, 2, 1)
    assert np.allclose(P, ref, rtol=1e-12, atol=0)
    assert np.allclose(P.sum(2), 1.0, atol=1e-12)
    assert np.allclose(orc.px_hsoft(s + np.float32(3.0), nb, T), P, rtol=1e-12)      # shift invariance


def test_px_hpool_hv_vs_matmul(orc):
    r = np.random.default_rng(12)
    nb, T = 2, 144
    P = _f16(r.random((nb, 16, T)) / T)
    y = _f16(r.standard_normal((nb * T, 1024)))
    wv = _f16(r.standard_normal((1024, 1024)) * 0.03)
    o = orc.px_hpool_hv(P.view(np.uint16), y.view(np.uint16), nb, T, wv.view(np.uint16))
    pooled = np.matmul(P.astype(np.float64), y.astype(np.float64).reshape(nb, T, 1024))      # [nb][16][1024]
    w = wv.astype(np.float64).reshape(16, 64, 1024)
    ref = np.einsum("hnd,bhd->bhn", w, pooled).reshape(nb, 1024)
    assert np.allclose(o, ref, rtol=1e-12, atol=1e-12)
    o2 = orc.px_hpool_hv((P.astype(np.float32) * 2).astype(np.float16).view(np.uint16), y.view(np.uint16), nb, T,
                         wv.view(np.uint16))
    assert np.allclose(o2, 2 * o, rtol=1e-12, atol=1e-12)                                   # linear in P


def test_px_pe_and_pembed_vs_float64(orc):
    """k_ppe + k_pembed (px_kernels.cu:16-50, 133-138): the patch GEMM against numpy's float64 matmul (one fp16
    rounding), and LN_1e-5(x + pos[m % T]) g + b against the float64 formula (one fp16 rounding; a row whose x + pos
    is constant gives b)."""
    r = np.random.default_rng(13)
    M, T = 64, 40
    inp = np.zeros((M, 592), np.float16)
    inp[:, :588] = _f16(r.uniform(-1, 1, (M, 588)))
    pe = np.zeros((1024, 592), np.float16)
    pe[:, :588] = _f16(r.standard_normal((1024, 588)) * 0.05)
    x = orc.px_pe(inp.view(np.uint16), pe.view(np.uint16)).view(np.float16)
    ref = inp.astype(np.float64) @ pe.astype(np.float64).T
    assert np.all(np.abs(x.astype(np.float64) - ref) <= 2.0 ** -11 * np.abs(ref) + 2.0 ** -25)
    pos = (r.standard_normal((T, 1024)) * 0.3).astype(np.float32)
    g = (1 + 0.1 * r.standard_normal(1024)).astype(np.float32)
    b = (0.1 * r.standard_normal(1024)).astype(np.float32)
    x2 = x.copy()
    pos[3] = 0.0
    x2[3] = np.float16(0.5)                                              # x + pos constant on row 3: variance 0
    y = orc.px_pembed(x2.view(np.uint16), T, pos, g, b).view(np.float16).astype(np.float64)
    assert (y[3] == b.astype(np.float16).astype(np.float64)).all()
    v = x2.astype(np.float64) + pos[np.arange(M) % T].astype(np.float64)
    mean = v.mean(1, keepdims=True)
    yr = (v - mean) / np.sqrt(((v - mean) ** 2).mean(1, keepdims=True) + 1e-5) * g + b
    rows = np.arange(M) != 3
    assert np.all(np.abs(y[rows] - yr[rows]) <= 2.0 ** -10 * np.abs(yr[rows]) + 1e-5 * np.abs(yr[rows]).max())
