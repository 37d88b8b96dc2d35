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
