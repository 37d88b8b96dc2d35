"""Pins the CPU oracle (oracle/xt_oracle.c) before it is trusted as the checker.

Each check compares the oracle with something independent of it: torch's float8_e4m3fn / bfloat16 / float16 casts,
numpy float64 linear algebra, closed forms of the OCP E4M3 format, or the per-tensor special case that reduces the
block-scaled GEMM to the reference's `alpha * acc` (src/engine/eva.h:415-418).
"""
import numpy as np
import pytest
import torch


# ---------------------------------------------------------------- E4M3 codec
def test_decode_table_matches_torch(orc):
    codes = torch.arange(256, dtype=torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()
    lut = orc.E4M3_LUT
    nan = np.isnan(ref)
    assert (np.isnan(lut) == nan).all()
    assert nan.sum() == 2 and nan[0x7F] and nan[0xFF]
    assert (lut[~nan] == ref[~nan]).all()


def test_decode_closed_forms(orc):
    lut = orc.E4M3_LUT
    assert lut[0x00] == 0.0 and lut[0x01] == 2.0 ** -9 and lut[0x07] == 7 * 2.0 ** -9
    assert lut[0x08] == 2.0 ** -6 and lut[0x38] == 1.0 and lut[0x7E] == 448.0
    pos = lut[:0x7F]
    assert (np.diff(pos) > 0).all(), "codes 0..0x7E increase"
    assert (lut[0x80:0xFF] == -lut[:0x7F]).all()


def test_encode_roundtrip_and_midpoints(orc):
    # every finite code encodes back to itself; exact midpoints between neighbours go to the even code
    lut = orc.E4M3_LUT
    codes = np.arange(0x7F, dtype=np.uint8)
    assert (orc.e4m3_encode(lut[codes]) == codes).all()
    assert (orc.e4m3_encode(-lut[codes[1:]]) == codes[1:] | 0x80).all()
    lo, hi = lut[codes[:-1]].astype(np.float64), lut[codes[1:]].astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    assert (mid.astype(np.float64) == (lo + hi) / 2).all()
    got = orc.e4m3_encode(mid)
    even = np.where(codes[:-1] % 2 == 0, codes[:-1], codes[1:])
    assert (got == even).all()
    # just above / below a midpoint goes to the nearer code
    up = np.nextafter(mid, np.float32(np.inf))
    dn = np.nextafter(mid, np.float32(-np.inf))
    assert (orc.e4m3_encode(up) == codes[1:]).all()
    assert (orc.e4m3_encode(dn) == codes[:-1]).all()


def test_encode_saturates_and_flushes(orc):
    big = np.array([448.0, 448.5, 463.9, 464.0, 480.0, 1e6, 3.4e38, np.inf], np.float32)
    assert (orc.e4m3_encode(big) == 0x7E).all()
    assert (orc.e4m3_encode(-big) == 0xFE).all()
    tiny = np.array([0.0, 1e-30, 2.0 ** -11, 2.0 ** -10], np.float32)  # 2^-10 is a tie between 0 and 2^-9 -> 0
    assert (orc.e4m3_encode(tiny) == 0).all()
    assert orc.e4m3_encode(np.array([np.nextafter(np.float32(2.0 ** -10), np.float32(1))]))[0] == 1


@pytest.mark.parametrize("exp_lo,exp_hi", [(110, 118), (118, 126), (126, 131), (131, 137)])
def test_encode_exhaustive_vs_torch(orc, exp_lo, exp_hi):
    # every fp32 bit pattern with biased exponent in [exp_lo, exp_hi), both signs: values 2^-17 .. 2^10
    for sign in (0, 1):
        first = (sign << 31) | (exp_lo << 23)
        count = (exp_hi - exp_lo) << 23
        got = orc.e4m3_encode_bits(first, count)
        x = (np.arange(count, dtype=np.uint64) + first).astype(np.uint32).view(np.float32)
        ref = torch.from_numpy(np.clip(x, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert (got == ref).all(), f"exponents [{exp_lo},{exp_hi}) sign {sign}"


def test_encode_outside_exhaustive_range(orc):
    # below 2^-17 everything is +-0; at or above 2^10 everything saturates (strided over every pattern)
    for sign in (0, 1):
        lo = orc.e4m3_encode_bits((sign << 31), 110 << 23)[:: 9973]
        assert (lo == (sign << 7)).all()
        hi = orc.e4m3_encode_bits((sign << 31) | (137 << 23), (255 - 137) << 23)[:: 9973]
        assert (hi == ((sign << 7) | 0x7E)).all()


# ---------------------------------------------------------------- bf16 / fp16
def _specials():
    r = np.random.default_rng(0)
    x = np.concatenate([r.standard_normal(200000).astype(np.float32) * 10.0 ** r.integers(-8, 5, 200000),
                        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, 6e-8, 3e-8, 2.0 ** -24, 2.0 ** -25,
                                  1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8],
                                 np.float32)])
    return x.astype(np.float32)


def test_bf16_rne_vs_torch(orc):
    x = _specials()
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = np.array([orc.lib.xo_f32_to_bf16(float(v)) for v in x[:20000]] +
                   [orc.lib.xo_f32_to_bf16(float(v)) for v in x[-14:]], np.uint16)
    assert (got == np.concatenate([ref[:20000], ref[-14:]])).all()


def test_f16_rne_vs_torch(orc):
    x = _specials()
    ref = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    sel = np.concatenate([np.arange(20000), np.arange(x.size - 14, x.size)])
    got = np.array([orc.lib.xo_f32_to_f16(float(x[i])) for i in sel], np.uint16)
    assert (got == ref[sel]).all()
    back = np.array([orc.lib.xo_f16_to_f32(int(h)) for h in ref[sel]], np.float32)
    assert (back == torch.from_numpy(ref[sel].view(np.int16)).view(torch.float16).float().numpy()).all()


# ---------------------------------------------------------------- block packing
def _contract_scale(amax):
    """export_eva.py:64-66's sc = amax / 448 in float64, rounded once to fp32 (a float64 quotient of two fp32 values
    rounds to the correctly rounded fp32 quotient: 53 >= 2 * 24 + 2), 1 below 2^-116."""
    amax = np.asarray(amax, np.float32).astype(np.float64)
    return np.where(amax < 2.0 ** -116, 1.0, amax / 448.0).astype(np.float32)


def test_block_scale_rule(orc):
    """xo_block_scale = amax / 448 correctly rounded, on binade edges, near the zero-block threshold and on 20000 random
    maxima (where amax * float32(1 / 448), a plausible slip, differs from the quotient in a large share of cases)."""
    edge = [2.0 ** -116, np.nextafter(np.float32(2.0 ** -116), np.float32(0)), 2.0 ** -100, 1e-30, 0.5, 1.0, 1.75,
            1.9999999, 447.0, 448.0, np.nextafter(np.float32(448), np.float32(1e9)), 449.0, 896.0, 3e38]
    r = np.random.default_rng(11)
    rnd = (r.random(20000) * 2.0 ** r.integers(-60, 60, 20000)).astype(np.float32)
    v = np.concatenate([np.array(edge, np.float32), rnd])
    got = np.array([orc.lib.xo_block_scale(float(a)) for a in v], np.float32)
    assert (got == _contract_scale(v)).all()
    slip = (v * np.float32(1.0 / 448.0)).astype(np.float32)
    assert np.mean(slip != got) > 0.1, "the random maxima must tell a quotient from a product with 1/448"
    assert orc.lib.xo_block_scale(0.0) == 1.0 and orc.lib.xo_block_scale(2.0 ** -117) == 1.0


def _blocks_ok(x, q, s, orc):
    """decode(q) * s reconstructs x to E4M3 precision; every non-zero block's maximum decodes to exactly 448."""
    M, K = x.shape
    dq = orc.e4m3_decode(q)[:, :K].reshape(M, K // 128, 128)
    sc = s[:, :M].T[:, :, None]
    xr = x.reshape(M, K // 128, 128)
    err = np.abs(dq * sc - xr)
    assert (err <= np.maximum(np.abs(xr) * 2.0 ** -4, sc * 2.0 ** -10) * 1.0001).all()
    amax = np.abs(xr).max(2)
    nz = amax >= 2.0 ** -116
    assert (np.abs(dq).max(2)[nz] == 448.0).all()
    assert (s[:, :M].T[~nz] == 1.0).all()


def test_quant_act_vs_independent(orc):
    r = np.random.default_rng(1)
    x = r.standard_normal((67, 512)).astype(np.float32)
    x[3] = 0.0
    x[5, :128] *= 1e-3
    x[7, 256:384] = 1e-40  # below the zero-block threshold
    q, s = orc.quant_act(x, lds=70)
    xb = x.reshape(67, 4, 128)
    amax = np.abs(xb).max(2)
    sc = _contract_scale(amax)
    assert (s[:, :67].T == sc).all() and (s[:, 67:] == 0).all()
    inv = (np.float32(1) / sc).astype(np.float32)
    y = np.clip(xb * inv[:, :, None], -448, 448).astype(np.float32)
    ref = torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy().reshape(67, 512)
    assert (q == ref).all()
    _blocks_ok(x, q, s, orc)


def test_quant_w_vs_independent(orc):
    r = np.random.default_rng(2)
    w = (r.standard_normal((300, 256)) * 0.02).astype(np.float32)
    q, s = orc.quant_w(w)
    assert q.shape == (384, 256) and s.shape == (3, 2)
    assert (q[300:] == 0).all()
    for nb in range(3):
        for kb in range(2):
            blk = w[nb * 128:nb * 128 + 128, kb * 128:kb * 128 + 128]
            sc = _contract_scale(np.abs(blk).max())
            assert s[nb, kb] == sc
            y = np.clip(blk / sc, -448, 448).astype(np.float32)
            ref = torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert (q[nb * 128:nb * 128 + blk.shape[0], kb * 128:kb * 128 + 128] == ref).all()


# ---------------------------------------------------------------- block-scaled GEMM
def _operands(M, N, K, seed=3):
    r = np.random.default_rng(seed)
    x = r.standard_normal((M, K)).astype(np.float32)
    w = (r.standard_normal((N, K)) * 0.02).astype(np.float32)
    return x, w


def _numpy_ref(orc, qa, sa, qw, sw, M, N, K):
    a = orc.e4m3_decode(qa).astype(np.float64)
    b = orc.e4m3_decode(qw[:N]).astype(np.float64)
    out = np.zeros((M, N))
    for kb in range(K // 128):
        ks = slice(kb * 128, kb * 128 + 128)
        part = a[:, ks] @ b[:, ks].T
        out += part * sa[kb, :M, None].astype(np.float64) * np.repeat(sw[:, kb], 128)[None, :N].astype(np.float64)
    return out


def test_gemm_f64_vs_numpy(orc):
    M, N, K = 37, 300, 384
    x, w = _operands(M, N, K)
    qa, sa = orc.quant_act(x)
    qw, sw = orc.quant_w(w)
    ref = _numpy_ref(orc, qa, sa, qw, sw, M, N, K)
    got = orc.gemm_f64_rows(qa, sa, qw, sw, N, np.arange(M))
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("avx2", [0, 1])
def test_gemm_f32_vs_f64(orc, avx2):
    M, N, K = 65, 260, 512
    x, w = _operands(M, N, K, seed=4)
    qa, sa = orc.quant_act(x)
    qw, sw = orc.quant_w(w)
    ref = orc.gemm_f64_rows(qa, sa, qw, sw, N, np.arange(M))
    cf, cb = orc.gemm_f32(qa, sa, qw, sw, N, avx2=avx2, want_bf16=True)
    assert np.abs(cf - ref).max() <= 1e-5 * np.abs(ref).max()
    b = torch.from_numpy(cf).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert (cb == b).all()


def test_gemm_per_tensor_special_case(orc):
    """All block scales equal: the block-scaled product is alpha * (qa . qw^T), the reference's alpha epilogue."""
    M, N, K = 20, 128, 256
    r = np.random.default_rng(5)
    qa = r.integers(0, 256, (M, K), dtype=np.uint8)
    qw = r.integers(0, 256, (N, K), dtype=np.uint8)
    qa[(qa & 0x7F) == 0x7F] = 0
    qw[(qw & 0x7F) == 0x7F] = 0
    a_s, w_s = np.float32(0.0123), np.float32(0.0457)
    sa = np.full((K // 128, M), a_s, np.float32)
    sw = np.full((1, K // 128), w_s, np.float32)
    alpha = float(np.float64(a_s) * np.float64(w_s))
    ref = alpha * (orc.e4m3_decode(qa).astype(np.float64) @ orc.e4m3_decode(qw).astype(np.float64).T)
    got = orc.gemm_f64_rows(qa, sa, qw, sw, N, np.arange(M))
    assert np.allclose(got, ref, rtol=1e-12, atol=0)


def test_kcheck_generator():
    """kcheck.c:21-22 LCG restated: first values from seed 12345."""
    from tests.kcheck import Lcg
    g = Lcg()
    v = [g.next_u32() for _ in range(3)]
    rs = 12345
    exp = []
    for _ in range(3):
        rs = (rs * 1664525 + 1013904223) & 0xFFFFFFFF
        exp.append(rs)
    assert v == exp
    f = Lcg().frand()
    assert -1.0 <= f < 1.0


# ---------------------------------------------------------------- LayerNorm -> E4M3
def test_ln_quant_vs_float64(orc):
    r = np.random.default_rng(6)
    x = (r.standard_normal((33, 1024)) * 3 + 0.5).astype(np.float16)
    g = (1 + 0.1 * r.standard_normal(1024)).astype(np.float32)
    b = (0.05 * r.standard_normal(1024)).astype(np.float32)
    q, s, y = orc.ln_quant(x.view(np.uint16), g, b)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    var = ((xd - mu) ** 2).mean(1, keepdims=True)
    ref = (xd - mu) / np.sqrt(var + 1e-6) * g + b
    assert np.abs(y - ref).max() < 1e-5 * np.abs(ref).max()
    q2, s2 = orc.quant_act(y)
    assert (q2 == q).all() and (s2 == s).all()


def test_kcheck_generators_c_match_python(orc):
    from tests.kcheck import Lcg as PyLcg
    a, b = PyLcg(), orc.Lcg()
    assert (a.frand_n(1000) == b.frand(1000)).all()
    assert (a.e4m3_bytes(5000) == b.e4m3(5000)).all()
    assert a.rs == int(b.rs[0])
