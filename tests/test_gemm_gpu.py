"""GPU parity of the E4M3 packing kernels and the block-scaled FP8 GEMM, through the C-ABI (libxtag_eva.so).

Packing is bit-exact against the oracle; the GEMM is within 1e-3 (max-abs relative to max |ref|, and normwise) of
the fp64 dequantized product, checked on the fp32-output build of the same kernel; the bf16 output is the RNE of
the fp32 output. Shapes: the EVA02-L qkv shape at batch 1 (M=1025, K=1024, N=3072), the layer shapes at M=8200 on
sampled rows, ragged M, and the reference's own kcheck.c method for k_oproj (LCG operands, 97 sampled rows).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _run(rc, what):
    assert rc == 0, f"{what} returned {rc}"
    torch.cuda.synchronize()


# ---------------------------------------------------------------- E4M3 encoder, every fp32 bit pattern
def test_e4m3_encoder_exhaustive(dev, xt, orc):
    chunk = 1 << 28
    out = torch.empty(chunk, dtype=torch.uint8, device=dev)
    for c in range(16):
        first = c * chunk
        _say(f"encoder chunk {c}")
        _run(xt.lib.eva_k_e4m3_bits(first, chunk, xt.ptr(out), _stream()), "eva_k_e4m3_bits")
        got = out.cpu().numpy()
        ref = orc.e4m3_encode_bits(first, chunk)
        bad = got != ref
        if c in (7, 15):                              # NaN patterns (outside the contract) sit at the chunk's top
            bad[0x0F800001:] = False
        assert not bad.any(), f"first mismatch at bits {hex(first + int(np.argmax(bad)))}"


# ---------------------------------------------------------------- activation / weight packing
def _act_inputs(M, K, seed):
    r = np.random.default_rng(seed)
    x = r.standard_normal((M, K)).astype(np.float32)
    x[0] = 0.0                                        # zero row -> scale 1
    if M > 3:
        x[1, :128] *= 1e-30                           # tiny block
        x[2, 128:256] = 448.0 * 3                     # constant block, saturating
        x[3, ::7] = 0.0
    return x


@pytest.mark.parametrize("kind", ["bf16", "fp32"])
@pytest.mark.parametrize("M,K", [(1025, 1024), (37, 2816), (1, 128)])
def test_quant_act_bitexact(dev, xt, orc, kind, M, K):
    _say(f"quant_act {kind} M={M} K={K}")
    x = _act_inputs(M, K, seed=M + K)
    if kind == "bf16":
        xt_in = torch.from_numpy(x).to(torch.bfloat16)
        x = xt_in.float().numpy()
        in_kind = 0
    else:
        xt_in = torch.from_numpy(x)
        in_kind = 1
    lds = M + 3
    d_x = xt_in.to(dev)
    d_q = torch.zeros((M, K), dtype=torch.uint8, device=dev)
    d_s = torch.zeros((K // 128, lds), dtype=torch.float32, device=dev)
    _run(xt.lib.eva_k_quant_act(xt.ptr(d_x), in_kind, K, M, K, xt.ptr(d_q), K, xt.ptr(d_s), lds, _stream()),
         "eva_k_quant_act")
    q, s = orc.quant_act(x, lds=lds)
    assert (d_q.cpu().numpy() == q).all()
    assert (d_s.cpu().numpy() == s).all()


@pytest.mark.parametrize("N,K", [(3072, 1024), (10861, 1024), (1024, 2816)])
def test_quant_w_bitexact(dev, xt, orc, N, K):
    _say(f"quant_w N={N} K={K}")
    r = np.random.default_rng(N)
    w = (r.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[:128, :128] = 0.0                               # zero block -> scale 1
    NB = (N + 127) // 128
    d_w = torch.from_numpy(w).to(dev)
    d_q = torch.full((NB * 128, K), 0x55, dtype=torch.uint8, device=dev)
    d_s = torch.zeros((NB, K // 128), dtype=torch.float32, device=dev)
    _run(xt.lib.eva_k_quant_w(xt.ptr(d_w), N, K, xt.ptr(d_q), xt.ptr(d_s), _stream()), "eva_k_quant_w")
    q, s = orc.quant_w(w)
    assert (d_q.cpu().numpy() == q).all()
    assert (d_s.cpu().numpy() == s).all()


# ---------------------------------------------------------------- block-scaled GEMM
def _packed(M, N, K, seed):
    r = np.random.default_rng(seed)
    x = r.standard_normal((M, K)).astype(np.float32)
    w = (r.standard_normal((N, K)) * 0.02).astype(np.float32)
    return x, w


def _gpu_gemm(dev, xt, qa, sa, qw, sw, M, N, K, out_kind):
    d_a = torch.from_numpy(qa).to(dev)
    d_sa = torch.from_numpy(np.ascontiguousarray(sa)).to(dev)
    d_w = torch.from_numpy(qw).to(dev)
    d_sw = torch.from_numpy(sw).to(dev)
    dt = torch.bfloat16 if out_kind == 0 else torch.float32
    d_c = torch.full((M, N), float("nan"), dtype=dt, device=dev)
    _run(xt.lib.eva_k_gemm(xt.ptr(d_a), K, xt.ptr(d_sa), sa.shape[1], xt.ptr(d_w), xt.ptr(d_sw), M, N, K,
                           xt.ptr(d_c), N, out_kind, _stream()), "eva_k_gemm")
    return d_c.cpu()


def _check_gemm(c, ref):
    c = c.astype(np.float64)
    assert np.isfinite(c).all()
    err = np.abs(c - ref)
    _say(f"  max err / max|ref| {err.max() / np.abs(ref).max():.3g}, "
         f"normwise {np.linalg.norm(c - ref) / np.linalg.norm(ref):.3g}")
    assert err.max() <= 1e-3 * np.abs(ref).max(), f"max err {err.max()} vs max|ref| {np.abs(ref).max()}"
    assert np.linalg.norm(c - ref) <= 1e-3 * np.linalg.norm(ref)


@pytest.mark.parametrize("M,N,K", [(1025, 3072, 1024), (1, 128, 128), (17, 384, 256), (255, 1024, 2816),
                                   (129, 10861, 1024),
                                   # 256 x 256 tiles (>= 256 tiles): one, three and an odd number of K blocks, ragged M
                                   (4100, 4096, 128), (4096, 4096, 384), (4000, 4224, 640)])
def test_gemm_parity(dev, xt, orc, M, N, K):
    _say(f"gemm M={M} N={N} K={K}")
    x, w = _packed(M, N, K, seed=M * 7 + N)
    qa, sa = orc.quant_act(x)
    qw, sw = orc.quant_w(w)
    rows = np.arange(M) if M * N * K <= 4e9 else np.linspace(0, M - 1, 97).astype(np.int32)
    ref = orc.gemm_f64_rows(qa, sa, qw, sw, N, rows)
    c32 = _gpu_gemm(dev, xt, qa, sa, qw, sw, M, N, K, 1).numpy()
    _check_gemm(c32[rows], ref)
    c16 = _gpu_gemm(dev, xt, qa, sa, qw, sw, M, N, K, 0)
    rne = torch.from_numpy(c32).to(torch.bfloat16)
    assert torch.equal(c16.view(torch.int16), rne.view(torch.int16)), "bf16 store is not RNE of the fp32 result"


@pytest.mark.parametrize("N,K", [(3072, 1024), (1024, 1024), (5632, 1024), (1024, 2816)])
def test_gemm_layer_shapes_m8200(dev, xt, orc, N, K):
    M = 8200
    _say(f"gemm layer shape M={M} N={N} K={K}")
    x, w = _packed(M, N, K, seed=N + K)
    qa, sa = orc.quant_act(x)
    qw, sw = orc.quant_w(w)
    rows = np.array(sorted(set(np.linspace(0, M - 1, 61).astype(np.int32)) | {M - 1, M - 8, 127, 128}), np.int32)
    ref = orc.gemm_f64_rows(qa, sa, qw, sw, N, rows)
    c32 = _gpu_gemm(dev, xt, qa, sa, qw, sw, M, N, K, 1).numpy()
    _check_gemm(c32[rows], ref)


def test_gemm_kcheck_oproj_method(dev, xt, orc):
    """kcheck.c:100-127 restated for the k_oproj operands: LCG E4M3 bytes (no NaN, exponent <= 9), alpha 0.001
    (all activation scales 0.001, all weight scales 1), fp64 loops on the 97 rows m = 7919 i mod 8200."""
    from tests.kcheck import sample_rows
    rows_n, D = 8 * 1025, 1024
    g = orc.Lcg(12345)
    g.frand(8 * 1024 * 588 + 1024 * 588)              # k_pe's operands come first (kcheck.c:80-83, 588 draws a row)
    a = g.e4m3(rows_n * D).reshape(rows_n, D)
    w = g.e4m3(D * D).reshape(D, D)
    sa = np.full((D // 128, rows_n), 0.001, np.float32)
    sw = np.ones((D // 128, D // 128), np.float32)
    rows = sample_rows(rows_n)
    ref = orc.gemm_f64_rows(a, sa, w, sw, D, rows)
    c = _gpu_gemm(dev, xt, a, sa, w, sw, rows_n, D, D, 1).numpy()[rows].astype(np.float64)
    err = np.abs(c - ref).max()
    _say(f"kcheck k_oproj-style max |err| {err:.3g} (max |ref| {np.abs(ref).max():.3f})")
    # kcheck's operands span products 2^-18 .. 56 inside one K block; the f8f6f4 matrix core sums them with less
    # than fp32 precision (observed ~6e-5 of max |ref|), so the bound is the GEMM contract, 1e-3
    assert err <= 1e-3 * np.abs(ref).max()
