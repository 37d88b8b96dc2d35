"""GPU parity of the 2:4-sparse weight path (EVA_SPARSE24) through the C-ABI.

- eva_k_prune24 and eva_k_pack24 are bit-exact against the oracle's xo_prune24 / xo_pack24 (themselves pinned by
  tests/test_sparse_oracle.py against numpy restatements of src/tools/prune24.py and of the layout's definition).
- eva_k_gemm_sp (v_smfmac_f32_16x16x128_fp8_fp8) against the oracle's fp64 product of the same pruned weights (the
  "dense-decoded reference"): the GEMM contract, max |C - Cref| <= 1e-3 max |Cref| and normwise 1e-3; and against the
  dense kernel on the same pruned weights, which sums the same products.
- The four layer kernels with sparse weights against the same kernels with the pruned weights stored dense: identical
  epilogues, so outputs agree to one rounding unit of their type.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

T, D, HID, HIDP = 1025, 1024, 2730, 2816


def _say(*a):
    print(*a, flush=True)


def _st():
    return torch.cuda.current_stream().cuda_stream


def _ok(rc, what):
    assert rc == 0, f"{what} returned {rc}"
    torch.cuda.synchronize()


_KEEP = []


@pytest.fixture(autouse=True)
def _release():
    yield
    _KEEP.clear()


def _d(a, dev):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    _KEEP.append(t)
    return t


def _codes(rng, shape, few=False):
    if few:
        mags = np.array([0x00, 0x20, 0x30, 0x38, 0x40, 0x48], np.uint8)
        q = mags[rng.integers(0, len(mags), size=shape)]
    else:
        q = rng.integers(0, 0x7F, size=shape).astype(np.uint8)
    return q | (rng.integers(0, 2, size=shape).astype(np.uint8) << 7)


def _pack_dev(xt, dev, q):
    N, K = q.shape
    vals = torch.empty((N // 16, K // 128, 64, 16), dtype=torch.uint8, device=dev)
    idx = torch.empty((N // 16, K // 128, 64), dtype=torch.int32, device=dev)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    _ok(xt.lib.eva_k_pack24(xt.ptr(_d(q, dev)), N, K, xt.ptr(vals), xt.ptr(idx), xt.ptr(bad), _st()), "eva_k_pack24")
    _KEEP.extend([vals, idx])
    return vals, idx, int(bad.item())


@pytest.mark.parametrize("few", [False, True])
def test_prune24_bitexact(dev, xt, orc, few):
    rng = np.random.default_rng(21 + few)
    q = _codes(rng, (512, 1024), few)
    d_q = _d(q, dev)
    _ok(xt.lib.eva_k_prune24(xt.ptr(d_q), 512, 1024, _st()), "eva_k_prune24")
    assert (d_q.cpu().numpy() == orc.prune24(q)).all()


def test_pack24_bitexact(dev, xt, orc):
    rng = np.random.default_rng(31)
    for few in (False, True):
        p = orc.prune24(_codes(rng, (256, 2816), few))
        vals, idx, bad = _pack_dev(xt, dev, p)
        rv, ri = orc.pack24(p)
        assert bad == 0
        assert (vals.cpu().numpy() == rv).all()
        assert (idx.cpu().numpy().view(np.uint32) == ri).all()
    dense = _codes(rng, (16, 128))
    dense[0, :4] = [0x38, 0x40, 0x48, 0x30]                                # one group with 4 nonzero bytes
    assert _pack_dev(xt, dev, dense)[2] >= 1


def _gemm_case(orc, M, N, K, seed):
    r = np.random.default_rng(seed)
    qa, sa = orc.quant_act(r.standard_normal((M, K)).astype(np.float32))
    qw, sw = orc.quant_w((r.standard_normal((N, K)) * 0.02).astype(np.float32))
    return qa, sa, orc.prune24(qw), sw


@pytest.mark.parametrize("M,N,K", [(1025, 3072, 1024), (777, 1024, 2816), (8200, 1024, 1024)])
def test_gemm_sp_contract(dev, xt, orc, M, N, K):
    _say(f"eva_k_gemm_sp M={M} N={N} K={K}")
    qa, sa, qp, sw = _gemm_case(orc, M, N, K, 41 + M)
    vals, idx, bad = _pack_dev(xt, dev, qp)
    assert bad == 0
    d_qa, d_sa, d_sw = _d(qa, dev), _d(sa, dev), _d(sw, dev)
    c_sp = torch.empty((M, N), dtype=torch.float32, device=dev)
    c_dn = torch.empty((M, N), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_gemm_sp(xt.ptr(d_qa), K, xt.ptr(d_sa), M, xt.ptr(vals), xt.ptr(idx), xt.ptr(d_sw), M, N, K,
                             xt.ptr(c_sp), N, 1, _st()), "eva_k_gemm_sp")
    _ok(xt.lib.eva_k_gemm(xt.ptr(d_qa), K, xt.ptr(d_sa), M, xt.ptr(_d(qp, dev)), xt.ptr(d_sw), M, N, K, xt.ptr(c_dn), N,
                          1, _st()), "eva_k_gemm")
    sp, dn = c_sp.cpu().numpy().astype(np.float64), c_dn.cpu().numpy().astype(np.float64)
    rows = np.unique(np.concatenate([(np.arange(97) * 7919) % M, [0, M - 1]])).astype(np.int32)
    ref = orc.gemm_f64_rows(qa, sa, qp, sw, N, rows)
    amax = np.abs(ref).max()
    err = np.abs(sp[rows] - ref).max() / amax
    nerr = np.linalg.norm(sp[rows] - ref) / np.linalg.norm(ref)
    vs_dense = np.abs(sp - dn).max() / np.abs(dn).max()
    _say(f"  vs fp64: max {err:.2e}, normwise {nerr:.2e}; vs dense kernel on pruned weights: {vs_dense:.2e}")
    assert err <= 1e-3 and nerr <= 1e-3
    assert vs_dense <= 1e-4


def test_gemm_sp_extreme_scales(dev, xt, orc):
    """Block scales over a wide range on the sparse loop, whose per-K-block promotion must honour any fp32 scale: rows
    with a block 2^-60 smaller than the rest (at K block 5, and at block 0), a row 2^70 larger throughout, a row with one
    block 2^70 larger, and waves of ordinary rows next to them: every row within 1e-3 of its own fp64 maximum, and
    within 1e-4 of the dense kernel on the same pruned weights. (A variant that carried the accumulators in units of
    each block's scale product overflows on such rows unless it checks them first.)"""
    M, N, K = 320, 512, 1024
    r = np.random.default_rng(77)
    x = r.standard_normal((M, K)).astype(np.float32)
    x[70, 640:768] *= np.float32(2.0 ** -60)      # wave of rows 64..127: scale product below 2^-40 at K block 5
    x[75, 0:128] *= np.float32(2.0 ** -60)        # the same wave, at block 0 as well
    x[200, :] *= np.float32(2.0 ** 70)            # wave of rows 192..255: products above 2^40 from the start
    x[260, 384:512] *= np.float32(2.0 ** 70)      # wave of rows 256..319: one huge block at K block 3
    qa, sa = orc.quant_act(x)
    qw, sw = orc.quant_w((r.standard_normal((N, K)) * 0.02).astype(np.float32))
    qp = orc.prune24(qw)
    vals, idx, bad = _pack_dev(xt, dev, qp)
    assert bad == 0
    d_qa, d_sa, d_sw = _d(qa, dev), _d(sa, dev), _d(sw, dev)
    c_sp = torch.empty((M, N), dtype=torch.float32, device=dev)
    c_dn = torch.empty((M, N), dtype=torch.float32, device=dev)
    _ok(xt.lib.eva_k_gemm_sp(xt.ptr(d_qa), K, xt.ptr(d_sa), M, xt.ptr(vals), xt.ptr(idx), xt.ptr(d_sw), M, N, K,
                             xt.ptr(c_sp), N, 1, _st()), "eva_k_gemm_sp")
    _ok(xt.lib.eva_k_gemm(xt.ptr(d_qa), K, xt.ptr(d_sa), M, xt.ptr(_d(qp, dev)), xt.ptr(d_sw), M, N, K, xt.ptr(c_dn), N,
                          1, _st()), "eva_k_gemm")
    sp, dn = c_sp.cpu().numpy().astype(np.float64), c_dn.cpu().numpy().astype(np.float64)
    rows = np.arange(M, dtype=np.int32)
    ref = orc.gemm_f64_rows(qa, sa, qp, sw, N, rows)
    assert np.isfinite(sp).all()
    rmax = np.abs(ref).max(1, keepdims=True)
    err = (np.abs(sp - ref) / rmax).max(1)
    vs_dense = (np.abs(sp - dn) / np.abs(dn).max(1, keepdims=True)).max(1)
    _say(f"  worst row vs fp64 {err.max():.2e} (rows 70, 75, 200, 260: {err[[70, 75, 200, 260]]}), "
         f"vs dense {vs_dense.max():.2e}")
    assert err.max() <= 1e-3
    assert vs_dense.max() <= 1e-4


# ---------------------------------------------------------------- layer kernels: sparse vs dense on pruned weights
class _Layer:
    def __init__(self, torch_, xt, orc, dev, M, seed=5):
        self.xt, self.dev, self.M = xt, dev, M
        g = torch.Generator(device=dev)
        g.manual_seed(seed)
        self.lds = lds = M + 64
        z = lambda *s, dt=torch.uint8: torch.zeros(*s, dtype=dt, device=dev)
        x = torch.randn(M, D, generator=g, device=dev)
        h = torch.randn(M, HIDP, generator=g, device=dev) * 0.3
        h[:, HID:] = 0
        self.a8, self.as_ = z(M, D), z(8, lds, dt=torch.float32)
        self.m8, self.ms = z(M, HIDP), z(22, lds, dt=torch.float32)
        _ok(xt.lib.eva_k_quant_act(xt.ptr(x), 1, D, M, D, xt.ptr(self.a8), D, xt.ptr(self.as_), lds, _st()), "act")
        _ok(xt.lib.eva_k_quant_act(xt.ptr(h), 1, HIDP, M, HIDP, xt.ptr(self.m8), HIDP, xt.ptr(self.ms), lds, _st()), "h")
        hn = h.double()
        blocks = hn.view(M, 22, 128)
        self.stat = torch.stack([blocks.sum(2).T, (blocks ** 2).sum(2).T], -1).float().contiguous()
        self.stat = torch.nn.functional.pad(self.stat, (0, 0, 0, lds - M)).contiguous()
        scratch = z(2 * HIDP * D, dt=torch.float32)
        self.w = {}
        for name, n_in, k_in, n_out, k_out, perm in (("qkv", 3 * D, D, 3 * D, D, 1), ("oproj", D, D, D, D, 0),
                                                     ("fc1", 2 * 2736, D, 2 * HIDP, D, 0), ("fc2", D, HID, D, HIDP, 0)):
            w16 = (torch.randn(n_in, k_in, generator=g, device=dev) * 0.02).half()
            q, s = z(n_out, k_out), z(n_out // 128, k_out // 128, dt=torch.float32)
            _ok(xt.lib.eva_k_prep_w(xt.ptr(w16), k_in, n_in, k_in, n_out, k_out, perm, None, xt.ptr(scratch),
                                    xt.ptr(q), xt.ptr(s), _st()), "prep")
            _ok(xt.lib.eva_k_prune24(xt.ptr(q), n_out, k_out, _st()), "prune")
            vals = z(n_out // 16, k_out // 128, 64, 16)
            idx = z(n_out // 16, k_out // 128, 64, dt=torch.int32)
            _ok(xt.lib.eva_k_pack24(xt.ptr(q), n_out, k_out, xt.ptr(vals), xt.ptr(idx), None, _st()), "pack")
            self.w[name] = (q, s, vals, idx)
        self.cn = torch.randn(D, generator=g, device=dev) * 0.1
        self.dn = torch.randn(D, generator=g, device=dev) * 0.01
        self.cs = torch.rand(1024, 32, 2, generator=g, device=dev)
        self.x0 = torch.randn(M, D, generator=g, device=dev).half()


def _close16(name, a, b, kind):
    """Values of two 16-bit outputs (bf16 or fp16 bit patterns) agree to one rounding unit of the type relative to the
    value, plus 1e-4 of the tensor's largest value: both sums are of the same products in different orders (~1e-5
    relative), which near a cancellation can even flip the sign of a tiny value."""
    if kind == "bf16":
        fa = (a.astype(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        fb = (b.astype(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        unit = 2.0 ** -7
    else:
        fa = a.view(np.float16).astype(np.float64)
        fb = b.view(np.float16).astype(np.float64)
        unit = 2.0 ** -10
    err = np.abs(fa - fb)
    bound = unit * np.abs(fa) + 1e-4 * np.abs(fa).max()
    worst = float((err / bound).max())
    _say(f"  {name}: worst err / bound {worst:.3f}, elements differing {np.mean(err > 0):.2e}")
    assert worst <= 1.0, name


@pytest.fixture(scope="module")
def layer(dev, xt, orc):
    return _Layer(torch, xt, orc, dev, 2 * T)


def test_qkv_sp(dev, xt, layer):
    L, M = layer, layer.M
    nb = M // T
    outs = []
    for sp in (False, True):
        q, k, vt = (torch.zeros(nb, 16, 1088, 64, dtype=torch.int16, device=dev) for _ in range(3))
        wq, ws, vals, idx = L.w["qkv"]
        if sp:
            rc = xt.lib.eva_k_qkv_sp(xt.ptr(L.a8), xt.ptr(L.as_), L.lds, xt.ptr(vals), xt.ptr(idx), xt.ptr(ws),
                                     xt.ptr(L.cs), xt.ptr(q), xt.ptr(k), xt.ptr(vt), M, _st())
        else:
            rc = xt.lib.eva_k_qkv(xt.ptr(L.a8), xt.ptr(L.as_), L.lds, xt.ptr(wq), xt.ptr(ws), xt.ptr(L.cs), xt.ptr(q),
                                  xt.ptr(k), xt.ptr(vt), M, _st())
        _ok(rc, "qkv")
        outs.append([t.cpu().numpy() for t in (q, k, vt)])
    for name, a, b in zip("q k vt".split(), outs[0], outs[1]):
        _close16(name, a, b, "bf16")


def test_oproj_fc2_sp(dev, xt, layer):
    L, M = layer, layer.M
    for name in ("oproj", "fc2"):
        outs = []
        for sp in (False, True):
            x = L.x0.clone()
            wq, ws, vals, idx = L.w[name]
            w, wx = (vals, idx) if sp else (wq, None)
            if name == "oproj":
                args = (xt.ptr(L.a8), xt.ptr(L.as_), L.lds, xt.ptr(w)) + ((xt.ptr(wx),) if sp else ()) + \
                       (xt.ptr(ws), xt.ptr(x), M, _st())
                rc = (xt.lib.eva_k_oproj_sp if sp else xt.lib.eva_k_oproj)(*args)
            else:
                args = (xt.ptr(L.m8), xt.ptr(L.ms), L.lds, xt.ptr(w)) + ((xt.ptr(wx),) if sp else ()) + \
                       (xt.ptr(ws), xt.ptr(L.stat), xt.ptr(L.cn), xt.ptr(L.dn), xt.ptr(x), M, _st())
                rc = (xt.lib.eva_k_fc2_sp if sp else xt.lib.eva_k_fc2)(*args)
            _ok(rc, name)
            outs.append(x.cpu().numpy())
        _close16(name, outs[0], outs[1], "f16")


def test_fc1_sp(dev, xt, orc, layer):
    L, M = layer, layer.M
    outs = []
    for sp in (False, True):
        m8 = torch.zeros(M, HIDP, dtype=torch.uint8, device=dev)
        ms = torch.zeros(22, L.lds, dtype=torch.float32, device=dev)
        st = torch.zeros(22, L.lds, 2, dtype=torch.float32, device=dev)
        wq, ws, vals, idx = L.w["fc1"]
        if sp:
            rc = xt.lib.eva_k_fc1_sp(xt.ptr(L.a8), xt.ptr(L.as_), L.lds, xt.ptr(vals), xt.ptr(idx), xt.ptr(ws),
                                     xt.ptr(m8), xt.ptr(ms), xt.ptr(st), M, _st())
        else:
            rc = xt.lib.eva_k_fc1(xt.ptr(L.a8), xt.ptr(L.as_), L.lds, xt.ptr(wq), xt.ptr(ws), xt.ptr(m8), xt.ptr(ms),
                                  xt.ptr(st), M, _st())
        _ok(rc, "fc1")
        outs.append((m8.cpu().numpy(), ms.cpu().numpy()[:, :M], st.cpu().numpy()[:, :M]))
    (a8, as_, ast), (b8, bs, bst) = outs
    diff = np.mean(a8 != b8)
    _say(f"  fc1: E4M3 codes differing {diff:.2e}, scales rel {np.abs(bs / as_ - 1).max():.2e}")
    assert diff < 2e-3
    assert np.abs(bs / as_ - 1).max() < 1e-4
    assert np.abs(bst - ast).max() <= 1e-4 * np.abs(ast).max()
