"""GPU parity at the sizes the benchmark measures.

1. The four fused layer kernels (k_qkv + RoPE, k_oproj + residual, k_fc1 + SwiGLU + E4M3 repack, k_fc2 + folded LN +
   residual), dense and 2:4-sparse, at M = 8200 token rows (batch 8): 396, 132, 726 and 132 tiles of 256 x 256, so
   the partial last row tile, the short single wave of the 1024-column GEMMs and the XCD tile raster all run. Sampled
   rows (every tile-boundary row class, the last rows, a random spread) are checked against the fp64 product of the
   same packed operands through the oracle's epilogues (src/engine/eva_kernels.cu:41-114, 134-162, 211-279, 286-334).
2. The engine at batch 32 and at batch 64 with 2600 extra head rows (13461 in all): each image's scores equal that
   image's batch-1 engine scores bit for bit (the batch-1 forward is the one checked step by step against the oracle
   in test_forward_gpu.py). Rows of a batch are computed independently, so batching may not move a score.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

T, D, TP, HIDP = 1025, 1024, 1088, 2816
NB = 8
M = NB * T
LDS = (M + 255) // 256 * 256


def _say(*a):
    print(*a, flush=True)


def _st():
    return torch.cuda.current_stream().cuda_stream


def _ok(rc, what):
    assert rc == 0, f"{what} returned {rc}"
    torch.cuda.synchronize()


def _rows():
    r = np.random.default_rng(8200)
    fixed = [0, 1, 255, 256, 1024, 1025, 1026, 2049, 4095, 4096, 5125, 7935, 7936, 8191, 8192, 8193, 8198, 8199]
    return np.unique(np.concatenate([fixed, r.choice(M, 46, replace=False)])).astype(np.int32)


def _f16(u):
    return np.asarray(u).view(np.uint16).view(np.float16).astype(np.float64)


def _bf16(u):
    return (np.asarray(u).view(np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def _close(name, got, ref, scale, unit):
    err = np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))
    worst = float((err / (unit * np.abs(ref) + 2e-4 * scale)).max())
    _say(f"  {name}: worst err / bound {worst:.3f}")
    assert worst <= 1.0, name


class Weights:
    """One layer's weights packed on the GPU as the engine's bring-up packs them (eva_k_prep_w), optionally 2:4-pruned
    and packed for the sparse kernels; the oracle's packing of the same fp16 weights (natural row order)."""

    def __init__(self, xt, orc, dev, sparse, seed=5):
        r = np.random.default_rng(seed)
        L, P, st = xt.lib, xt.ptr, _st()
        self.keep = []
        up = lambda a: self._k(torch.from_numpy(np.ascontiguousarray(a)).to(dev))
        z8 = lambda *s: self._k(torch.zeros(*s, dtype=torch.uint8, device=dev))
        zf = lambda *s: self._k(torch.zeros(*s, dtype=torch.float32, device=dev))
        scratch = torch.empty(2 * HIDP * D, dtype=torch.float32, device=dev)
        w12 = np.zeros((2 * HIDP, D), np.float32)
        units = np.arange(2730)
        for half in (0, 1):                                   # g and x rows of the 2730 real units; pads stay zero
            w12[32 * (units // 16) + 16 * half + units % 16] = r.standard_normal((2730, D)) * 0.02
        shapes = {"qkv": (r.standard_normal((3 * D, D)) * 0.02, 1),
                  "oproj": (r.standard_normal((D, D)) * 0.02, 0),
                  "fc1": (w12, 0),
                  "fc2": (np.concatenate([r.standard_normal((D, 2730)) * 0.02, np.zeros((D, 86))], 1), 0)}
        self.dev_w, self.ref = {}, {}
        for name, (w, perm) in shapes.items():
            w16 = w.astype(np.float16)
            n, k = w16.shape
            q, s = z8(n, k), zf(n // 128, k // 128)
            _ok(L.eva_k_prep_w(P(up(w16)), k, n, k, n, k, perm, None, P(scratch), P(q), P(s), st), "prep " + name)
            qw, sw = orc.quant_w(w16.astype(np.float32))
            if sparse:
                _ok(L.eva_k_prune24(P(q), n, k, st), "prune " + name)
                v, x = z8(n // 16, k // 128, 64, 16), self._k(torch.zeros(n // 16, k // 128, 64, dtype=torch.int32,
                                                                          device=dev))
                _ok(L.eva_k_pack24(P(q), n, k, P(v), P(x), None, st), "pack " + name)
                self.dev_w[name] = (v, x, s)
                qw = orc.prune24(qw)
            else:
                self.dev_w[name] = (q, None, s)
            self.ref[name] = (qw, sw)

    def _k(self, t):
        self.keep.append(t)
        return t


@pytest.fixture(scope="module", params=[False, True], ids=["dense", "sparse24"])
def layer_setup(request, dev, xt, orc):
    sparse = request.param
    _say(f"M=8200 layer kernels, {'2:4-sparse' if sparse else 'dense'} weights")
    W = Weights(xt, orc, dev, sparse)
    r = np.random.default_rng(11)
    x = r.standard_normal((M, D)).astype(np.float32)
    qa, sa = orc.quant_act(x)
    sa_l = np.zeros((8, LDS), np.float32)
    sa_l[:, :M] = sa
    return sparse, W, qa, sa, sa_l


def _launch(xt, name, sparse, W, *args):
    L = xt.lib
    w, wx, s = W.dev_w[name]
    P = xt.ptr
    fn = {"qkv": L.eva_k_qkv_sp if sparse else L.eva_k_qkv, "oproj": L.eva_k_oproj_sp if sparse else L.eva_k_oproj,
          "fc1": L.eva_k_fc1_sp if sparse else L.eva_k_fc1, "fc2": L.eva_k_fc2_sp if sparse else L.eva_k_fc2}[name]
    head = args[:3]
    tail = args[3:]
    wargs = (P(w), P(wx), P(s)) if sparse else (P(w), P(s))
    return fn(*head, *wargs, *tail)


def test_qkv_m8200(dev, xt, orc, layer_setup):
    sparse, W, qa, sa, sa_l = layer_setup
    P = xt.ptr
    rows = _rows()
    ang = np.random.default_rng(12).random((1024, 32)) * 6.28
    cs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)
    q = torch.zeros((NB, 16, TP, 64), dtype=torch.int16, device=dev)
    k, vt = torch.zeros_like(q), torch.zeros((NB, 16, 64, TP), dtype=torch.int16, device=dev)
    d_a, d_s, d_cs = (torch.from_numpy(a).to(dev) for a in (qa, sa_l, cs))
    _ok(_launch(xt, "qkv", sparse, W, P(d_a), P(d_s), LDS, P(d_cs), P(q), P(k), P(vt), M, _st()), "qkv")
    qw, sw = W.ref["qkv"]
    acc = np.zeros((M, 3 * D), np.float32)
    acc[rows] = orc.gemm_f64_rows(qa, sa, qw, sw, 3 * D, rows)
    rq, rk, rvt = orc.qkv_epi(acc, NB, cs)
    b, t = rows // T, rows % T
    scale = np.abs(acc[rows]).max()
    for name, got, ref in (("q", q, rq), ("k", k, rk)):
        g = got.cpu().numpy().view(np.uint16)[b, :, t]
        _close(name, _bf16(g), _bf16(ref[b, :, t]), scale, 2.0 ** -7)
    g = vt.cpu().numpy().view(np.uint16)[b, :, :, t]
    _close("vt", _bf16(g), _bf16(rvt[b, :, :, t]), scale, 2.0 ** -7)
    assert (q.cpu().numpy()[:, :, T:] == 0).all() and (vt.cpu().numpy()[..., T:] == 0).all()


def test_oproj_m8200(dev, xt, orc, layer_setup):
    sparse, W, qa, sa, sa_l = layer_setup
    P = xt.ptr
    rows = _rows()
    x = (np.random.default_rng(13).standard_normal((M, D)) * 2).astype(np.float16)
    d_x = torch.from_numpy(x.view(np.int16)).to(dev)
    d_a, d_s = torch.from_numpy(qa).to(dev), torch.from_numpy(sa_l).to(dev)
    _ok(_launch(xt, "oproj", sparse, W, P(d_a), P(d_s), LDS, P(d_x), M, _st()), "oproj")
    qw, sw = W.ref["oproj"]
    acc = orc.gemm_f64_rows(qa, sa, qw, sw, D, rows).astype(np.float32)
    ref = orc.oproj_epi(acc, x.view(np.uint16)[rows])
    got = d_x.cpu().numpy().view(np.uint16)
    _close("x", _f16(got[rows]), _f16(ref), np.abs(acc).max(), 2.0 ** -10)
    other = np.ones(M, bool)
    other[rows] = False
    assert np.isfinite(_f16(got[other])).all()


def test_fc1_m8200(dev, xt, orc, layer_setup):
    sparse, W, qa, sa, sa_l = layer_setup
    P = xt.ptr
    rows = _rows()
    m8 = torch.zeros((M, HIDP), dtype=torch.uint8, device=dev)
    ms = torch.zeros((22, LDS), dtype=torch.float32, device=dev)
    stt = torch.zeros((22, LDS, 2), dtype=torch.float32, device=dev)
    d_a, d_s = torch.from_numpy(qa).to(dev), torch.from_numpy(sa_l).to(dev)
    _ok(_launch(xt, "fc1", sparse, W, P(d_a), P(d_s), LDS, P(m8), P(ms), P(stt), M, _st()), "fc1")
    qw, sw = W.ref["fc1"]
    h, stat = orc.fc1_epi(orc.gemm_f64_rows(qa, sa, qw, sw, 2 * HIDP, rows).astype(np.float32))
    q, s = orc.quant_act(h)
    g_ms = ms.cpu().numpy()[:, rows]
    assert np.abs(g_ms / s - 1).max() < 1e-4
    g8 = m8.cpu().numpy()[rows]
    frac = np.mean(g8 != q)
    _say(f"  E4M3 codes differing: {frac:.2e}")
    assert frac < 2e-3
    dq = orc.e4m3_decode(g8) * np.repeat(g_ms.T, 128, 1)
    assert np.abs(dq - h).max() <= 2.0 ** -3 * np.abs(h).max() + 1e-6
    g_st = stt.cpu().numpy()[:, rows]
    assert np.abs(g_st[..., 0] - stat[..., 0]).max() <= 1e-4 * np.abs(stat[..., 1]).max() ** 0.5 + 1e-5
    assert np.abs(g_st[..., 1] / np.maximum(stat[..., 1], 1e-12) - 1).max() < 1e-4
    assert (m8.cpu().numpy()[:, 2730:] == 0).all()


def test_fc2_m8200(dev, xt, orc, layer_setup):
    sparse, W, _, _, _ = layer_setup
    P = xt.ptr
    rows = _rows()
    r = np.random.default_rng(14)
    h = (r.standard_normal((M, HIDP)) * 0.3 + 0.1).astype(np.float32)
    h[:, 2730:] = 0
    ha, hs = orc.quant_act(h)
    hs_l = np.zeros((22, LDS), np.float32)
    hs_l[:, :M] = hs
    hb = h.astype(np.float64).reshape(M, 22, 128)
    stat = np.zeros((22, LDS, 2), np.float32)
    stat[:, :M, 0], stat[:, :M, 1] = hb.sum(2).T, (hb * hb).sum(2).T
    c = (r.standard_normal(D) * 0.5).astype(np.float32)
    d = (r.standard_normal(D) * 0.1).astype(np.float32)
    x = (r.standard_normal((M, D)) * 2).astype(np.float16)
    d_x = torch.from_numpy(x.view(np.int16)).to(dev)
    dv = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    d_h, d_hs, d_st, d_c, d_d = dv(ha), dv(hs_l), dv(stat), dv(c), dv(d)
    _ok(_launch(xt, "fc2", sparse, W, P(d_h), P(d_hs), LDS, P(d_st), P(d_c), P(d_d), P(d_x), M, _st()), "fc2")
    qw, sw = W.ref["fc2"]
    acc = orc.gemm_f64_rows(ha, hs, qw, sw, D, rows).astype(np.float32)
    st_r = stat[:, rows]
    ref = orc.fc2_epi(acc, st_r, c, d, x.view(np.uint16)[rows])
    S, Q = st_r[..., 0].sum(0), st_r[..., 1].sum(0)
    mean = S / 2730.0
    rstd = 1.0 / np.sqrt(np.maximum(Q / 2730.0 - mean ** 2, 0) + 1e-6)
    _close("x", _f16(d_x.cpu().numpy().view(np.uint16)[rows]), _f16(ref), np.abs(rstd[:, None] * acc).max(),
           2.0 ** -10)


# ---------------------------------------------------------------- the engine at the benchmark's batches
@pytest.fixture(scope="module")
def synth_blob(tmp_path_factory):
    from xtagger_amd import blob
    path = str(tmp_path_factory.mktemp("blob") / "eva02_synth_v2.bin")
    _say("writing synthetic v2 blob")
    blob.write_v2(path, blob.synth_model(seed=0, nt=10861))
    return path


def test_engine_batch32_and_batch64_head13461_match_batch1(dev, synth_blob):
    from xtagger_amd import blob
    from xtagger_amd.engine import Engine
    nt0, extra = 10861, 13461 - 10861
    inp = blob.synth_inputs(64, seed=41)
    _say("engine nb=1 (extra 2600), 64 images one by one")
    e = Engine(synth_blob, device=0, nb=1, extra=extra)
    e.ready()
    single = []
    for i in range(64):
        e.submit(i % 8, inp[i:i + 1])
        single.append(e.wait(i % 8, 1)[0])
    e.close()
    single = np.stack(single)
    assert np.abs(single[:, nt0:] - 1.0 / (1.0 + np.exp(16.0))).max() < 1e-6   # unwritten extra rows never fire
    for nb, ex in ((32, 0), (64, extra)):
        _say(f"engine nb={nb} extra={ex}")
        e = Engine(synth_blob, device=0, nb=nb, extra=ex)
        e.ready()
        e.submit(0, inp[:nb])
        s = e.wait(0, nb)
        e.close()
        ref = single[:nb, :nt0 + ex]
        d = np.abs(s - ref)
        _say(f"  max |batch - single| {d.max():.3g}, bitwise equal rows {int((d.max(1) == 0).sum())}/{nb}, "
             f"differing images {np.flatnonzero(d.max(1) > 0).tolist()}")
        # every kernel computes a row from that row (or that image) alone, in an order that does not depend on where
        # the row sits in its tile: the scores are bit-identical
        assert np.array_equal(s, ref)


def test_sparse_engine_batch32_matches_batch1(dev, synth_blob):
    """The 2:4-sparse engine (EVA_SPARSE24) at the benchmark's batch 32, which runs as two halves of 16 on the engine's
    two lanes: every image's scores equal those of an nb = 1 sparse engine, bit for bit."""
    from xtagger_amd import blob
    from xtagger_amd.engine import Engine
    nb = 32
    inp = blob.synth_inputs(nb, seed=43)
    _say("sparse engine nb=1, 32 images one by one")
    e = Engine(synth_blob, device=0, nb=1, sparse=True)
    e.ready()
    single = []
    for i in range(nb):
        e.submit(i % 8, inp[i:i + 1])
        single.append(e.wait(i % 8, 1)[0])
    e.close()
    single = np.stack(single)
    _say("sparse engine nb=32")
    e = Engine(synth_blob, device=0, nb=nb, sparse=True)
    e.ready()
    e.submit(0, inp)
    s = e.wait(0, nb)
    e.close()
    d = np.abs(s - single)
    _say(f"  max |batch - single| {d.max():.3g}, differing images {np.flatnonzero(d.max(1) > 0).tolist()}")
    assert np.array_equal(s, single)

