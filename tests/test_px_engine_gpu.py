"""The PixAI engine (px_open .. px_close, src/engine/px.h) on synthetic pixai.bin files: its captured forward gives the
same scores, bit for bit, as the px_k_* / eva_k_* kernel sequence of px.h:110-190 run by hand on the same tensors
(each kernel's parity against the oracle is tested on its own), through both the resident-input path and
px_submit / px_wait, for a full batch and a partial one; on the calibrated v3 blob (export_pixai.py with a
calibration file) likewise, and equal to the v2 engine where the two files' quantizations coincide."""
import ctypes as C

import numpy as np
import pytest
import torch

from xtagger_amd import blob
from xtagger_amd.engine import PxEngine

pytestmark = pytest.mark.gpu

D, T5, PH, NT = 1024, 5184, 4736, 500


def _say(*a):
    print(*a, flush=True)


def _chain(xt, m, d_in, nb, dev, layers=None):
    """px_forward (px.h:110-190) by hand: weights packed as the engine packs them, every kernel in the same order.
    layers: the blocks' tensors (default m's v2 blocks); a v3 block (blob.px_v3_layer's tensors with its table row
    under "t") holds E4M3 weights, packed with one scale per tensor: wdq for qkv, out-proj and fc1, wdq3 adq3 for fc2,
    whose input fc1 packs as gelu rs."""
    M, P = nb * T5, xt.ptr
    st = torch.cuda.current_stream().cuda_stream
    keep = []

    def up(a):
        t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        keep.append(t)
        return t

    def z(*s, dt=torch.uint8):
        t = torch.zeros(*s, dtype=dt, device=dev)
        keep.append(t)
        return t

    def pack(w, n_in, k, n_out, perm=0, scale=None):
        q, s = z(n_out, k), z(n_out // 128, k // 128, dt=torch.float32)
        if scale is not None:
            assert w.dtype == np.uint8
            assert xt.lib.eva_k_prep_w8(P(up(w)), k, n_in, k, n_out, k, perm, float(scale), P(q), P(s), st) == 0
        else:
            scratch = torch.empty(n_out * k, dtype=torch.float32, device=dev)
            assert xt.lib.eva_k_prep_w(P(up(w)), k, n_in, k, n_out, k, perm, None, P(scratch), P(q), P(s), st) == 0
        torch.cuda.synchronize()
        return q, s

    x, h8, hs = z(M, D, dt=torch.int16), z(M, D), z(8, M, dt=torch.float32)
    q, k, vt = z(M * D, dt=torch.int16), z(M * D, dt=torch.int16), z(M * D, dt=torch.int16)
    o8, os_, m8, ms = z(M, D), z(8, M, dt=torch.float32), z(M, PH), z(PH // 128, M, dt=torch.float32)
    ok = lambda rc: rc == 0 or pytest.fail("launch failed")
    ok(xt.lib.px_k_pe(P(d_in), P(up(m["pe"])), P(x), M, st))
    ok(xt.lib.px_k_pembed(P(x), P(up(m["pos"])), T5, P(up(m["lnpw"])), P(up(m["lnpb"])), M, st))
    cs = {576: up(m["csw"]), 5184: up(m["csg"])}
    for i, L in enumerate(layers if layers is not None else m["layers"]):
        Ls = 5184 if (i & 7) == 7 else 576
        t = L.get("t", [None] * 8)
        wqkv, sqkv = pack(L["wqkv"], 3 * D, D, 3 * D, 1, t[0])
        wo, so = pack(L["wo"], D, D, D, 0, t[1])
        w1, s1 = pack(L["w1"], PH, D, PH, 0, t[2])
        w2, s2 = pack(L["w2"], D, PH, D, 0, None if t[3] is None else np.float32(t[3] * t[7]))
        ok(xt.lib.eva_k_ln(P(x), P(up(L["ln1w"])), P(up(L["ln1b"])), P(h8), P(hs), M, M, st))
        ok(xt.lib.px_k_qkv(P(h8), P(hs), M, P(wqkv), P(sqkv), P(up(L["bqkv"])), P(cs[Ls]), Ls, P(q), P(k), P(vt), M,
                           st))
        ok(xt.lib.eva_k_flash_seq(P(q), P(k), P(vt), P(o8), P(os_), M, M // Ls, Ls, Ls, None, st))
        ok(xt.lib.px_k_proj(P(o8), P(os_), M, P(wo), P(so), P(up(L["bo"])), P(x), M, st))
        ok(xt.lib.eva_k_ln(P(x), P(up(L["ln2w"])), P(up(L["ln2b"])), P(h8), P(hs), M, M, st))
        ok(xt.lib.px_k_fc1(P(h8), P(hs), M, P(w1), P(s1), P(up(L["b1"])), P(up(L["rs"])), P(m8), P(ms), M, st))
        ok(xt.lib.px_k_fc2(P(m8), P(ms), M, P(w2), P(s2), P(up(L["b2"])), P(x), M, st))
        torch.cuda.synchronize()
    y, s = z(M, D, dt=torch.int16), z(M, 16, dt=torch.float32)
    stat, part = z(nb, T5 // 576, 16, 2, dt=torch.float32), z(nb, T5 // 288, 16, D, dt=torch.float32)
    o, oq, oqs, out = z(nb, D, dt=torch.float32), z(nb, D), z(8, nb, dt=torch.float32), z(nb, NT, dt=torch.float32)
    ldh = (NT + 63) // 64 * 64
    hq, hsc = z(NT, D), z(8, ldh, dt=torch.float32)
    ok(xt.lib.eva_k_quant_act(P(up(m["hw"][:NT])), 2, D, NT, D, P(hq), D, P(hsc), ldh, st))
    ok(xt.lib.px_k_hln(P(x), P(up(m["hnw"])), P(up(m["hnb"])), P(up(m["hpos"])), T5, P(up(m["U"])), P(y), P(s), M, st))
    ok(xt.lib.px_k_hstat(P(s), P(stat), nb, T5, st))
    ok(xt.lib.px_k_hpool(P(s), P(stat), P(y), None, P(part), nb, T5, st))
    ok(xt.lib.px_k_hproj(P(part), T5 // 288, P(up(m["wv"])), P(o), nb, st))
    ok(xt.lib.eva_k_quant_act(P(o), 1, D, nb, D, P(oq), D, P(oqs), nb, st))
    ok(xt.lib.eva_k_head(P(oq), P(oqs), nb, P(hq), P(hsc), ldh, P(up(m["hb"])), P(out), nb, NT, st))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_px_engine_matches_kernel_chain(dev, xt, tmp_path):
    nb = 2
    _say("px engine: synthetic pixai.bin v2")
    m = blob.synth_px_model(seed=5, nt=NT)
    m["layers"][3]["rs"] = (np.random.default_rng(7).random(PH) + 0.5).astype(np.float32)   # one calibrated layer
    path = tmp_path / "pixai.bin"
    blob.write_px_v2(str(path), m)
    r = np.random.default_rng(6)
    inp = np.zeros((nb, T5, 592), np.float16)
    inp[..., :588] = r.uniform(-1, 1, (nb, T5, 588)).astype(np.float16)
    eng = PxEngine(path, nb=nb)
    try:
        eng.ready()
        assert eng.nt == NT and eng.nb == nb
        d_in = torch.from_numpy(inp).to(dev)
        ref = _chain(xt, m, d_in, nb, dev)
        # px_submit / px_wait: host inputs through the pinned staging buffer, a full batch then a partial one
        eng.submit(1, inp)
        sub = eng.wait(1, nb)
        _say("  engine scores: min %.4f max %.4f" % (sub.min(), sub.max()))
        assert np.isfinite(sub).all() and sub.std() > 1e-3
        assert (sub == ref).all(), f"engine differs from the kernel chain: max |d| {np.abs(sub - ref).max():.3g}"
        eng.submit(3, inp[:1])
        assert (eng.wait(3, 1) == ref[:1]).all()
        assert eng.query(3) == 1
        # resident-input path: copy the operands into the engine's device input (a device-to-device hipMemcpy
        # returns before the copy ends: synchronise the device before the replay on the engine's stream)
        hip = C.CDLL("libamdhip64.so")
        assert hip.hipMemcpy(C.c_void_p(eng.dev_input()), C.c_void_p(d_in.data_ptr()), C.c_size_t(inp.nbytes), 3) == 0
        assert hip.hipDeviceSynchronize() == 0
        eng.run()
        eng.sync()
        got = np.empty((nb, NT), np.float32)
        assert hip.hipMemcpy(C.c_void_p(got.ctypes.data), C.c_void_p(eng.dev_output()), C.c_size_t(got.nbytes), 2) == 0
        assert (got == ref).all(), f"resident path differs: max |d| {np.abs(got - ref).max():.3g}"
    finally:
        eng.close()


def test_px_batch_halves(dev, tmp_path):
    """A batch runs as two halves of even size at once (px_open_nb with nb = 6: 4 inputs on the engine stream, 2 on the
    second lane). Full, partial (n = 3: the second lane idle, n = 5: one input on it) and resident batches give every
    image the scores a one-lane nb = 2 engine gives it, bit for bit."""
    m = blob.synth_px_model(seed=8, nt=NT)
    path = tmp_path / "pixai.bin"
    blob.write_px_v2(str(path), m)
    r = np.random.default_rng(12)
    inp = np.zeros((6, T5, 592), np.float16)
    inp[..., :588] = r.uniform(-1, 1, (6, T5, 588)).astype(np.float16)
    _say("px halves: nb = 2 reference engine")
    e2 = PxEngine(path, nb=2)
    try:
        e2.ready()
        ref = []
        for i in range(0, 6, 2):
            e2.submit(0, inp[i:i + 2])
            ref.append(e2.wait(0, 2).copy())
    finally:
        e2.close()
    ref = np.concatenate(ref)
    assert np.isfinite(ref).all() and ref.std() > 1e-3
    _say("px halves: nb = 6 engine (4 + 2)")
    e = PxEngine(path, nb=6)
    try:
        e.ready()
        e.submit(0, inp)
        assert np.array_equal(e.wait(0, 6), ref)
        e.submit(1, inp[3:6])
        assert np.array_equal(e.wait(1, 3), ref[3:6])
        e.submit(2, inp[1:6])
        assert np.array_equal(e.wait(2, 5), ref[1:6])
        hip = C.CDLL("libamdhip64.so")
        d_in = torch.from_numpy(inp).to(dev)
        torch.cuda.synchronize()
        assert hip.hipMemcpy(C.c_void_p(e.dev_input()), C.c_void_p(d_in.data_ptr()), C.c_size_t(inp.nbytes), 3) == 0
        assert hip.hipDeviceSynchronize() == 0
        e.run()
        e.sync()
        out_t = torch.empty((6, e.nt), dtype=torch.float32, device=dev)
        assert hip.hipMemcpy(C.c_void_p(out_t.data_ptr()), C.c_void_p(e.dev_output()), C.c_size_t(out_t.numel() * 4),
                             3) == 0
        assert hip.hipDeviceSynchronize() == 0
        assert np.array_equal(out_t.cpu().numpy(), ref)
    finally:
        e.close()


def _inputs(nb, seed):
    r = np.random.default_rng(seed)
    inp = np.zeros((nb, T5, 592), np.float16)
    inp[..., :588] = r.uniform(-1, 1, (nb, T5, 588)).astype(np.float16)
    return inp


def test_px_v3_engine_matches_kernel_chain(dev, xt, tmp_path):
    """The calibrated blob (export_pixai.py v3: SmoothQuant factors folded into LN1, the V rows, LN2 and the fc2
    columns, per-tensor E4M3 block weights, the [32][12] scale table leading the blob, rs = 1 / (adq3 s3)) read by
    px_open: the same scores, bit for bit, as the kernel chain on the blob's own tensors (blob.px_v3_layer), each
    weight packed by eva_k_prep_w8 with its table scale (fc2: wdq3 adq3) and fc1 run with the blob's rs."""
    nb = 2
    _say("px engine: synthetic pixai.bin v3 (synthetic calibration maxima)")
    m = blob.synth_px_model(seed=5, nt=NT)
    calib = blob.synth_px_calib(m, seed=3)
    path = tmp_path / "pixai_v3.bin"
    _, _, table = blob.write_px_v3(str(path), m, calib)
    layers = []
    for i, L in enumerate(m["layers"]):
        ts, row = blob.px_v3_layer(L, calib["act"][i], calib["h"][i], calib["qkv"][i])
        assert np.array_equal(row, table[i])
        d = {k: a for k, a, _ in ts}
        d["t"] = row
        layers.append(d)
    assert not any((d["rs"] == 1).all() for d in layers)
    inp = _inputs(nb, 6)
    eng = PxEngine(path, nb=nb)
    try:
        eng.ready()
        assert eng.nt == NT
        ref = _chain(xt, m, torch.from_numpy(inp).to(dev), nb, dev, layers)
        eng.submit(0, inp)
        got = eng.wait(0, nb)
        _say("  v3 engine scores: min %.4f max %.4f" % (got.min(), got.max()))
        assert np.isfinite(got).all() and got.std() > 1e-3
        assert (got == ref).all(), f"v3 engine differs from the kernel chain: max |d| {np.abs(got - ref).max():.3g}"
    finally:
        eng.close()


def _pin(w, p):
    """w with the first element of every 128 x 128 block set to +-p (p above every |w|): every block's |max| and the
    tensor's are p, so the block scales of a v2 file and the per-tensor scale of a v3 file are both p / 448"""
    w = w.astype(np.float32)
    assert np.abs(w).max() < p
    w[::128, ::128] = np.where(w[::128, ::128] < 0, -p, p)
    return w.astype(np.float16)


def test_px_v3_equals_v2_where_quantizations_coincide(dev, tmp_path):
    """The v3 engine computes what the v2 engine computes, bit for bit, on a model where the two files' quantizations
    coincide: every 128 x 128 block of every block weight holds the tensor's |max| 1/8 (per-tensor and block scales
    are both 1/8 / 448, so the E4M3 codes are the same), calibration maxima equal to the weight-column maxima (every
    SmoothQuant factor is exactly 1) and a headroom that makes adq3 = 2^-6: fc1 then packs gelu 64 (the same codes
    with block scales 64 times larger, both exact) and fc2's scale wdq3 adq3 brings the product back exactly."""
    m = blob.synth_px_model(seed=8, nt=NT)
    cm = lambda w: np.abs(w.astype(np.float32)).max(0)
    calib = {"act": [], "h": [], "qkv": []}
    for L in m["layers"]:
        for k in ("wqkv", "wo", "w1", "w2"):
            L[k] = _pin(L[k], 0.125)
        calib["act"].append(np.stack([cm(L["wqkv"]), cm(L["wo"]), cm(L["w1"])]))
        calib["h"].append(cm(L["w2"]))
        calib["qkv"].append(np.ones((3, D), np.float32))
    calib = {k: np.asarray(v, np.float32) for k, v in calib.items()}
    p2, p3 = tmp_path / "pixai_v2.bin", tmp_path / "pixai_v3.bin"
    blob.write_px_v2(str(p2), m)
    _, _, table = blob.write_px_v3(str(p3), m, calib, headroom=56.0)
    assert (table[:, :4] == np.float32(0.125 / 448)).all() and (table[:, 7] == 2.0 ** -6).all()
    inp = _inputs(2, 9)
    out = []
    for p in (p2, p3):
        _say(f"px v2 / v3 equality: engine on {p.name}")
        e = PxEngine(p, nb=2)
        try:
            e.ready()
            e.submit(0, inp)
            out.append(e.wait(0, 2).copy())
        finally:
            e.close()
    _say("  v3 vs v2: max |d| %.3g" % np.abs(out[1] - out[0]).max())
    assert np.isfinite(out[0]).all() and out[0].std() > 1e-3
    assert np.array_equal(out[1], out[0])
