"""The reference's eva02.bin version-2 weight blob (src/tools/export_eva.py:122-153; read by src/engine/eva.h:573-604
and eva.h:380-430 with EVA_VER 2): writer for synthetic random-init EVA02-L weights, and a reader.

Layout: 16-byte header "EVA2", u32 version 2, u32 nt (tags), u32 nbytes, 240 zero bytes, then the tensors, each on
a 256-byte boundary of the blob:
    pe fp16 [1024][592] (c * 196 + ky * 14 + kx, columns 588..591 zero), pos fp32 [1025][1024] (cls and conv bias
    folded), rope fp32 [1024][32][2] (cos, sin per rotary pair), then 24 x [ln1 w, b fp32 [1024], Wqkv fp16
    [3072][1024] (q rows carry log2(e) / sqrt(64)), Wo fp16 [1024][1024], ln2 w, b, W12 fp16 [2 * 2736][1024] (g / x
    interleaved in 16-unit chunks, pad units zero), mlp-LN w, b fp32 [2736], W2 fp16 [1024][2736]], fc_norm w, b,
    head fp16 [ntp][1024], head bias fp32 [ntp] (ntp = nt rounded up to 8).

Synthetic weights (no checkpoint is available offline): block weights N(0, 0.02); LayerNorm gamma 1 + N(0, 0.1),
beta N(0, 0.02); pe and pos N(0, 0.02); head N(0, head_std), bias N(0, 0.1). The rope table follows EVA02's 2-D
rotary embedding as an assumption (the real table lives in the ONNX constants): pair p < 16 rotates with the patch
row, p >= 16 with the column, angle = pos * 16 / 32 * 10000^(-(p % 16) / 16).
"""
import struct

import numpy as np

D, T, NP, K0, K0P, HID, HIDP_V2, NL, NH = 1024, 1025, 1024, 588, 592, 2730, 2736, 24, 16
QSCALE = float(np.log2(np.e)) / 8.0


def rope_table():
    t = np.arange(NP)
    r, c = (t // 32).astype(np.float64), (t % 32).astype(np.float64)
    p = np.arange(32)
    theta = 10000.0 ** (-(p % 16) / 16.0)
    pos = np.where(p[None, :] < 16, r[:, None], c[:, None]) * (16.0 / 32.0)
    ang = pos * theta[None, :]
    return np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32)


def interleave(gx):
    """[g (HIDP rows) | x (HIDP rows)] -> 16-unit chunks [g c | x c] (export_eva.py:60-62)."""
    return gx.reshape(2, HIDP_V2 // 16, 16, -1).transpose(1, 0, 2, 3).reshape(2 * HIDP_V2, -1)


class _Blob:
    def __init__(self):
        self.buf = bytearray()
        self.off = {}

    def put(self, name, a, dt):
        self.buf += b"\0" * (-len(self.buf) % 256)
        self.off[name] = len(self.buf)
        self.buf += np.ascontiguousarray(a, dtype=dt).tobytes()


def synth_model(seed=0, nt=10861, nl=NL, head_std=0.02, layer_scale=1.0, qk_scale=1.0, lead_tags=0, lead=1.0):
    """Random-init EVA02-L tensors in the v2 export layout (fp16 / fp32 numpy arrays).
    layer_scale multiplies the two residual-branch outputs of every block (Wo and W2), as a trained network's layer
    scale keeps its blocks near the identity; qk_scale multiplies the q and k rows of Wqkv (sharper attention);
    lead_tags tags (chosen by the seed) get `lead` added to their bias, so that the top-50 has a margin at rank 50/51
    as a tagger's confident tags do."""
    r = np.random.default_rng(seed)
    f16, f32 = np.float16, np.float32

    def n(shape, std):
        return (r.standard_normal(shape, dtype=np.float32) * std).astype(f32)

    m = {"nt": nt, "nl": nl}
    pe = np.zeros((D, K0P), f32)
    pe[:, :K0] = n((D, K0), 0.02)
    m["pe"] = pe.astype(f16)
    m["pos"] = n((T, D), 0.02)
    m["rope"] = rope_table()
    layers = []
    for _ in range(nl):
        L = {}
        L["ln1w"], L["ln1b"] = 1 + n(D, 0.1), n(D, 0.02)
        wqkv = n((3 * D, D), 0.02)
        wqkv[:2 * D] *= np.float32(qk_scale)
        wqkv[:D] *= QSCALE
        L["wqkv"] = wqkv.astype(f16)
        L["wo"] = (n((D, D), 0.02) * np.float32(layer_scale)).astype(f16)
        L["ln2w"], L["ln2b"] = 1 + n(D, 0.1), n(D, 0.02)
        w12 = np.zeros((2 * HIDP_V2, D), f32)
        w12[:HID] = n((HID, D), 0.02)
        w12[HIDP_V2:HIDP_V2 + HID] = n((HID, D), 0.02)
        L["w12"] = interleave(w12).astype(f16)
        mw, mb = np.zeros(HIDP_V2, f32), np.zeros(HIDP_V2, f32)
        mw[:HID], mb[:HID] = 1 + n(HID, 0.1), n(HID, 0.02)
        L["mlnw"], L["mlnb"] = mw, mb
        w2 = np.zeros((D, HIDP_V2), f32)
        w2[:, :HID] = n((D, HID), 0.02) * np.float32(layer_scale)
        L["w2"] = w2.astype(f16)
        layers.append(L)
    m["layers"] = layers
    m["fnw"], m["fnb"] = 1 + n(D, 0.1), n(D, 0.02)
    ntp = (nt + 7) & ~7
    hw = np.zeros((ntp, D), f32)
    hw[:nt] = n((nt, D), head_std)
    hb = np.zeros(ntp, f32)
    hb[:nt] = n(nt, 0.1)
    if lead_tags:
        hb[r.choice(nt, lead_tags, replace=False)] += np.float32(lead)
    m["hw"], m["hb"] = hw.astype(f16), hb
    return m


def write_v2(path, m):
    """Write model tensors m (synth_model layout, 24 layers) as an eva02.bin v2 file."""
    assert m["nl"] == NL, "the v2 blob always holds 24 layers"
    b = _Blob()
    b.put("pe", m["pe"], np.float16)
    b.put("pos", m["pos"], np.float32)
    b.put("rope", m["rope"], np.float32)
    for i, L in enumerate(m["layers"]):
        b.put(f"ln1w{i}", L["ln1w"], np.float32)
        b.put(f"ln1b{i}", L["ln1b"], np.float32)
        b.put(f"wqkv{i}", L["wqkv"], np.float16)
        b.put(f"wo{i}", L["wo"], np.float16)
        b.put(f"ln2w{i}", L["ln2w"], np.float32)
        b.put(f"ln2b{i}", L["ln2b"], np.float32)
        b.put(f"w12{i}", L["w12"], np.float16)
        b.put(f"mlnw{i}", L["mlnw"], np.float32)
        b.put(f"mlnb{i}", L["mlnb"], np.float32)
        b.put(f"w2{i}", L["w2"], np.float16)
    b.put("fnw", m["fnw"], np.float32)
    b.put("fnb", m["fnb"], np.float32)
    b.put("hw", m["hw"], np.float16)
    b.put("hb", m["hb"], np.float32)
    with open(path, "wb") as f:
        f.write(struct.pack("<4sIII", b"EVA2", 2, m["nt"], len(b.buf)))
        f.write(b"\0" * 240)
        f.write(b.buf)
    return len(b.buf)


def synth_calib(m, seed=0, spread=4.0):
    """Synthetic calibration maxima for write_v3 (the real ones come from the reference's -DEVA_CALIB engine, which
    needs CUDA): per layer the per-channel |max| of the four block-GEMM inputs (LN1 out, attention out, LN2 out over
    1024 channels, the SwiGLU output over 2736 units) and of the rotated q, k and v. Each is a log-uniform draw in
    [1 / spread, spread] times a typical size, with a few outlier channels 20x larger."""
    r = np.random.default_rng(seed)
    nl = len(m["layers"])

    def draw(shape, typ):
        a = typ * np.exp(r.uniform(-np.log(spread), np.log(spread), shape))
        idx = r.choice(shape[-1], 4, replace=False)
        a[..., idx] *= 20.0
        return a.astype(np.float32)
    return {"act": np.stack([np.stack([draw((D,), 4.0), draw((D,), 0.5), draw((D,), 4.0)]) for _ in range(nl)]),
            "h": np.stack([np.concatenate([draw((HID,), 1.0), np.zeros(HIDP_V2 - HID, np.float32)]) for _ in range(nl)]),
            "qkv": np.stack([np.stack([draw((D,), 1.0), draw((D,), 4.0), draw((D,), 2.0)]) for _ in range(nl)])}


def _e4m3_codes(x):
    """RNE to OCP E4M3 of values already clipped to +-448 (the ml_dtypes cast of export_eva.py:66), as bytes"""
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _e4m3_values(q):
    import torch
    return torch.from_numpy(np.ascontiguousarray(q, np.uint8)).view(torch.float8_e4m3fn).to(torch.float32).numpy()


def _smooth(a, w, alpha):
    """SmoothQuant factors of one GEMM (export_eva.py:52-58, export_pixai.py:53-58): per input channel
    clip(amax_act^alpha / amax_wcol^(1 - alpha), 1e-3, 1e3), 1 where either maximum is 0; fp32 as numpy computes them"""
    f32 = np.float32
    wa = np.abs(w).max(0)
    ok = (a > 0) & (wa > 0)
    sm = np.ones_like(a)
    sm[ok] = np.clip(a[ok] ** f32(alpha) / wa[ok] ** f32(1 - alpha), 1e-3, 1e3)
    return sm


def _fp8_tensor(w):
    """E4M3 codes of w with one scale amax / 448 for the whole tensor (export_eva.py:64-66, export_pixai.py:60-62)"""
    f32 = np.float32
    sc = float(np.abs(w).max()) / 448.0
    return _e4m3_codes(np.clip(w / f32(sc), -448.0, 448.0)), f32(sc)


def wd_v3_layer(L, act, h, qkv, alpha=0.5, headroom=1.25):
    """One block of the calibrated export (export_eva.py:96-153) on the v2 tensors L (synth_model's layer layout) and
    the block's calibration maxima (act [3][1024]: LN1 out, attention out, LN2 out; h [2736]: the SwiGLU output; qkv
    [3][1024]: the rotated q, k and v). Returns (w1, b1, [E4M3 Wqkv, Wo, W12, W~2], w2, b2, rs, c, d) and the block's
    table row: SmoothQuant factors s = clip(amax_act^alpha / amax_wcol^(1 - alpha), 1e-3, 1e3) (52-58) folded into the
    producers (LN1 gamma / beta, the Wv rows, LN2 gamma / beta) and the weight columns; the MLP LayerNorm folded into
    fc2 (W~ = W2 diag(gamma) with the h smoothing in its columns, c = W~ 1 from the E4M3 W~, d = W2 beta); every block
    weight E4M3 with one scale amax / 448 (64-66); row = the four weight and four activation dequantization scales
    (max * headroom / 448), then q, k, v's; rs = 1 / (adq_h s~)."""
    f32 = np.float32
    smooth = lambda a, w: _smooth(a, w, alpha)
    row = np.zeros(12, f32)
    w1, b1 = L["ln1w"].astype(f32).copy(), L["ln1b"].astype(f32).copy()
    wqkv = L["wqkv"].astype(f32)
    wo = L["wo"].astype(f32)
    w2, b2 = L["ln2w"].astype(f32).copy(), L["ln2b"].astype(f32).copy()
    w12 = L["w12"].astype(f32)
    mwp, mbp = L["mlnw"].astype(f32), L["mlnb"].astype(f32)
    wf2 = L["w2"].astype(f32)
    dn = wf2 @ mbp
    wf2 = wf2 * mwp[None, :]
    a = [act[0], act[1], act[2], h]
    s = [smooth(a[0], wqkv), smooth(a[1], wo), smooth(a[2], w12), smooth(a[3], wf2)]
    w1 /= s[0]
    b1 /= s[0]
    wqkv *= s[0]
    wqkv[2 * D:] /= s[1][:, None]
    wo *= s[1]
    w2 /= s[2]
    b2 /= s[2]
    w12 *= s[2]
    wf2 *= s[3]
    mats = []
    for k, w in enumerate((wqkv, wo, w12, wf2)):
        q, row[k] = _fp8_tensor(w)
        mats.append(q)
        row[4 + k] = f32(float((a[k] / s[k]).max()) * headroom / 448.0)
    row[8] = f32(float(qkv[0].max()) * headroom / 448.0)
    row[9] = f32(float(qkv[1].max()) * headroom / 448.0)
    row[10] = f32(float((qkv[2] / s[1]).max()) * headroom / 448.0)
    rs = (f32(1.0) / row[7]) / s[3]
    c = (_e4m3_values(mats[3]) * row[3] / s[3]).sum(1).astype(f32)
    return (w1, b1, mats, w2, b2, rs, c, dn.astype(f32)), row


def write_v3(path, m, calib, alpha=0.5, headroom=1.25):
    """Write model tensors m (synth_model layout) as an eva02.bin v3 file: the reference's calibrated export
    (export_eva.py:96-153) restated on the v2 tensors and the calibration maxima calib (synth_calib's layout), one
    block at a time by wd_v3_layer; the [24][12] table of the blocks' rows leads the blob."""
    nl = len(m["layers"])
    assert nl == NL, "the blob always holds 24 layers"
    table = np.zeros((nl, 12), np.float32)
    layers = []
    for i, L in enumerate(m["layers"]):
        ly, table[i] = wd_v3_layer(L, calib["act"][i], calib["h"][i], calib["qkv"][i], alpha, headroom)
        layers.append(ly)
    b = _Blob()
    b.put("table", table, np.float32)
    b.put("pe", m["pe"], np.float16)
    b.put("pos", m["pos"], np.float32)
    b.put("rope", m["rope"], np.float32)
    for i, (w1, b1, mats, w2, b2, rs, c, dn) in enumerate(layers):
        b.put(f"ln1w{i}", w1, np.float32)
        b.put(f"ln1b{i}", b1, np.float32)
        b.put(f"wqkv{i}", mats[0], np.uint8)
        b.put(f"wo{i}", mats[1], np.uint8)
        b.put(f"ln2w{i}", w2, np.float32)
        b.put(f"ln2b{i}", b2, np.float32)
        b.put(f"w12{i}", mats[2], np.uint8)
        b.put(f"rs{i}", rs, np.float32)
        b.put(f"w2{i}", mats[3], np.uint8)
        b.put(f"cn{i}", c, np.float32)
        b.put(f"dn{i}", dn, np.float32)
    b.put("fnw", m["fnw"], np.float32)
    b.put("fnb", m["fnb"], np.float32)
    b.put("hw", m["hw"], np.float16)
    b.put("hb", m["hb"], np.float32)
    with open(path, "wb") as f:
        f.write(struct.pack("<4sIII", b"EVA2", 3, m["nt"], len(b.buf)))
        f.write(b"\0" * 240)
        f.write(b.buf)
    return b


def read_v2(path):
    """Parse an eva02.bin v2 file into the synth_model dictionary layout (arrays view the file bytes)."""
    raw = np.fromfile(path, np.uint8)
    magic, ver, nt, nbytes = struct.unpack("<4sIII", raw[:16].tobytes())
    if magic != b"EVA2" or ver != 2:
        raise ValueError(f"{path} is not an eva02.bin v2")
    blob = raw[256:256 + nbytes]
    if blob.size != nbytes:
        raise ValueError(f"{path} is truncated")
    off = [0]

    def take(shape, dt):
        off[0] = (off[0] + 255) & ~255
        cnt = int(np.prod(shape)) * np.dtype(dt).itemsize
        a = blob[off[0]:off[0] + cnt].view(dt).reshape(shape)
        off[0] += cnt
        return a

    ntp = (nt + 7) & ~7
    m = {"nt": nt, "nl": NL}
    m["pe"] = take((D, K0P), np.float16)
    m["pos"] = take((T, D), np.float32)
    m["rope"] = take((NP, 32, 2), np.float32)
    m["layers"] = []
    for _ in range(NL):
        L = {}
        L["ln1w"], L["ln1b"] = take(D, np.float32), take(D, np.float32)
        L["wqkv"] = take((3 * D, D), np.float16)
        L["wo"] = take((D, D), np.float16)
        L["ln2w"], L["ln2b"] = take(D, np.float32), take(D, np.float32)
        L["w12"] = take((2 * HIDP_V2, D), np.float16)
        L["mlnw"], L["mlnb"] = take(HIDP_V2, np.float32), take(HIDP_V2, np.float32)
        L["w2"] = take((D, HIDP_V2), np.float16)
        m["layers"].append(L)
    m["fnw"], m["fnb"] = take(D, np.float32), take(D, np.float32)
    m["hw"] = take((ntp, D), np.float16)
    m["hb"] = take(ntp, np.float32)
    if off[0] != nbytes:
        raise ValueError(f"{path}: layout mismatch ({off[0]} vs {nbytes} bytes)")
    return m


def synth_smooth_inputs(nb, seed=1):
    """nb patch operands like synth_inputs, from smooth 448^2 images: per channel a base level in [0, 1) plus a
    vertical and a horizontal sinusoid (amplitude < 0.3, under 3 periods), plus N(0, 0.05) pixel noise, clipped to
    [0, 1]. Neighbouring patches see similar content, so the pooled features carry the image rather than the noise."""
    r = np.random.default_rng(seed)
    yy, xx = np.meshgrid(np.linspace(0, 1, 448), np.linspace(0, 1, 448), indexing="ij")
    img = np.empty((nb, 448, 448, 3), np.float32)
    for b in range(nb):
        for c in range(3):
            base = r.random()
            a1, a2 = r.random(2) * 0.3
            f1, f2 = r.random(2) * 3
            img[b, :, :, c] = base + a1 * np.sin(2 * np.pi * f1 * yy) + a2 * np.cos(2 * np.pi * f2 * xx)
    img = np.clip(img + 0.05 * r.standard_normal(img.shape).astype(np.float32), 0, 1)
    bgr = img[..., ::-1] * 2.0 - 1.0
    p = bgr.reshape(nb, 32, 14, 32, 14, 3).transpose(0, 1, 3, 5, 2, 4).reshape(nb, NP, K0)
    out = np.zeros((nb, NP, K0P), np.float16)
    out[:, :, :K0] = p.astype(np.float16)
    return out


def synth_inputs(nb, seed=1):
    """nb patch operands fp16 [1024][592] from 448^2 RGB images with pixels U[0, 1]: BGR scaled to [-1, 1], element
    c * 196 + ky * 14 + kx of patch (py, px), columns 588..591 zero (procimg.h:858-866, 1606-1607)."""
    r = np.random.default_rng(seed)
    img = r.random((nb, 448, 448, 3), dtype=np.float32)
    bgr = img[..., ::-1] * 2.0 - 1.0
    p = bgr.reshape(nb, 32, 14, 32, 14, 3).transpose(0, 1, 3, 5, 2, 4).reshape(nb, NP, K0)
    out = np.zeros((nb, NP, K0P), np.float16)
    out[:, :, :K0] = p.astype(np.float16)
    return out


# ---- PixAI (ViTDet-L) pixai.bin version 2 (src/tools/export_pixai.py:110-152; read by src/engine/px.h:196-253 with
# PX_VER 2): "PXAI", u32 2, u32 nt, u32 nbytes, 240 zero bytes, then every tensor on a 256-byte boundary:
#   pe fp16 [1024][592], pos fp32 [5184][1024], pre-LN w, b fp32 [1024], rope fp32 [576][32][2] (windows) and
#   [5184][32][2] (global), 32 x [ln1 w, b, Wqkv fp16 [3072][1024] (q rows carry log2(e) / 8), bqkv fp32 [3072] (q part
#   likewise), Wo fp16 [1024][1024], bo, ln2 w, b, W1 fp16 [4736][1024], b1 fp32 [4736], rs fp32 [4736] (ones without
#   calibration), W2 fp16 [1024][4736], b2], head LN w, b, U fp32 [16][1024], hpos fp16 [5184][1024], Wv fp16
#   [1024][1024], head fp16 [ntp][1024], head bias fp32 [ntp] (ntp = nt rounded up to 8).
PX_T, PX_LW, PX_HID, PX_NL = 5184, 576, 4736, 32


def synth_px_layer(r, std=0.02):
    f16, f32 = np.float16, np.float32

    def n(shape, s):
        return (r.standard_normal(shape, dtype=np.float32) * s).astype(f32)

    L = {"ln1w": 1 + n(D, 0.1), "ln1b": n(D, 0.02), "ln2w": 1 + n(D, 0.1), "ln2b": n(D, 0.02)}
    wqkv, bqkv = n((3 * D, D), std), n(3 * D, 0.05)
    wqkv[:D] *= QSCALE
    bqkv[:D] *= QSCALE
    L["wqkv"], L["bqkv"] = wqkv.astype(f16), bqkv
    L["wo"], L["bo"] = n((D, D), std).astype(f16), n(D, 0.05)
    L["w1"], L["b1"] = n((PX_HID, D), std).astype(f16), n(PX_HID, 0.05)
    L["rs"] = np.ones(PX_HID, f32)
    L["w2"], L["b2"] = n((D, PX_HID), std).astype(f16), n(D, 0.05)
    return L


def synth_px_model(seed=0, nt=1000, head_std=0.05):
    """Random-init PixAI tensors in the v2 export layout. Rope tables are (cos, sin) of random angles: the kernels
    only need a valid table (the real one lives in the ONNX constants)."""
    r = np.random.default_rng(seed)
    f16, f32 = np.float16, np.float32

    def n(shape, s):
        return (r.standard_normal(shape, dtype=np.float32) * s).astype(f32)

    def rope(rows):
        a = r.random((rows, 32)) * 6.283185307179586
        return np.stack([np.cos(a), np.sin(a)], -1).astype(f32)

    m = {"nt": nt}
    pe = np.zeros((D, K0P), f32)
    pe[:, :K0] = n((D, K0), 0.02)
    m["pe"], m["pos"] = pe.astype(f16), n((PX_T, D), 0.02)
    m["lnpw"], m["lnpb"] = 1 + n(D, 0.1), n(D, 0.02)
    m["csw"], m["csg"] = rope(PX_LW), rope(PX_T)
    m["layers"] = [synth_px_layer(r) for _ in range(PX_NL)]
    m["hnw"], m["hnb"] = 1 + n(D, 0.1), n(D, 0.02)
    m["U"], m["hpos"] = n((16, D), 0.05), n((PX_T, D), 0.02).astype(f16)
    m["wv"] = n((D, D), 0.03).astype(f16)
    ntp = (nt + 7) & ~7
    hw, hb = np.zeros((ntp, D), f32), np.zeros(ntp, f32)
    hw[:nt], hb[:nt] = n((nt, D), head_std), n(nt, 0.1)
    m["hw"], m["hb"] = hw.astype(f16), hb
    return m


def px_tensors(m):
    """(name, array, dtype) in the blob's order."""
    f16, f32 = np.float16, np.float32
    out = [("pe", m["pe"], f16), ("pos", m["pos"], f32), ("lnpw", m["lnpw"], f32), ("lnpb", m["lnpb"], f32),
           ("csw", m["csw"], f32), ("csg", m["csg"], f32)]
    for i, L in enumerate(m["layers"]):
        for k, dt in (("ln1w", f32), ("ln1b", f32), ("wqkv", f16), ("bqkv", f32), ("wo", f16), ("bo", f32),
                      ("ln2w", f32), ("ln2b", f32), ("w1", f16), ("b1", f32), ("rs", f32), ("w2", f16), ("b2", f32)):
            out.append((f"{k}{i}", L[k], dt))
    out += [("hnw", m["hnw"], f32), ("hnb", m["hnb"], f32), ("U", m["U"], f32), ("hpos", m["hpos"], f16),
            ("wv", m["wv"], f16), ("hw", m["hw"], f16), ("hb", m["hb"], f32)]
    return out


def _px_stream(path, ver, nt, tensors):
    """Write (name, array, dtype) tensors as a pixai.bin of version ver, each on a 256-byte boundary of the blob, one
    at a time (a PixAI blob is 0.5 - 0.9 GB); returns each tensor's blob offset and the blob's byte count."""
    off, pos = {}, 0
    with open(path, "wb") as f:
        f.write(struct.pack("<4sIII", b"PXAI", ver, nt, 0))
        f.write(b"\0" * 240)
        for name, a, dt in tensors:
            pad = -pos % 256
            f.write(b"\0" * pad)
            pos += pad
            off[name] = pos
            data = np.ascontiguousarray(a, dtype=dt).tobytes()
            f.write(data)
            pos += len(data)
        f.seek(12)
        f.write(struct.pack("<I", pos))
    return off, pos


def write_px_v2(path, m):
    """Write model tensors m (synth_px_model layout) as a pixai.bin v2 file, streamed tensor by tensor."""
    return _px_stream(path, 2, m["nt"], px_tensors(m))[1]


def synth_px_calib(m, seed=0, spread=4.0):
    """Synthetic calibration maxima for write_px_v3 in the layout of the reference's PixAI calibration file
    (export_pixai.py:35-39, written by px.h's -DPX_CALIB engine, which needs CUDA): per block the per-channel |max| of
    the four block-GEMM inputs (LN1 out, attention out, LN2 out over 1024 channels, the GELU output over 4736 units)
    and of q, k, v. Each is a log-uniform draw in [1 / spread, spread] times a typical size, with a few outlier
    channels 20x larger."""
    r = np.random.default_rng(seed)
    nl = len(m["layers"])

    def draw(n, typ):
        a = typ * np.exp(r.uniform(-np.log(spread), np.log(spread), n))
        a[r.choice(n, 4, replace=False)] *= 20.0
        return a.astype(np.float32)
    return {"act": np.stack([np.stack([draw(D, 4.0), draw(D, 0.5), draw(D, 4.0)]) for _ in range(nl)]),
            "h": np.stack([draw(PX_HID, 1.0) for _ in range(nl)]),
            "qkv": np.stack([np.stack([draw(D, 1.0), draw(D, 4.0), draw(D, 2.0)]) for _ in range(nl)])}


def px_v3_layer(L, act, h, qkv, alpha=0.5, headroom=1.25):
    """One block of the reference's calibrated PixAI export (export_pixai.py:80-99) on the v2 tensors L and the
    block's calibration maxima (act [3][1024], h [4736], qkv [3][1024]): SmoothQuant factors folded into LN1's gamma /
    beta (QKV input), the V rows and bias (out-proj input), LN2's gamma / beta (fc1 input) and the fc2 columns (GELU
    output, whose 1 / s reaches the activations through rs); each block weight E4M3 with one scale amax / 448.
    Returns the block's tensors in blob order and its row of the scale table [wdq x4, adq x4, q, k, v, 0]."""
    f32 = np.float32
    w1, b1 = L["ln1w"].astype(f32).copy(), L["ln1b"].astype(f32).copy()
    wqkv, bqkv = L["wqkv"].astype(f32), L["bqkv"].astype(f32).copy()
    wo, bo = L["wo"].astype(f32), L["bo"].astype(f32)
    w2, b2 = L["ln2w"].astype(f32).copy(), L["ln2b"].astype(f32).copy()
    wf1, bf1 = L["w1"].astype(f32), L["b1"].astype(f32)
    wf2, bf2 = L["w2"].astype(f32), L["b2"].astype(f32)
    a = [act[0], act[1], act[2], h]
    s = [_smooth(a[0], wqkv, alpha), _smooth(a[1], wo, alpha), _smooth(a[2], wf1, alpha), _smooth(a[3], wf2, alpha)]
    w1 /= s[0]
    b1 /= s[0]
    wqkv *= s[0]
    wqkv[2 * D:] /= s[1][:, None]
    bqkv[2 * D:] /= s[1]
    wo *= s[1]
    w2 /= s[2]
    b2 /= s[2]
    wf1 *= s[2]
    wf2 *= s[3]
    row = np.zeros(12, f32)
    mats = []
    for k, w in enumerate((wqkv, wo, wf1, wf2)):
        q, row[k] = _fp8_tensor(w)
        mats.append(q)
        row[4 + k] = f32(float((a[k] / s[k]).max()) * headroom / 448.0)
    row[8] = f32(float(qkv[0].max()) * headroom / 448.0)
    row[9] = f32(float(qkv[1].max()) * headroom / 448.0)
    row[10] = f32(float((qkv[2] / s[1]).max()) * headroom / 448.0)
    rs = (f32(1.0) / row[7]) / s[3]
    u8 = np.uint8
    return [("ln1w", w1, f32), ("ln1b", b1, f32), ("wqkv", mats[0], u8), ("bqkv", bqkv, f32), ("wo", mats[1], u8),
            ("bo", bo, f32), ("ln2w", w2, f32), ("ln2b", b2, f32), ("w1", mats[2], u8), ("b1", bf1, f32),
            ("rs", rs, f32), ("w2", mats[3], u8), ("b2", bf2, f32)], row


def write_px_v3(path, m, calib, alpha=0.5, headroom=1.25):
    """Write model tensors m (synth_px_model layout) as a pixai.bin v3 file: the reference's calibrated export
    (export_pixai.py:68-99 per block by px_v3_layer, 114-132 for the order) with calib in synth_px_calib's layout.
    The [32][12] scale table leads the blob; it is written last, over its placeholder, once every block is done.
    Returns (tensor offsets, blob bytes, table)."""
    nl = len(m["layers"])
    assert nl == PX_NL, "the blob always holds 32 blocks"
    table = np.zeros((nl, 12), np.float32)
    head = px_tensors(m)

    def tensors():
        yield ("table", table, np.float32)
        yield from head[:6]
        for i, L in enumerate(m["layers"]):
            ts, table[i] = px_v3_layer(L, calib["act"][i], calib["h"][i], calib["qkv"][i], alpha, headroom)
            for k, a, dt in ts:
                yield (f"{k}{i}", a, dt)
        yield from head[6 + 13 * nl:]
    off, size = _px_stream(path, 3, m["nt"], tensors())
    with open(path, "r+b") as f:
        f.seek(256)
        f.write(table.tobytes())
    return off, size, table
