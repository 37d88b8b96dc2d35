"""CPU checks of the C-ABI library: it loads, and exports every function include/*.h declares (no GPU calls)."""
import ctypes
import glob
import os
import re

import numpy as np

from xtagger_amd import LIB_PATH, REPO_DIR


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(REPO_DIR, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b((?:eva|px)_\w+)\s*\(", src, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    assert os.path.exists(LIB_PATH), "libxtag_eva.so not built"
    lib = ctypes.CDLL(LIB_PATH)
    names = declared_functions()
    assert len(names) >= 4
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_bad_shapes_rejected_without_gpu():
    from xtagger_amd import lib as L
    # argument checks run before any HIP call: K not a multiple of 128
    assert L.lib.eva_k_gemm(None, 100, None, 1, None, None, 1, 128, 100, None, 128, 0, None) == -1
    assert L.lib.eva_k_quant_act(None, 0, 100, 1, 100, None, 100, None, 1, None) == -1
    assert L.lib.eva_k_quant_w(None, 128, 100, None, None, None) == -1


def test_px_bad_shapes_rejected_without_gpu():
    """The PixAI block kernels check rows, L and lds before any HIP call (rows not a multiple of L, L not a multiple
    of 64, lds < rows, rows past 2^19)."""
    from xtagger_amd import lib as L
    n = None
    assert L.lib.px_k_qkv(n, n, 1152, n, n, n, n, 576, n, n, n, 1000, n) == -1
    assert L.lib.px_k_qkv(n, n, 1152, n, n, n, n, 96, n, n, n, 1152, n) == -1
    assert L.lib.px_k_proj(n, n, 10, n, n, n, n, 64, n) == -1
    assert L.lib.px_k_fc1(n, n, 10, n, n, n, n, n, n, 64, n) == -1
    assert L.lib.px_k_fc2(n, n, 1 << 20, n, n, n, n, (1 << 19) + 1, n) == -1


def test_open_rejects_bad_header(tmp_path):
    """eva.h:580-586: a file that is not an EVA2 v2 or v3 blob, or a v3 blob whose scale table is cut short, fails
    eva_open with -1 (no device call)."""
    from xtagger_amd.engine import Engine
    p = tmp_path / "bad.bin"
    p.write_bytes(b"NOPE" + b"\0" * 300)
    import pytest
    with pytest.raises(RuntimeError):
        Engine(str(p))
    import struct
    p.write_bytes(struct.pack("<4sIII", b"EVA2", 3, 10861, 100) + b"\0" * 300)
    with pytest.raises(RuntimeError):
        Engine(str(p))
    with pytest.raises(RuntimeError):
        Engine(str(tmp_path / "missing.bin"))


def test_px_open_rejects_bad_files(tmp_path):
    """px.h:357-372: a file that is not a pixai.bin v2 or v3 (another magic or version, no tags), a v3 file whose scale
    table is cut short or holds a scale that is not positive and finite, or an odd batch, fails px_open with -1 (no
    device call)."""
    import struct
    import pytest
    from xtagger_amd.engine import PxEngine
    p = tmp_path / "bad.bin"
    tab = np.full((32, 12), 0.01, np.float32)
    tab[5, 3] = 0.0
    bad_tab = struct.pack("<4sIII", b"PXAI", 3, 100, 0) + b"\0" * 240 + tab.tobytes()
    for data in (b"NOPE" + b"\0" * 312, struct.pack("<4sIII", b"PXAI", 4, 100, 0) + b"\0" * 300,
                 struct.pack("<4sIII", b"PXAI", 3, 100, 0) + b"\0" * 300,
                 struct.pack("<4sIII", b"PXAI", 2, 0, 0) + b"\0" * 300, bad_tab):
        p.write_bytes(data)
        with pytest.raises(RuntimeError):
            PxEngine(str(p))
    p.write_bytes(struct.pack("<4sIII", b"PXAI", 2, 10, 0) + b"\0" * 300)
    with pytest.raises(RuntimeError):
        PxEngine(str(p), nb=3)
    with pytest.raises(RuntimeError):
        PxEngine(str(tmp_path / "missing.bin"))


def _px_walk(ver, ntp):
    """Byte offsets of the PixAI blob's tensors as the reference's reader takes them (px.h:196-253 px_layout: EVA_TAKE
    rounds every offset up to 256; v3, PX_WB 1, leads with the [32][12] fp32 table and holds the four block weights as
    E4M3 bytes), restated from that walk, independently of the writer."""
    D, T, LW, HID, K0P, NL = 1024, 5184, 576, 4736, 592, 32
    wb = 1 if ver == 3 else 2
    sizes = ([("table", NL * 12 * 4)] if ver == 3 else []) + [
        ("pe", D * K0P * 2), ("pos", T * D * 4), ("lnpw", D * 4), ("lnpb", D * 4), ("csw", LW * 32 * 2 * 4),
        ("csg", T * 32 * 2 * 4)]
    for i in range(NL):
        sizes += [(f"ln1w{i}", D * 4), (f"ln1b{i}", D * 4), (f"wqkv{i}", 3 * D * D * wb), (f"bqkv{i}", 3 * D * 4),
                  (f"wo{i}", D * D * wb), (f"bo{i}", D * 4), (f"ln2w{i}", D * 4), (f"ln2b{i}", D * 4),
                  (f"w1{i}", HID * D * wb), (f"b1{i}", HID * 4), (f"rs{i}", HID * 4), (f"w2{i}", D * HID * wb),
                  (f"b2{i}", D * 4)]
    sizes += [("hnw", D * 4), ("hnb", D * 4), ("U", 16 * D * 4), ("hpos", T * D * 2), ("wv", D * D * 2),
              ("hw", ntp * D * 2), ("hb", ntp * 4)]
    off, out = 0, {}
    for name, n in sizes:
        off = (off + 255) & ~255
        out[name] = off
        off += n
    return out, off


def test_px_blob_layouts_match_the_reference_walk(tmp_path):
    """blob.write_px_v2's and blob.write_px_v3's tensors sit where px.h's px_layout takes them and the header's byte
    count is the walk's end (the engine checks the same count, px.h:247-250); the v3 file's scale table is at the
    blob's start and a weight's E4M3 bytes at the walk's offset."""
    import struct
    from xtagger_amd import blob
    m = _fake_px_model(13, fill=0.01)
    want2, end2 = _px_walk(2, 16)
    assert blob._px_stream(os.devnull, 2, 13, blob.px_tensors(m)) == (want2, end2)
    p3 = str(tmp_path / "v3.bin")
    calib = blob.synth_px_calib(m, seed=1)
    off3, n3, table = blob.write_px_v3(p3, m, calib)
    want3, end3 = _px_walk(3, 16)
    assert (off3, n3) == (want3, end3)
    with open(p3, "rb") as f:
        assert struct.unpack("<4sIII", f.read(16)) == (b"PXAI", 3, 13, end3)
        f.seek(256)
        assert np.array_equal(np.frombuffer(f.read(table.nbytes), np.float32).reshape(32, 12), table)
        f.seek(256 + want3["w27"])
        ts, _ = blob.px_v3_layer(m["layers"][7], calib["act"][7], calib["h"][7], calib["qkv"][7])
        assert np.array_equal(np.frombuffer(f.read(1024 * 4736), np.uint8), dict((k, a) for k, a, _ in ts)["w2"].ravel())


def test_px_v3_layer_keeps_every_gemm():
    """blob.px_v3_layer restates one block of the calibrated export (export_pixai.py:80-99). SmoothQuant moves a
    factor from each GEMM's input to its weight columns, so every GEMM of the block must compute what the v2 block
    computes, up to the E4M3 rounding of its weights (one scale per tensor): for normalised rows xh, attention-like rows
    z and GELU-like outputs g, LN1'(xh) W~qkv^T wdq0 equals LN1(xh) Wqkv^T on the q and k rows; the v rows, which
    carry 1 / s1, through W~o wdq1 give the v2 block's v Wo^T; LN2'(xh) W~1^T wdq2 equals LN2(xh) W1^T; and
    (g rs) (W~2 wdq3 adq3)^T equals g W2^T. Calibration maxima spread 16x with 20x outliers make the factors far from
    1: a fold left out (the V rows' 1 / s1, rs without 1 / s3) moves a GEMM by 60% or more, the rounding by under 5%.
    Every weight's largest code is 448 (scale = amax / 448)."""
    from xtagger_amd import blob
    r = np.random.default_rng(4)
    L = blob.synth_px_layer(r)
    c = blob.synth_px_calib({"layers": [L]}, seed=2, spread=16.0)
    ts, t = blob.px_v3_layer(L, c["act"][0], c["h"][0], c["qkv"][0])
    V = {k: a for k, a, _ in ts}
    f = lambda a: np.asarray(a, np.float64)
    dec = lambda k: blob._e4m3_values(V[k]).astype(np.float64)
    rel = lambda a, b: np.linalg.norm(a - b) / np.linalg.norm(b)
    for k in ("wqkv", "wo", "w1", "w2"):
        assert V[k].dtype == np.uint8 and np.abs(dec(k)).max() == 448.0
    xh, z, g = r.standard_normal((64, 1024)), r.standard_normal((64, 1024)), np.abs(r.standard_normal((64, 4736)))
    y2 = (xh * f(L["ln1w"]) + f(L["ln1b"])) @ f(L["wqkv"]).T
    y3 = (xh * f(V["ln1w"]) + f(V["ln1b"])) @ (dec("wqkv") * t[0]).T
    assert rel(y3[:, :2048], y2[:, :2048]) < 0.05
    o2 = y2[:, 2048:] @ f(L["wo"]).T
    assert rel(y3[:, 2048:] @ (dec("wo") * t[1]).T, o2) < 0.05
    assert rel(y3[:, 2048:] @ f(L["wo"]).T, o2) > 0.5                  # V rows left unfolded
    u2 = (xh * f(L["ln2w"]) + f(L["ln2b"])) @ f(L["w1"]).T
    assert rel((xh * f(V["ln2w"]) + f(V["ln2b"])) @ (dec("w1") * t[2]).T, u2) < 0.05
    p2 = g @ f(L["w2"]).T
    w2 = dec("w2") * (np.float64(t[3]) * t[7])
    assert rel((g * f(V["rs"])) @ w2.T, p2) < 0.05
    assert rel((g / t[7]) @ w2.T, p2) > 0.5                              # rs without 1 / s3
    assert rel(z @ (dec("wo") * t[1]).T, z @ f(L["wo"]).T) > 0.5         # the out-proj columns carry s1


def test_wd_v3_layer_keeps_every_gemm():
    """blob.wd_v3_layer restates one block of the calibrated wd export (export_eva.py:96-153): every GEMM of the v3
    block must compute what the v2 block computes, up to the E4M3 rounding of its weights. For normalised rows xh:
    LN1'(xh) W~qkv^T wdq0 equals LN1(xh) Wqkv^T on the q and k rows; the v rows, which carry 1 / s1, through W~o wdq1
    give the v2 block's v Wo^T; LN2'(xh) W~12^T wdq2 equals LN2(xh) W12^T. The MLP LayerNorm is folded into fc2: for
    SwiGLU-like rows g with mean mu and 1 / std r over the 2730 units, r ((g rs) (W~2 wdq3 adq3)^T - mu c) + d equals
    LNm(g) W2^T. g has mean 1 and the MLP LayerNorm bias is made large, so that the c and d terms each carry a
    visible share; calibration maxima spread 16x with 20x outliers make the smoothing factors far from 1. A fold left
    out (the V rows' 1 / s1, rs without 1 / s3, c or d) moves a GEMM by 50% or more, the rounding by under 5%."""
    from xtagger_amd import blob
    r = np.random.default_rng(4)
    m = blob.synth_model(seed=7, nt=8, nl=1)
    L = dict(m["layers"][0])
    L["mlnb"] = L["mlnb"] * np.float32(50.0)
    c = blob.synth_calib(m, seed=2, spread=16.0)
    (w1, b1, mats, w2, b2, rs, cn, dn), t = blob.wd_v3_layer(L, c["act"][0], c["h"][0], c["qkv"][0])
    f = lambda a: np.asarray(a, np.float64)
    dec = lambda q: blob._e4m3_values(q).astype(np.float64)
    rel = lambda a, b: np.linalg.norm(a - b) / np.linalg.norm(b)
    for q in mats:
        assert q.dtype == np.uint8 and np.abs(dec(q)).max() == 448.0
    D, HID, HP = 1024, 2730, 2736
    xh = r.standard_normal((64, D))
    y2 = (xh * f(L["ln1w"]) + f(L["ln1b"])) @ f(L["wqkv"]).T
    y3 = (xh * f(w1) + f(b1)) @ (dec(mats[0]) * t[0]).T
    assert rel(y3[:, :2 * D], y2[:, :2 * D]) < 0.05
    o2 = y2[:, 2 * D:] @ f(L["wo"]).T
    assert rel(y3[:, 2 * D:] @ (dec(mats[1]) * t[1]).T, o2) < 0.05
    assert rel(y3[:, 2 * D:] @ f(L["wo"]).T, o2) > 0.5                  # V rows left unfolded
    u2 = (xh * f(L["ln2w"]) + f(L["ln2b"])) @ f(L["w12"]).T
    assert rel((xh * f(w2) + f(b2)) @ (dec(mats[2]) * t[2]).T, u2) < 0.05
    g = np.zeros((64, HP))
    g[:, :HID] = r.standard_normal((64, HID)) * np.abs(r.standard_normal(HID)) + 1.0
    mu = g[:, :HID].mean(1, keepdims=True)
    rstd = 1 / np.sqrt(g[:, :HID].var(1, keepdims=True) + 1e-6)
    gn = np.zeros_like(g)
    gn[:, :HID] = (g[:, :HID] - mu) * rstd
    p2 = (gn * f(L["mlnw"]) + f(L["mlnb"])) @ f(L["w2"]).T
    W = dec(mats[3]) * (np.float64(t[3]) * t[7])
    assert rel(rstd * ((g * f(rs)) @ W.T - mu * f(cn)) + f(dn), p2) < 0.05
    assert rel(rstd * ((g / t[7]) @ W.T - mu * f(cn)) + f(dn), p2) > 0.5   # rs without 1 / s3
    assert rel(rstd * ((g * f(rs)) @ W.T) + f(dn), p2) > 0.5               # c left out
    assert rel(rstd * ((g * f(rs)) @ W.T - mu * f(cn)), p2) > 0.5          # d left out


def _fake_px_model(nt, fill=0.0):
    """Constant tensors of the v2 shapes (cheap: broadcast views)."""
    f16, f32 = np.float16, np.float32
    z = lambda shape, dt: np.broadcast_to(np.full(1, fill, dt), shape)
    L = {"ln1w": z(1024, f32), "ln1b": z(1024, f32), "wqkv": z((3072, 1024), f16), "bqkv": z(3072, f32),
         "wo": z((1024, 1024), f16), "bo": z(1024, f32), "ln2w": z(1024, f32), "ln2b": z(1024, f32),
         "w1": z((4736, 1024), f16), "b1": z(4736, f32), "rs": z(4736, f32), "w2": z((1024, 4736), f16),
         "b2": z(1024, f32)}
    ntp = (nt + 7) & ~7
    return {"nt": nt, "pe": z((1024, 592), f16), "pos": z((5184, 1024), f32), "lnpw": z(1024, f32),
            "lnpb": z(1024, f32), "csw": z((576, 32, 2), f32), "csg": z((5184, 32, 2), f32), "layers": [L] * 32,
            "hnw": z(1024, f32), "hnb": z(1024, f32), "U": z((16, 1024), f32), "hpos": z((5184, 1024), f16),
            "wv": z((1024, 1024), f16), "hw": z((ntp, 1024), f16), "hb": z(ntp, f32)}


def test_blob_roundtrip_small(tmp_path):
    """The v2 writer / reader agree and the byte layout is the one eva.h walks (256-byte aligned tensors)."""
    from xtagger_amd import blob
    import numpy as np
    m = blob.synth_model(seed=1, nt=17, nl=24, head_std=0.02)
    n = blob.write_v2(str(tmp_path / "b.bin"), m)
    r = blob.read_v2(str(tmp_path / "b.bin"))
    assert r["nt"] == 17 and r["hw"].shape == (24, 1024)
    assert np.array_equal(r["layers"][5]["w2"], m["layers"][5]["w2"])
    assert np.array_equal(r["rope"], m["rope"])
    raw = open(tmp_path / "b.bin", "rb").read()
    assert raw[:4] == b"EVA2" and len(raw) == 256 + n


def test_c_program_against_header(tmp_path):
    """tests/abi_check.c, compiled by gcc against include/xtag_eva.h alone and linked to libxtag_eva.so: struct layout,
    rejected files and arguments (-1 with the eva: message), a failed open that eva_close accepts."""
    import subprocess
    exe = str(tmp_path / "abi_check")
    libdir = os.path.dirname(LIB_PATH)
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(REPO_DIR, "include"),
                    os.path.join(REPO_DIR, "tests", "abi_check.c"), "-o", exe, "-L", libdir, "-l:libxtag_eva.so",
                    "-Wl,-rpath," + libdir], check=True)
    r = subprocess.run([exe, str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "abi ok" in r.stdout, r.stdout + r.stderr
    assert "eva: " in r.stderr                                  # the reference's error convention


def _eva_walk(ver, ntp):
    """Byte offsets of the wd blob's tensors as the reference's reader takes them (eva.h:380-428 eva_layout: EVA_TAKE
    rounds every offset up to 256; v3 leads with the [24][12] fp32 table and stores E4M3 weights with rs | W~2 | c | d
    in place of the MLP LN's gamma | beta | W2), restated from that walk, independently of the writer."""
    D, T, NP, K0P, HIDP, NL = 1024, 1025, 1024, 592, 2736, 24
    wb = 1 if ver == 3 else 2
    sizes = ([("table", NL * 12 * 4)] if ver == 3 else []) + [("pe", D * K0P * 2), ("pos", T * D * 4),
                                                           ("rope", NP * 32 * 2 * 4)]
    for i in range(NL):
        sizes += [(f"ln1w{i}", D * 4), (f"ln1b{i}", D * 4), (f"wqkv{i}", 3 * D * D * wb), (f"wo{i}", D * D * wb),
                  (f"ln2w{i}", D * 4), (f"ln2b{i}", D * 4), (f"w12{i}", 2 * HIDP * D * wb)]
        if ver == 3:
            sizes += [(f"rs{i}", HIDP * 4), (f"w2{i}", D * HIDP), (f"cn{i}", D * 4), (f"dn{i}", D * 4)]
        else:
            sizes += [(f"mlnw{i}", HIDP * 4), (f"mlnb{i}", HIDP * 4), (f"w2{i}", D * HIDP * 2)]
    sizes += [("fnw", D * 4), ("fnb", D * 4), ("hw", ntp * D * 2), ("hb", ntp * 4)]
    off, out = 0, {}
    for name, n in sizes:
        off = (off + 255) & ~255
        out[name] = off
        off += n
    return out, off


def test_wd_blob_layouts_match_the_reference_walk(tmp_path):
    """blob.write_v2 and blob.write_v3 put every tensor where eva.h's eva_layout takes it, and the header's byte count
    is the walk's end (the engine checks the same count, eva.h:424-427)."""
    import struct
    from xtagger_amd import blob
    m = blob.synth_model(seed=3, nt=13)
    p2 = str(tmp_path / "v2.bin")
    nbytes = blob.write_v2(p2, m)
    want, end = _eva_walk(2, 16)
    assert nbytes == end
    with open(p2, "rb") as f:
        assert struct.unpack("<4sIII", f.read(16)) == (b"EVA2", 2, 13, end)
    b3 = blob.write_v3(str(tmp_path / "v3.bin"), m, blob.synth_calib(m, seed=1))
    want3, end3 = _eva_walk(3, 16)
    assert len(b3.buf) == end3 and b3.off == want3
    with open(str(tmp_path / "v3.bin"), "rb") as f:
        assert struct.unpack("<4sIII", f.read(16)) == (b"EVA2", 3, 13, end3)
    # every v2 tensor's bytes sit at the walk's offset
    raw = np.fromfile(p2, np.uint8)[256:]
    f16, f32 = np.float16, np.float32
    exp = {"pe": (m["pe"], f16), "pos": (m["pos"], f32), "rope": (m["rope"], f32), "fnw": (m["fnw"], f32),
           "fnb": (m["fnb"], f32), "hw": (m["hw"], f16), "hb": (m["hb"], f32)}
    for i, L in enumerate(m["layers"]):
        for k, dt in (("ln1w", f32), ("ln1b", f32), ("wqkv", f16), ("wo", f16), ("ln2w", f32), ("ln2b", f32),
                      ("w12", f16), ("mlnw", f32), ("mlnb", f32), ("w2", f16)):
            exp[f"{k}{i}"] = (L[k], dt)
    assert set(exp) == set(want)
    for name, (a, dt) in exp.items():
        bts = np.ascontiguousarray(a, dt).view(np.uint8).reshape(-1)
        assert np.array_equal(raw[want[name]:want[name] + bts.size], bts), name

