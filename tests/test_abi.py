"""CPU checks of the C-ABI library: it loads, and exports every function include/*.h declares (no GPU calls)."""
import ctypes
import glob
import os
import re

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
    """eva.h:580-586: a file that is not an EVA2 v2 blob fails eva_open with -1 (no device call)."""
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
