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
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(eva_\w+)\s*\(", src, flags=re.M):
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
