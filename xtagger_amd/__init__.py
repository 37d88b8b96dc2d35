"""xtagger_amd: the wd / EVA02-Large tagger engine of HoloArchivists/xTagger rebuilt for one AMD MI355X (gfx950).

The product is the C-ABI shared library ``libxtag_eva.so`` (declared in ``include/xtag_eva.h``); this package only
loads it and wraps it for Python callers. There is no Python or CPU fallback: importing :mod:`xtagger_amd.lib`
raises if the library has not been built.
"""
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_PATH = os.path.join(PKG_DIR, "libxtag_eva.so")
HEADER_PATH = os.path.join(REPO_DIR, "include", "xtag_eva.h")
