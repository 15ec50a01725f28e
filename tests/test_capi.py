"""The C ABI library loads and exports every entry point declared in include/*.h (no GPU call)."""
import ctypes
import glob
import os
import re

from conftest import ROOT, import_pkg


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        txt = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        for m in re.finditer(r"^\s*(?:int|void|long|double)\s+(f16_\w+)\s*\(", txt, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_exports_declared_symbols():
    L = import_pkg("_lib")
    lib = L.lib()
    declared = declared_symbols()
    assert declared, "no declarations found in include/"
    for name in declared:
        assert hasattr(lib, name), name
    assert declared == set(L.exported_symbols()) | (declared - set(L.exported_symbols()))
    for name in L.exported_symbols():
        assert name in declared, f"{name} bound in _lib but not declared in include/"


def test_library_has_gfx950_code_object():
    path = import_pkg("_lib").LIB_PATH
    assert b"gfx950" in open(path, "rb").read()
