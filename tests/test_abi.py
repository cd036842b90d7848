"""The C ABI library loads and exports every symbol include/thrml_hip.h
declares (no GPU needed: nothing here launches a kernel)."""
import ctypes
import os
import re

import thrml_hip
from thrml_hip import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    src = open(os.path.join(ROOT, "include", "thrml_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(thrml_[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = _declared()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    bound = {n for n, _, _ in _lib.SIGNATURES}
    assert set(_declared()) <= bound, set(_declared()) - bound


def test_host_only_entry_points_and_errors():
    lib = _lib.load()
    assert lib.thrml_version() >= 100
    # invalid arguments fail with a message and no GPU access
    rc = lib.thrml_lattice_edges(0, 1, None, None)
    assert rc == _lib.THRML_EINVAL and b"positive" in lib.thrml_last_error()
    rc = lib.thrml_erdos_renyi(10, 1.5, 1, None, None, 0)
    assert rc == _lib.THRML_EINVAL
    assert thrml_hip.RngKey(5).split(1)[0] == thrml_hip.RngKey(5)
