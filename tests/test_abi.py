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


def test_fast_math_bounds_predicate():
    """The verdict the library applies to its cached self-check before it
    creates a program: Gumbel error <= 4e-6 (the categorical kernels'
    margin), and exp + sigmoid relative errors + 2^-23 below the spin band
    2^-16.  A device outside either bound gets no program."""
    lib = _lib.load()

    def ok(g, e, s):
        v = (ctypes.c_float * 3)(g, e, s)
        return bool(lib.thrml_fast_math_bounds_ok(v))

    assert ok(0.0, 0.0, 0.0)
    assert ok(4e-6, 2.0**-18, 2.0**-18)          # measured values sit near 1.9e-6, 2^-22
    assert not ok(4.01e-6, 0.0, 0.0)               # Gumbel margin exceeded
    assert ok(0.0, 2.0**-17, 2.0**-18)             # 0.75 band + 2^-23 < band
    assert not ok(0.0, 2.0**-17, 2.0**-17)         # band + 2^-23 is not below the band
    assert not ok(0.0, 2.0**-16 - 2.0**-23, 0.0)  # equality fails: the bound is strict
    assert not lib.thrml_fast_math_bounds_ok(None)
