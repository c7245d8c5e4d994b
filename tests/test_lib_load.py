"""CPU-only: the built libraries load and export every entry point the public
headers declare (no kernel is launched)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared(header, prefix):
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"\w+)\s*\(", text)))


def test_pico_hip_exports_every_declared_symbol():
    from pico_amd import _lib

    lib = _lib.hip_lib()
    declared = _declared("pico_hip.h", "pk_")
    assert declared, "no pk_ declarations found"
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    # the Python binding table covers the header exactly
    assert sorted(_lib.PK_SIGNATURES) == declared


def test_hip_library_is_gfx950_code():
    from pico_amd import _lib

    blob = open(_lib.HIP_LIB_PATH, "rb").read()
    assert b"gfx950" in blob


def test_missing_library_fails_loudly(monkeypatch):
    from pico_amd import _lib

    monkeypatch.setattr(_lib, "_hip", None)
    monkeypatch.setattr(_lib, "HIP_LIB_PATH", "/nonexistent/libpico_hip.so")
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        _lib.hip_lib()


def test_oracle_library_loads():
    from oracle import oracle as O

    assert hasattr(O.lib(), "ora_matmul_avx")
