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


def test_pico_amd_exports_every_declared_function():
    """libpico_amd.so (pico's C API over GPU tensors) exports each function
    include/pico_amd.h declares and keeps its internals hidden.  Loading it
    starts no device work: HIP comes up on the first call that needs it."""
    import subprocess

    from pico_amd.pico import amd_lib

    lib = amd_lib()
    declared = _declared("pico_amd.h", "(?:pico_|arena_)")
    assert len(declared) > 60, declared
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    from pico_amd import _lib

    out = subprocess.run(["nm", "-D", "--defined-only", _lib.AMD_LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert not [s for s in exported if s.startswith("pkh_")]
    assert "x_state" in exported


def test_pico_binding_covers_the_header():
    from pico_amd import pico

    declared = set(_declared("pico_amd.h", "(?:pico_|arena_)"))
    bound = set(pico._SIGS) | set(pico._GPU_SIGS)
    assert bound <= declared, bound - declared


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
