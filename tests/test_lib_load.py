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


def test_mx8_launch_plans():
    """the MX8 product's launch plan (host logic, no GPU): a tile of the four
    shapes, a K split only where the tiles leave most of the chip idle, and
    workspace for exactly the split's planes"""
    from pico_amd import kernels as K

    for M, N, Kd in [(4096, 4096, 4096), (8192, 768, 768), (8192, 768, 32000), (768, 768, 8192),
                     (768, 32000, 8192), (1, 1, 1), (300, 257, 70), (2048, 768, 8192)]:
        tm, tn, s = K.mx8_plan(M, N, Kd)
        assert (tm, tn) in ((256, 256), (256, 128), (128, 256), (128, 128))
        assert 1 <= s <= 16
        tiles = -(-M // tm) * -(-N // tn)
        if s > 1:
            assert tiles * s <= 2 * 256 * 2 and tiles < 256
        assert K.mx8_workspace(M, N, Kd) == (s * M * N * 4 if s > 1 else 0)
    assert K.mx8_plan(4096, 4096, 4096)[2] == 1
