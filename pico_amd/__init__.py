"""pico_amd -- MI355X (gfx950) backend for the pico C training API.

The product is native: ``lib/libpico_hip.so`` (hand-written HIP kernels behind
the ``pk_*`` C-ABI of include/pico_hip.h) and ``lib/libpico_amd.so`` (pico's C
API over GPU tensors, include/pico_amd.h).  This package only loads them;
``kernels`` binds the launchers over torch device tensors and ``pico`` binds
the C API.  Nothing here computes on the CPU, and a missing library raises.
"""
from ._lib import HIP_LIB_PATH, AMD_LIB_PATH, PkError, hip_lib  # noqa: F401

__all__ = ["hip_lib", "PkError", "HIP_LIB_PATH", "AMD_LIB_PATH"]
