"""Loader for the in-tree native libraries of the MI355X backend.

``libpico_hip.so`` holds the hand-written gfx950 kernels behind the ``pk_*``
C-ABI (include/pico_hip.h); ``libpico_amd.so`` holds pico's C API over GPU
tensors (include/pico_amd.h).  Both are built in-tree by ``pico_amd/Makefile``.

torch is imported first on purpose: its wheel ships its own HIP runtime with
the same soname as /opt/rocm's, and loading torch first makes our libraries
bind to that one runtime instead of pulling in a second copy.

There is no fallback: if a library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (see module docstring: must precede the CDLL loads)

HERE = os.path.dirname(os.path.abspath(__file__))
LIBDIR = os.path.join(HERE, "lib")
HIP_LIB_PATH = os.path.join(LIBDIR, "libpico_hip.so")
AMD_LIB_PATH = os.path.join(LIBDIR, "libpico_amd.so")

c_i64 = ctypes.c_int64
c_f = ctypes.c_float
c_p = ctypes.c_void_p
c_int = ctypes.c_int
c_char = ctypes.c_char
c_size = ctypes.c_size_t

# name -> argument types (all return int status unless listed in _RESTYPES)
PK_SIGNATURES = {
    "pk_device_info": [ctypes.POINTER(c_int), ctypes.POINTER(c_int), ctypes.c_char_p, c_int],
    "pk_gemm_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64, c_f, c_p,
                    c_i64, c_p],
    "pk_gemm_workspace_f32": [c_i64, c_i64, c_i64],
    "pk_gemm_ex_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64, c_f, c_p,
                       c_i64, c_p, c_size, c_p],
    "pk_gemm_noalloc_scratch_bytes": [],
    "pk_gemm_noalloc_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64,
                            c_f, c_p, c_i64, c_p],
    "pk_gemm_fp8_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64, c_f,
                        c_p, c_i64, c_p],
    "pk_gemm_ex_fp8_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64,
                           c_f, c_p, c_i64, c_p, c_size, c_p],
    "pk_gemm_small_product_f32": [c_i64, c_i64, c_i64],
    "pk_gemm_add_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64, c_f,
                        c_p, c_i64, c_p, c_i64, c_int, c_p, c_p, c_size, c_p],
    "pk_gemm_swiglu_bwd_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64,
                               c_p, c_i64, c_p, c_i64, c_p, c_p, c_i64, c_int, c_int, c_p, c_p],
    "pk_gemm_swiglu_fwd_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64,
                               c_p, c_i64, c_p, c_i64, c_int, c_p, c_p],
    "pk_fp8_scales_f32": [c_i64, c_i64, c_p, c_i64, c_i64, c_i64, c_p, c_i64, c_p, c_p],
    "pk_fp8_quantized_bytes": [c_i64, c_i64, ctypes.POINTER(c_i64)],
    "pk_fp8_quantize_f32": [c_i64, c_i64, c_p, c_i64, c_int, c_p, c_p, c_i64, c_p],
    "pk_gemm_fp8q_f32": [c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64, c_p, c_f, c_p, c_i64,
                         c_p],
    "pk_mx8_bytes": [c_i64, c_i64],
    "pk_mx8_quantize_f32": [c_i64, c_i64, c_p, c_i64, c_int, c_p, c_p],
    "pk_gemm_mx8_f32": [c_i64, c_i64, c_i64, c_f, c_p, c_p, c_f, c_p, c_i64, c_p, c_i64, c_p],
    "pk_gemm_mx8_workspace": [c_i64, c_i64, c_i64],
    "pk_mx8_quantize2_f32": [c_i64, c_i64, c_p, c_i64, c_p, c_p, c_p],
    "pk_bf16q_bytes": [c_i64, c_i64],
    "pk_bf16q_quantize_f32": [c_i64, c_i64, c_p, c_i64, c_int, c_p, c_p],
    "pk_bf16q_quantize2_f32": [c_i64, c_i64, c_p, c_i64, c_p, c_p, c_p],
    "pk_gemm_bf16q_workspace": [c_i64, c_i64, c_i64],
    "pk_gemm_bf16q_f32": [c_i64, c_i64, c_i64, c_f, c_p, c_p, c_f, c_p, c_i64, c_p, c_i64, c_p],
    "pk_gemm_bf16q_ex_f32": [c_i64, c_i64, c_i64, c_f, c_p, c_p, c_f, c_p, c_i64, c_p, c_i64, c_p,
                             c_size, c_p],
    "pk_bf16x3q_bytes": [c_i64, c_i64],
    "pk_bf16x3q_quantize_f32": [c_i64, c_i64, c_p, c_i64, c_int, c_p, c_p],
    "pk_gemm_bf16x3q_workspace": [c_i64, c_i64, c_i64],
    "pk_gemm_bf16x3q_f32": [c_i64, c_i64, c_i64, c_f, c_p, c_p, c_f, c_p, c_i64, c_p, c_i64, c_p],
    "pk_gemm_bf16x3q_ex_f32": [c_i64, c_i64, c_i64, c_f, c_p, c_p, c_f, c_p, c_i64, c_p, c_i64, c_p,
                               c_size, c_p],
    "pk_gemm_mx8_ex_f32": [c_i64, c_i64, c_i64, c_f, c_p, c_p, c_f, c_p, c_i64, c_p, c_i64, c_p,
                           c_size, c_p],
    "pk_gemm_mx8_plan": [c_i64, c_i64, c_i64, ctypes.POINTER(c_int), ctypes.POINTER(c_int),
                         ctypes.POINTER(c_int)],
    "pk_gemm_bf16_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64, c_f,
                         c_p, c_i64, c_p],
    "pk_gemm_ex_bf16_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64,
                            c_f, c_p, c_i64, c_p, c_size, c_p],
    "pk_gemm_bf16x3_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64, c_f,
                         c_p, c_i64, c_p],
    "pk_gemm_ex_bf16x3_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_p, c_i64,
                            c_f, c_p, c_i64, c_p, c_size, c_p],
    "pk_gemm_batched_f32": [c_char, c_char, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_i64, c_i64,
                            c_p, c_i64, c_i64, c_i64, c_f, c_p, c_i64, c_i64, c_i64, c_i64,
                            c_i64, c_int, c_p],
    "pk_binary_f32": [c_int, c_int, c_p, c_p, c_p, c_p, c_p, c_p, c_p],
    "pk_binary_bwd_f32": [c_int, c_int, c_int, c_p, c_p, c_p, c_i64, c_p, c_p, c_p, c_int, c_p],
    "pk_unary_f32": [c_int, c_i64, c_p, c_p, c_p],
    "pk_unary_bwd_f32": [c_int, c_i64, c_p, c_p, c_p, c_p, c_int, c_p],
    "pk_relu_f32": [c_i64, c_p, c_p, c_p],
    "pk_relu_bwd_f32": [c_i64, c_p, c_p, c_p, c_int, c_p],
    "pk_fill_f32": [c_i64, c_f, c_p, c_p],
    "pk_fill2d_f32": [c_i64, c_i64, c_f, c_p, c_i64, c_p],
    "pk_fill_normal_f32": [c_i64, ctypes.c_uint64, c_f, c_f, c_p, c_p],
    "pk_axpy_f32": [c_i64, c_f, c_p, c_p, c_p, c_int, c_p],
    "pk_reduce_sum_f32": [c_i64, c_p, c_f, c_p, c_int, c_p],
    "pk_sgd_f32": [c_i64, c_f, c_p, c_p, c_p],
    "pk_sgd_multi_f32": [c_int, c_p, c_p, c_p, c_f, c_p],
    "pk_adamw_f32": [c_i64, c_f, c_f, c_f, c_f, c_f, c_int, c_p, c_p, c_p, c_p, c_p],
    "pk_adamw_prep_f32": [c_p, c_f, c_f, c_f, c_p, c_p],
    "pk_adamw_multi_f32": [c_i64, c_p, c_f, c_f, c_f, c_f, c_f, c_p, c_p],
    "pk_xent_fwd_bwd_f32": [c_i64, c_i64, c_p, c_i64, c_p, c_p, c_p, c_i64, c_f, c_p, c_int,
                            c_p],
    "pk_xent_mean_f32": [c_i64, c_i64, c_p, c_i64, c_p, c_p, c_p, c_i64, c_f, c_int, c_f, c_p, c_p],
    "pk_argmax_f32": [c_i64, c_i64, c_p, c_i64, c_p, c_p],
    "pk_rmsnorm_fwd_f32": [c_i64, c_i64, c_f, c_p, c_p, c_p, c_p, c_p],
    "pk_rmsnorm_bwd_workspace": [c_i64, c_i64],
    "pk_rmsnorm_bwd_f32": [c_i64, c_i64, c_p, c_p, c_p, c_p, c_p, c_p, c_int, c_p, c_size, c_p],
    "pk_rmsnorm_bwd_into_f32": [c_i64, c_i64, c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_int, c_p, c_size,
                                c_p],
    "pk_rmsnorm_dg_reduce_f32": [c_i64, c_i64, c_p, c_size, c_p, c_int, c_p],
    "pk_swiglu_fwd_f32": [c_i64, c_i64, c_p, c_i64, c_p, c_i64, c_p, c_i64, c_p],
    "pk_swiglu_bwd_f32": [c_i64, c_i64, c_p, c_i64, c_p, c_i64, c_p, c_i64, c_p, c_p, c_i64,
                          c_int, c_p],
    "pk_attn_causal_fwd_f32": [c_i64, c_i64, c_i64, c_i64, c_i64, c_f, c_p, c_p, c_p, c_p, c_p,
                               c_p, c_p],
    "pk_attn_causal_bwd_f32": [c_i64, c_i64, c_i64, c_i64, c_i64, c_f, c_p, c_p, c_p, c_p, c_p,
                               c_p, c_p, c_p, c_p, c_int, c_p],
    "pk_flash_attn_supported": [c_i64, c_i64],
    "pk_flash_attn_fwd_f32": [c_i64, c_i64, c_i64, c_i64, c_i64, c_f, c_p, c_p, c_p, c_p, c_p,
                              c_p],
    "pk_flash_attn_fwd_bf16_f32": [c_i64, c_i64, c_i64, c_i64, c_i64, c_f, c_p, c_p, c_p, c_p,
                                   c_p, c_p],
    "pk_flash_attn_bwd_workspace": [c_i64, c_i64, c_i64],
    "pk_flash_attn_bwd_workspace_recompute": [c_i64, c_i64, c_i64],
    "pk_flash_attn_bwd_f32": [c_i64, c_i64, c_i64, c_i64, c_i64, c_f, c_p, c_p, c_p, c_p, c_p,
                              c_p, c_p, c_p, c_p, c_p, c_size, c_int, c_p],
    "pk_flash_attn_bwd_bf16_f32": [c_i64, c_i64, c_i64, c_i64, c_i64, c_f, c_p, c_p, c_p, c_p,
                                   c_p, c_p, c_p, c_p, c_p, c_p, c_size, c_int, c_p],
    "pk_flash_attn_fwd_bf16x3_f32": [c_i64, c_i64, c_i64, c_i64, c_i64, c_f, c_p, c_p, c_p, c_p,
                                     c_p, c_p],
    "pk_flash_attn_bwd_bf16x3_f32": [c_i64, c_i64, c_i64, c_i64, c_i64, c_f, c_p, c_p, c_p, c_p,
                                     c_p, c_p, c_p, c_p, c_p, c_p, c_size, c_int, c_p],
    "pk_flash_attn_fwd_fp8_f32": [c_i64, c_i64, c_i64, c_i64, c_i64, c_f, c_p, c_p, c_p, c_p,
                                  c_p, c_p, c_p],
    "pk_flash_attn_bwd_fp8_f32": [c_i64, c_i64, c_i64, c_i64, c_i64, c_f, c_p, c_p, c_p, c_p,
                                  c_p, c_p, c_p, c_p, c_p, c_p, c_p, c_size, c_int, c_p],
    "pk_causal_softmax_fwd_f32": [c_i64, c_i64, c_f, c_p, c_p, c_p, c_p],
    "pk_causal_softmax_bwd_f32": [c_i64, c_i64, c_p, c_p, c_p, c_p],
    "pk_embed_fwd_f32": [c_i64, c_i64, c_i64, c_p, c_p, c_p, c_p],
    "pk_embed_bwd_workspace": [c_i64],
    "pk_embed_bwd_f32": [c_i64, c_i64, c_i64, c_p, c_p, c_p, c_p, c_size, c_p],
    "pk_last_error": [],
}
_RESTYPES = {"pk_last_error": ctypes.c_char_p, "pk_rmsnorm_bwd_workspace": c_size,
             "pk_gemm_workspace_f32": c_size, "pk_flash_attn_bwd_workspace": c_size,
             "pk_flash_attn_bwd_workspace_recompute": c_size,
             "pk_embed_bwd_workspace": c_size, "pk_gemm_noalloc_scratch_bytes": c_size,
             "pk_fp8_quantized_bytes": c_size, "pk_mx8_bytes": c_size,
             "pk_gemm_mx8_workspace": c_size, "pk_bf16q_bytes": c_size,
             "pk_gemm_bf16q_workspace": c_size, "pk_bf16x3q_bytes": c_size,
             "pk_gemm_bf16x3q_workspace": c_size}

_hip = None


def hip_lib() -> ctypes.CDLL:
    """The pk_* launcher library; raises if it has not been built."""
    global _hip
    if _hip is None:
        if not os.path.exists(HIP_LIB_PATH):
            raise RuntimeError(
                f"pico_amd: {HIP_LIB_PATH} is missing; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` (there is no CPU fallback)")
        lib = ctypes.CDLL(HIP_LIB_PATH)
        for name, argtypes in PK_SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPES.get(name, c_int)
        _hip = lib
    return _hip


def exported_symbols() -> list[str]:
    """Every pk_* name include/pico_hip.h declares (used by the load test)."""
    return sorted(PK_SIGNATURES)


class PkError(RuntimeError):
    pass


def check(name: str, status: int) -> None:
    if status != 0:
        msg = hip_lib().pk_last_error().decode(errors="replace")
        raise PkError(f"{name} returned {status}: {msg}")
