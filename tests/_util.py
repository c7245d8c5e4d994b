"""Error metrics shared by the parity tests."""
import numpy as np


def gemm_err(C, A, B, ta="N", tb="N", C_ref=None):
    """max |C - C_ref| / sum_k |op(A)_ik||op(B)_kj|  (componentwise-normalised;
    C_ref from an fp64 product when not given)."""
    A64 = np.asarray(A, np.float64)
    B64 = np.asarray(B, np.float64)
    Aop = A64.T if ta == "T" else A64
    Bop = B64.T if tb == "T" else B64
    if C_ref is None:
        C_ref = Aop @ Bop
    denom = np.abs(Aop) @ np.abs(Bop)
    denom = np.maximum(denom, 1e-30)
    return float(np.max(np.abs(np.asarray(C, np.float64) - C_ref) / denom))


def row_err(x, ref):
    """max |x - ref| / max(|ref|, 1e-6 * max|ref|)"""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(float(np.max(np.abs(ref))) if ref.size else 0.0, 1e-30)
    denom = np.maximum(np.abs(ref), 1e-6 * scale)
    return float(np.max(np.abs(x - ref) / denom)) if ref.size else 0.0


def max_rel(x, ref):
    """max |x - ref| / max|ref| (norm-wise relative error)"""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(x - ref)) / max(float(np.max(np.abs(ref))), 1e-30))
