"""pk_gemm_noalloc_f32, the GEMM entry point that allocates nothing.

Its split-K partial planes live in a static device array instead of a caller
workspace.  It is compared through the C-ABI with pk_gemm_ex_f32 given a
workspace of its own: the same tiles, the same split and the same reduction
order, so the results must be equal bit for bit.  Two calls run back to back,
the second on a smaller product, so the second reads the array the first one
left behind; a product whose partials exceed the array is refused on the host.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import _lib

pytestmark = pytest.mark.gpu


def _ex(ta, tb, M, N, K, A, lda, B, ldb, beta, C, ldc, ws):
    L = _lib.hip_lib()
    _lib.check("pk_gemm_ex_f32", L.pk_gemm_ex_f32(
        ctypes.c_char(ta.encode()), ctypes.c_char(tb.encode()), M, N, K, 1.0, A.data_ptr(), lda,
        B.data_ptr(), ldb, beta, C.data_ptr(), ldc, ws.data_ptr(), ws.numel() * 4, None))


def _noalloc(ta, tb, M, N, K, A, lda, B, ldb, beta, C, ldc):
    L = _lib.hip_lib()
    return L.pk_gemm_noalloc_f32(ctypes.c_char(ta.encode()), ctypes.c_char(tb.encode()), M, N, K,
                                 1.0, A.data_ptr(), lda, B.data_ptr(), ldb, beta, C.data_ptr(),
                                 ldc, None)


# (ta, tb, M, N, K, beta): a d_model-768 weight gradient (A^T . dC, 14 K slices),
# then a smaller NN product with a ragged edge and accumulation
CASES = [("T", "N", 768, 768, 8192, 0.0), ("N", "N", 200, 136, 3000, 1.0)]


def test_noalloc_matches_workspace_entry_point_twice(dev):
    L = _lib.hip_lib()
    cap = L.pk_gemm_noalloc_scratch_bytes()
    assert cap == 128 << 20
    for i, (ta, tb, M, N, K, beta) in enumerate(CASES):
        need = L.pk_gemm_workspace_f32(M, N, K)
        assert 0 < need <= cap, (M, N, K, need)  # both products split K
        a_shape = (K, M) if ta == "T" else (M, K)
        b_shape = (N, K) if tb == "T" else (K, N)
        A = torch.from_numpy(O.uniform(M * K, 100 + i).reshape(a_shape)).to(dev)
        B = torch.from_numpy(O.uniform(K * N, 200 + i).reshape(b_shape)).to(dev)
        C0 = torch.from_numpy(O.uniform(M * N, 300 + i).reshape(M, N)).to(dev)
        lda, ldb = a_shape[1], b_shape[1]
        ref = C0.clone()
        ws = torch.empty(need // 4, device=dev)
        _ex(ta, tb, M, N, K, A, lda, B, ldb, beta, ref, N, ws)
        got = C0.clone()
        _lib.check("pk_gemm_noalloc_f32", _noalloc(ta, tb, M, N, K, A, lda, B, ldb, beta, got, N))
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"case {i}: not bit-equal to pk_gemm_ex_f32"
        # and both are the product (normalised error against float64)
        a64 = A.double().cpu().numpy()
        b64 = B.double().cpu().numpy()
        opa = a64.T if ta == "T" else a64
        opb = b64.T if tb == "T" else b64
        want = opa @ opb + beta * C0.double().cpu().numpy()
        den = np.abs(opa) @ np.abs(opb) + abs(beta) * np.abs(C0.double().cpu().numpy())
        assert np.max(np.abs(got.double().cpu().numpy() - want) / den) <= 1e-4


def test_noalloc_refuses_partials_above_its_scratch(dev):
    L = _lib.hip_lib()
    # A^T.B (a weight gradient's layout) splits K: 286 MiB of partial planes
    M, N, K = 1408, 2048, 65536
    need = L.pk_gemm_workspace_f32(M, N, K)
    assert need > L.pk_gemm_noalloc_scratch_bytes()
    # valid buffers of the right sizes, although a refused call touches none
    A = torch.zeros(K, M, device=dev)
    B = torch.zeros(K, N, device=dev)
    C = torch.full((M, N), 7.0, device=dev)
    st = _noalloc("T", "N", M, N, K, A, M, B, N, 0.0, C, N)
    assert st == -1
    assert b"static scratch" in L.pk_last_error()
    torch.cuda.synchronize()
    assert bool((C == 7.0).all())


def test_noalloc_long_k_forward_layout_runs_unsplit(dev):
    """The same shape as A.B: two 64x64 tiles per CU, so it runs unsplit and
    needs no scratch, whatever the A^T.B layout would."""
    L = _lib.hip_lib()
    M, N, K = 1408, 2048, 65536
    A = torch.ones(M, K, device=dev)
    B = torch.full((K, N), 0.5, device=dev)
    C = torch.full((M, N), 7.0, device=dev)
    assert _noalloc("N", "N", M, N, K, A, K, B, N, 0.0, C, N) == 0
    torch.cuda.synchronize()
    assert bool((C == 0.5 * K).all())


def test_noalloc_unsplit_product_needs_no_scratch(dev):
    """A product with enough tiles runs unsplit: same result as pk_gemm_f32."""
    L = _lib.hip_lib()
    M, N, K = 512, 512, 256
    assert L.pk_gemm_workspace_f32(M, N, K) == 0
    A = torch.from_numpy(O.uniform(M * K, 7).reshape(M, K)).to(dev)
    B = torch.from_numpy(O.uniform(K * N, 8).reshape(K, N)).to(dev)
    ref = torch.empty(M, N, device=dev)
    got = torch.empty(M, N, device=dev)
    _lib.check("pk_gemm_f32", L.pk_gemm_f32(b"N", b"N", M, N, K, 1.0, A.data_ptr(), K,
                                            B.data_ptr(), N, 0.0, ref.data_ptr(), N, None))
    _lib.check("pk_gemm_noalloc_f32", _noalloc("N", "N", M, N, K, A, K, B, N, 0.0, got, N))
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
