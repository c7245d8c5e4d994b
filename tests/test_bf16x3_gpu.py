"""fp32 products from three bf16 ones (pk_gemm_bf16x3_f32,
PICO_MATMUL_BF16X3): each operand x splits as hi = bf16(x), lo = bf16(x - hi)
and a.b is taken as ahi.bhi + ahi.blo + alo.bhi, accumulated in fp32.

* Integer operands of magnitude <= 300: hi and lo are small integers (the
  split is exact), every partial product and sum is an exact fp32 integer, so
  the result equals, bit for bit, the float64 sum of the three products with
  the split done on the host -- which pins the split, the three products and
  the dropped alo.blo term, for every tile shape, layout and edge path.
* Uniform operands: within the fp32 parity bound (1e-4, normalised as for
  the fp32 GEMM) of the float64 product, and far closer than plain bf16.
* The transformer step in PICO_MATMUL_BF16X3 mode meets the fp32 parity
  contract against the float64 reference: loss and every gradient <= 1e-4.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import kernels as K
from tests._util import gemm_err
from tests.test_bf16_gpu import bf16_round
from tests.test_gpt_gpu import _check_step

pytestmark = pytest.mark.gpu
TOL = 1e-4


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _split(x):
    hi = bf16_round(x).astype(np.float64)
    return hi, x.astype(np.float64) - hi


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,Kd", [(256, 256, 96), (512, 768, 64), (8192, 768, 32),
                                    (130, 257, 70), (64, 64, 96), (1000, 1376, 36)])
def test_bf16x3_integers_bitexact(dev, ta, tb, M, N, Kd):
    rng = np.random.default_rng(M * 7 + N + Kd)
    A = rng.integers(-300, 301, (M, Kd)).astype(np.float32)
    B = rng.integers(-300, 301, (Kd, N)).astype(np.float32)
    ah, al = _split(A)
    bh, bl = _split(B)
    assert np.all(np.abs(al) <= 2) and np.any(al != 0)  # the lo parts are in play
    want = ah @ bh + ah @ bl + al @ bh
    assert np.max(np.abs(want)) < 2 ** 24
    Ao = np.ascontiguousarray(A.T) if ta == "T" else A
    Bo = np.ascontiguousarray(B.T) if tb == "T" else B
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm_bf16x3(ta, tb, cu(Ao), cu(Bo), C)
    assert np.array_equal(host(C), want.astype(np.float32))


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N")])
@pytest.mark.parametrize("n", [512, 2048])
def test_bf16x3_uniform_within_fp32_bound(dev, ta, tb, n):
    A = O.uniform(n * n, 5).reshape(n, n)
    B = O.uniform(n * n, 6).reshape(n, n)
    C = torch.empty(n, n, device=dev)
    K.gemm_bf16x3(ta, tb, cu(A), cu(B), C)
    got = host(C)
    err = gemm_err(got, A, B, ta, tb)
    assert err <= TOL, err
    C16 = torch.empty(n, n, device=dev)
    K.gemm_bf16(ta, tb, cu(A), cu(B), C16)
    assert err * 20 < gemm_err(host(C16), A, B, ta, tb)


def test_bf16x3_split_k_workspace(dev):
    # a weight-gradient shape: K split through the workspace, deterministic
    M, N, Kd = 768, 2048, 8192
    A = O.uniform(Kd * M, 8).reshape(Kd, M)
    B = O.uniform(Kd * N, 9).reshape(Kd, N)
    ws = torch.empty(K.gemm_workspace(M, N, Kd) // 4, device=dev)
    C1, C2 = torch.empty(M, N, device=dev), torch.empty(M, N, device=dev)
    K.gemm_bf16x3("T", "N", cu(A), cu(B), C1, ws=ws)
    K.gemm_bf16x3("T", "N", cu(A), cu(B), C2, ws=ws)
    assert np.array_equal(host(C1), host(C2))
    assert gemm_err(host(C1), A, B, "T", "N") <= TOL


@pytest.fixture
def bf16x3_mode():
    from pico_amd.pico import Pico
    P = Pico()
    assert P.lib.pico_set_matmul_precision(2) == 0
    yield P
    assert P.lib.pico_set_matmul_precision(0) == 0


def test_bf16x3_transformer_step_meets_fp32_parity(bf16x3_mode):
    P = bf16x3_mode
    _check_step(P, dict(vocab=96, d_model=64, n_layers=2, n_heads=2, d_ff=160, batch=2,
                        seq_len=64), 11)
    _check_step(P, dict(vocab=8192, d_model=512, n_layers=1, n_heads=8, d_ff=1376, batch=16,
                        seq_len=256), 21)
