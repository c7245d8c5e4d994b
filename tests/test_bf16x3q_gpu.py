"""Split-bf16 operands held in HBM (pk_bf16x3q_quantize_f32 + pk_gemm_bf16x3q_f32):
fp32 products from three bf16 ones over operands cast once, pinned by what the
arithmetic fixes and by the fp32-operand kernel that computes the same sums.

* Casts: every value's hi part equals torch's bfloat16 of the fp32 value
  (nearest even) and its lo part torch's bfloat16 of x - hi, in the group
  layout (16 hi parts, then their 16 lo parts); the padding rows and columns
  are zero and the transposed read equals the cast of the transposed copy.
* Products: ahi.bhi + ahi.blo + alo.bhi in pk_gemm_bf16x3_f32's order, so an
  unsplit product equals pk_gemm_bf16x3_f32's bit for bit at every shape;
  integer operands of magnitude <= 300 (lo parts in play) give the float64 sum
  of the three products exactly, split and unsplit; uniform operands are
  within the fp32 parity bound of the float64 product.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import kernels as K
from tests._util import gemm_err
from tests.test_bf16x3_gpu import _split

pytestmark = pytest.mark.gpu
TOL = 1e-4


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def padded(R, Kd):
    return -(-R // 256) * 256, -(-Kd // 32) * 32


def split_layout(X):
    """the bytes a cast of X [R, Kd] holds: [Rp, Kv / 16 groups, 32] int16,
    each group's 16 hi parts then its 16 lo parts (torch's bfloat16)"""
    R, Kd = X.shape
    Rp, Kv = padded(R, Kd)
    x = torch.zeros(Rp, Kv, dtype=torch.float32)
    x[:R, :Kd] = torch.from_numpy(np.ascontiguousarray(X, np.float32))
    hi = x.to(torch.bfloat16)
    lo = (x - hi.to(torch.float32)).to(torch.bfloat16)
    g = Kv // 16
    h16 = hi.view(torch.int16).reshape(Rp, g, 16)
    l16 = lo.view(torch.int16).reshape(Rp, g, 16)
    return torch.cat([h16, l16], dim=2).numpy()


def cast_view(Q, R, Kd):
    Rp, Kv = padded(R, Kd)
    return host(Q)[:Rp * Kv * 4].view(np.int16).reshape(Rp, Kv // 16, 32)


def _mixed(R, Kd, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((R, Kd)).astype(np.float32)
    X *= np.exp2(rng.integers(-20, 20, (R, 1))).astype(np.float32)
    X[:, ::7] = 0.0
    return X


@pytest.mark.parametrize("R,Kd", [(1, 1), (70, 130), (256, 64), (300, 1000), (257, 33), (5, 32)])
def test_bf16x3q_cast_layout(dev, R, Kd):
    X = _mixed(R, Kd, R + 3 * Kd)
    X[0, 0] = 1.0 + 2.0 ** -8 + 2.0 ** -20  # hi rounds up; lo is negative
    Q = K.bf16x3q_quantize(cu(X), False)
    assert Q.numel() >= K.bf16x3q_bytes(R, Kd)
    assert np.array_equal(cast_view(Q, R, Kd), split_layout(X))


@pytest.mark.parametrize("R,Kd", [(1, 5), (130, 70), (512, 256), (300, 1000), (64, 33)])
def test_bf16x3q_cast_transposed_read(dev, R, Kd):
    X = _mixed(Kd, R, 5 * R + Kd)  # stored [Kd, R]; op(X) = X^T
    Qt = K.bf16x3q_quantize(cu(X), True)
    n = K.bf16x3q_bytes(R, Kd)
    assert np.array_equal(host(Qt)[:n], host(K.bf16x3q_quantize(cu(X.T.copy()), False))[:n])
    assert np.array_equal(cast_view(Qt, R, Kd), split_layout(X.T))


def _product(dev, X, Y, alpha=1.0, beta=0.0, C0=None, ws=None):
    M, Kd = X.shape
    N = Y.shape[1]
    A = K.bf16x3q_quantize(cu(X), False)
    B = K.bf16x3q_quantize(cu(Y), True)
    C = torch.full((M, N), float("nan"), device=dev) if C0 is None else cu(C0)
    K.gemm_bf16x3q(M, N, Kd, A, B, C, alpha=alpha, beta=beta, ws=ws)
    return host(C), A, B


SHAPES = [(256, 256, 64), (512, 768, 320), (1, 1, 1), (300, 257, 65), (1000, 333, 1000),
          (64, 4096, 128), (2048, 768, 4096), (257, 511, 4095), (130, 1376, 36)]


@pytest.mark.parametrize("M,N,Kd", SHAPES)
def test_bf16x3q_equals_fp32_operand_bf16x3(dev, M, N, Kd):
    """the same three products per 16 values of K, in the same order: an
    unsplit product equals pk_gemm_bf16x3_f32's bit for bit"""
    X = O.uniform(M * Kd, M + 7).reshape(M, Kd)
    Y = O.uniform(Kd * N, N + 8).reshape(Kd, N)
    got, _, _ = _product(dev, X, Y)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm_bf16x3("N", "N", cu(X), cu(Y), C)
    assert np.array_equal(got, host(C))
    assert gemm_err(got, X, Y) <= TOL


@pytest.mark.parametrize("M,N,Kd", [(256, 256, 96), (512, 768, 64), (130, 257, 70), (1000, 1376, 36)])
def test_bf16x3q_integers_bitexact(dev, M, N, Kd):
    rng = np.random.default_rng(M * 3 + N + Kd)
    X = rng.integers(-300, 301, (M, Kd)).astype(np.float32)
    Y = rng.integers(-300, 301, (Kd, N)).astype(np.float32)
    ah, al = _split(X)
    bh, bl = _split(Y)
    assert np.any(al != 0)  # the lo parts are in play
    want = (ah @ bh + ah @ bl + al @ bh).astype(np.float32)
    got, _, _ = _product(dev, X, Y)
    assert np.array_equal(got, want)
    got, _, _ = _product(dev, X, Y, alpha=-1.0, beta=1.0, C0=want)
    assert not np.any(got)


@pytest.mark.parametrize("M,N,Kd", [(768, 768, 8192), (2048, 768, 8192), (300, 200, 5000)])
def test_bf16x3q_k_split(dev, M, N, Kd):
    """a split K: integers exact with and without the workspace; uniform
    operands within the parity bound either way"""
    wsb = K.bf16x3q_workspace(M, N, Kd)
    ws = torch.empty(wsb // 4 + 1, device=dev)
    rng = np.random.default_rng(M + N + Kd)
    X = rng.integers(-16, 17, (M, Kd)).astype(np.float32)
    Y = rng.integers(-16, 17, (Kd, N)).astype(np.float32)
    ref = (X.astype(np.float64) @ Y.astype(np.float64)).astype(np.float32)
    got, A, B = _product(dev, X, Y, ws=ws)
    assert np.array_equal(got, ref)
    C = torch.empty(M, N, device=dev)
    K.gemm_bf16x3q(M, N, Kd, A, B, C)  # unsplit
    assert np.array_equal(host(C), ref)
    U = O.uniform(M * Kd, 3).reshape(M, Kd)
    V = O.uniform(Kd * N, 4).reshape(Kd, N)
    got, _, _ = _product(dev, U, V, ws=ws)
    assert gemm_err(got, U, V) <= TOL


def test_bf16x3q_epilogue_adds_x(dev):
    M, N, Kd = 300, 520, 200
    X = O.uniform(M * Kd, 1).reshape(M, Kd)
    Y = O.uniform(Kd * N, 2).reshape(Kd, N)
    P, A, B = _product(dev, X, Y)
    R = O.uniform(M * N, 3).reshape(M, N)
    b = O.uniform(N, 4)
    for Xadd, want in ((R, 2.0 * P + 0.5 * R), (b, 2.0 * P + 0.5 * b[None, :])):
        C = torch.full((M, N), float("nan"), device=dev)
        K.gemm_bf16x3q(M, N, Kd, A, B, C, alpha=2.0, beta=0.5, X=cu(Xadd))
        assert np.max(np.abs(host(C) - want)) <= 1e-6 * np.max(np.abs(want))


def test_bf16x3q_refusals(dev):
    from pico_amd import _lib

    L = _lib.hip_lib()
    Q = torch.zeros(K.bf16x3q_bytes(256, 128) + 16, dtype=torch.uint8, device=dev)
    C = torch.zeros(4, 4, device=dev)
    X = torch.zeros(4, 100, device=dev)
    assert L.pk_bf16x3q_quantize_f32(4, 100, X.data_ptr(), 100, 0, Q.data_ptr() + 8, None) != 0
    assert L.pk_bf16x3q_quantize_f32(4, 100, X.data_ptr(), 99, 0, Q.data_ptr(), None) != 0
    assert L.pk_gemm_bf16x3q_f32(4, 4, 100, 1.0, Q.data_ptr() + 4, Q.data_ptr(), 0.0, None, 0,
                                 C.data_ptr(), 4, None) != 0
    assert L.pk_gemm_bf16x3q_f32(4, 4, 100, 1.0, Q.data_ptr(), Q.data_ptr(), 1.0, None, 0,
                                 C.data_ptr(), 4, None) != 0
    assert L.pk_gemm_bf16x3q_f32(4, 4, 100, 1.0, Q.data_ptr(), Q.data_ptr(), 0.0, None, 0,
                                 C.data_ptr(), 3, None) != 0
