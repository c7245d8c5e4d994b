"""bf16 operands held in HBM (pk_bf16q_quantize_f32 / _quantize2_f32 +
pk_gemm_bf16q_f32): outside the fp32 parity contract, pinned by what the
arithmetic fixes.

* Casts: every 2-byte value equals torch's own bfloat16 conversion of the fp32
  value (round to nearest even), NaN stays NaN, the padding rows and columns
  are zero, the transposed read equals the cast of the transposed copy, and
  the one-read dual cast equals the two casts byte for byte.
* Products: a product of two bf16 values is exact in fp32, so integers of
  magnitude <= 256 give bit-exact results at every shape (ragged M, N, K,
  single rows, K of one value, K not a multiple of the 32-value slice, split
  and unsplit K), and uniform operands give the float64 product of the
  rounded operands up to fp32 summation error.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import kernels as K
from tests._util import gemm_err

pytestmark = pytest.mark.gpu
TOL = 1e-4


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def padded(R, Kd):
    return -(-R // 256) * 256, -(-Kd // 64) * 64


def bf16_view(Q, R, Kd):
    """the [Rp, Kv] int16 array a bf16 operand matrix holds"""
    Rp, Kv = padded(R, Kd)
    return host(Q)[:Rp * Kv * 2].view(np.int16).reshape(Rp, Kv)


def torch_bf16_bits(X):
    return torch.from_numpy(np.ascontiguousarray(X, np.float32)).to(torch.bfloat16).view(
        torch.int16).numpy()


def bf16_values(Q, R, Kd):
    """float64 values of the [R, Kd] part"""
    b = bf16_view(Q, R, Kd)[:R, :Kd].astype(np.int32) & 0xFFFF
    return (b << 16).astype(np.uint32).view(np.float32).astype(np.float64)


def _mixed(R, Kd, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((R, Kd)).astype(np.float32)
    X *= np.exp2(rng.integers(-20, 20, (R, 1))).astype(np.float32)
    X[:, ::7] = 0.0
    return X


@pytest.mark.parametrize("R,Kd", [(1, 1), (70, 130), (256, 64), (300, 1000), (257, 65)])
def test_bf16q_cast_matches_torch(dev, R, Kd):
    X = _mixed(R, Kd, R + Kd)
    X[0, 0] = 1.0 + 2.0 ** -8  # a tie: rounds to even (1.0)
    if Kd > 1:
        X[0, 1] = 1.0 + 3 * 2.0 ** -8  # a tie: rounds up to even
    Q = K.bf16q_quantize(cu(X), False)
    assert Q.numel() >= K.bf16q_bytes(R, Kd)
    got = bf16_view(Q, R, Kd)
    want = torch_bf16_bits(X)
    assert np.array_equal(got[:R, :Kd], want)
    assert not np.any(got[R:, :]) and not np.any(got[:, Kd:])


def test_bf16q_cast_nan_inf(dev):
    X = np.array([[np.nan, np.inf, -np.inf, -0.0, 3.4e38, 1e-40]], np.float32)
    v = bf16_values(K.bf16q_quantize(cu(X), False), 1, 6)[0]
    assert np.isnan(v[0]) and v[1] == np.inf and v[2] == -np.inf
    assert v[3] == 0.0 and np.signbit(v[3])
    assert np.array_equal(v[4:], torch.from_numpy(X[0, 4:]).to(torch.bfloat16).double().numpy())


@pytest.mark.parametrize("R,Kd", [(1, 5), (130, 70), (512, 256), (300, 1000)])
def test_bf16q_cast_transposed_read(dev, R, Kd):
    X = _mixed(Kd, R, 3 * R + Kd)  # stored [Kd, R]; op(X) = X^T
    Qt = K.bf16q_quantize(cu(X), True)
    Qc = K.bf16q_quantize(cu(X.T.copy()), False)
    n = K.bf16q_bytes(R, Kd)
    assert np.array_equal(host(Qt)[:n], host(Qc)[:n])


@pytest.mark.parametrize("M,N", [(1, 1), (70, 130), (256, 128), (300, 1000), (8192, 768)])
def test_bf16q_dual_cast_equals_two_casts(dev, M, N):
    X = _mixed(M, N, M + 5 * N)
    dX = cu(X)
    QR, QT = K.bf16q_quantize2(dX)
    assert np.array_equal(host(QR)[:K.bf16q_bytes(M, N)],
                          host(K.bf16q_quantize(dX, False))[:K.bf16q_bytes(M, N)])
    assert np.array_equal(host(QT)[:K.bf16q_bytes(N, M)],
                          host(K.bf16q_quantize(dX, True))[:K.bf16q_bytes(N, M)])
    wide = cu(np.concatenate([X, X[:, :N // 2 + 1] * 3.0], axis=1))
    QR2, QT2 = K.bf16q_quantize2(wide[:, :N])
    assert np.array_equal(host(QR2), host(QR)) and np.array_equal(host(QT2), host(QT))


def _product(dev, X, Y, alpha=1.0, beta=0.0, C0=None, ws=None):
    M, Kd = X.shape
    N = Y.shape[1]
    A = K.bf16q_quantize(cu(X), False)
    B = K.bf16q_quantize(cu(Y), True)
    C = torch.full((M, N), float("nan"), device=dev) if C0 is None else cu(C0)
    K.gemm_bf16q(M, N, Kd, A, B, C, alpha=alpha, beta=beta, ws=ws)
    return host(C), A, B


SHAPES = [(256, 256, 64), (512, 768, 320), (1, 1, 1), (300, 257, 65), (1000, 333, 1000),
          (64, 4096, 128), (4096, 4096, 512), (2048, 768, 4096), (257, 511, 4095)]


@pytest.mark.parametrize("M,N,Kd", SHAPES)
def test_bf16q_gemm_integers_bitexact(dev, M, N, Kd):
    rng = np.random.default_rng(M * 5 + N + Kd)
    mag = 256 if Kd <= 1000 else 64  # bf16 holds integers to 256 exactly
    X = rng.integers(-mag, mag + 1, (M, Kd)).astype(np.float32)
    Y = rng.integers(-mag, mag + 1, (Kd, N)).astype(np.float32)
    ref64 = X.astype(np.float64) @ Y.astype(np.float64)
    assert np.max(np.abs(ref64)) < 2 ** 24  # every partial sum exact in fp32
    ref = ref64.astype(np.float32)
    got, _, _ = _product(dev, X, Y)
    assert np.array_equal(got, ref)
    got, _, _ = _product(dev, X, Y, alpha=-1.0, beta=1.0, C0=ref)
    assert not np.any(got)


@pytest.mark.parametrize("M,N,Kd", [(1024, 1024, 1024), (300, 257, 70), (4096, 768, 768)])
def test_bf16q_gemm_equals_product_of_rounded_operands(dev, M, N, Kd):
    X = O.uniform(M * Kd, M + 1).reshape(M, Kd)
    Y = O.uniform(Kd * N, N + 2).reshape(Kd, N)
    C, A, B = _product(dev, X, Y)
    Xd, Yd = bf16_values(A, M, Kd), bf16_values(B, N, Kd)
    assert gemm_err(C, Xd, Yd.T) <= TOL
    assert gemm_err(C, X, Y) < 2 ** -6


@pytest.mark.parametrize("M,N,Kd", [(768, 768, 8192), (2048, 768, 8192), (8192, 768, 32000),
                                    (300, 200, 5000)])
def test_bf16q_gemm_k_split(dev, M, N, Kd):
    """a split K: integers exact with and without the workspace, alpha, beta
    and a row X through the split's reduction"""
    wsb = K.bf16q_workspace(M, N, Kd)
    ws = torch.empty(wsb // 4 + 1, device=dev)
    rng = np.random.default_rng(M + N + Kd)
    X = rng.integers(-16, 17, (M, Kd)).astype(np.float32)
    Y = rng.integers(-16, 17, (Kd, N)).astype(np.float32)
    ref = (X.astype(np.float64) @ Y.astype(np.float64)).astype(np.float32)
    got, A, B = _product(dev, X, Y, ws=ws)
    assert np.array_equal(got, ref)
    C = torch.empty(M, N, device=dev)
    K.gemm_bf16q(M, N, Kd, A, B, C)  # unsplit
    assert np.array_equal(host(C), ref)
    b = O.uniform(N, 12)
    K.gemm_bf16q(M, N, Kd, A, B, C, alpha=0.5, beta=2.0, X=cu(b), ws=ws)
    want = 0.5 * ref.astype(np.float64) + 2.0 * b[None, :].astype(np.float64)
    assert np.max(np.abs(host(C) - want)) <= 1e-6 * np.max(np.abs(want))


def test_bf16q_gemm_epilogue_adds_x(dev):
    M, N, Kd = 300, 520, 200
    X = O.uniform(M * Kd, 1).reshape(M, Kd)
    Y = O.uniform(Kd * N, 2).reshape(Kd, N)
    P, A, B = _product(dev, X, Y)
    R = O.uniform(M * N, 3).reshape(M, N)
    b = O.uniform(N, 4)
    for Xadd, want in ((R, 2.0 * P + 0.5 * R), (b, 2.0 * P + 0.5 * b[None, :])):
        C = torch.full((M, N), float("nan"), device=dev)
        K.gemm_bf16q(M, N, Kd, A, B, C, alpha=2.0, beta=0.5, X=cu(Xadd))
        assert np.max(np.abs(host(C) - want)) <= 1e-6 * np.max(np.abs(want))
    C = cu(R)
    K.gemm_bf16q(M, N, Kd, A, B, C, beta=1.0)
    assert np.max(np.abs(host(C) - (P + R))) <= 1e-6 * np.max(np.abs(P + R))


def test_bf16q_refusals(dev):
    from pico_amd import _lib

    L = _lib.hip_lib()
    Q = torch.zeros(K.bf16q_bytes(256, 128) + 16, dtype=torch.uint8, device=dev)
    C = torch.zeros(4, 4, device=dev)
    X = torch.zeros(4, 100, device=dev)
    assert L.pk_bf16q_quantize_f32(4, 100, X.data_ptr(), 100, 0, Q.data_ptr() + 8, None) != 0
    assert L.pk_bf16q_quantize_f32(4, 100, X.data_ptr(), 99, 0, Q.data_ptr(), None) != 0
    assert L.pk_bf16q_quantize2_f32(4, 100, X.data_ptr(), 99, Q.data_ptr(), Q.data_ptr(), None) != 0
    assert L.pk_gemm_bf16q_f32(4, 4, 100, 1.0, Q.data_ptr() + 4, Q.data_ptr(), 0.0, None, 0,
                               C.data_ptr(), 4, None) != 0
    assert L.pk_gemm_bf16q_f32(4, 4, 100, 1.0, Q.data_ptr(), Q.data_ptr(), 1.0, None, 0,
                               C.data_ptr(), 4, None) != 0
    assert L.pk_gemm_bf16q_f32(4, 4, 100, 1.0, Q.data_ptr(), Q.data_ptr(), 0.0, None, 0,
                               C.data_ptr(), 3, None) != 0
