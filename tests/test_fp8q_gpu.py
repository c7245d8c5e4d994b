"""Narrow-operand fp8 products (pk_fp8_quantize_f32 + pk_gemm_fp8q_f32):
outside the fp32 parity contract, pinned by what the arithmetic fixes, as the
fp32-operand fp8 products are (tests/test_fp8_gpu.py, whose e4m3 restatement
is reused here).

* Quantization: every byte decodes (by the format's definition, written out
  below: sign, 4-bit exponent with bias 7, 3-bit mantissa, subnormals, 0x7f /
  0xff NaN) to e4m3_round(scale * x), and equals torch's own float8_e4m3fn
  encoding of the clamped value; padding rows and columns are zero; the
  transposed read equals the quantization of the transposed copy.
* Products: a product of two e4m3 values is exact in fp32, so integers of
  magnitude <= 16 give bit-exact results at every shape (ragged M, N, K,
  single rows, K of one byte, K not a multiple of the 64-byte slice), and
  uniform operands give the float64 product of the rounded operands up to
  fp32 summation error; with the operands' scales the result is that product
  divided by both scales.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import kernels as K
from pico_amd._lib import PkError
from tests._util import gemm_err
from tests.test_fp8_gpu import e4m3_round

pytestmark = pytest.mark.gpu
TOL = 1e-4


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def e4m3_decode(b):
    """e4m3 bytes -> float64, from the format's definition"""
    b = np.asarray(b).astype(np.int64)
    s, e, m = (b >> 7) & 1, (b >> 3) & 15, b & 7
    v = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return np.where(s == 1, -v, v)


def test_e4m3_decode_known_bytes():
    b = np.array([0x00, 0x80, 0x01, 0x08, 0x38, 0x3C, 0xB8, 0x7E, 0xFE, 0x7F, 0xFF, 0x07])
    want = [0.0, -0.0, 2 ** -9, 2 ** -6, 1.0, 1.5, -1.0, 448.0, -448.0, np.nan, np.nan,
            7 * 2 ** -9]
    got = e4m3_decode(b)
    assert np.array_equal(got, np.array(want), equal_nan=True)


def one(v, dev):
    return torch.tensor([v], dtype=torch.float32, device=dev)


@pytest.mark.parametrize("R,Kd", [(1, 1), (70, 130), (256, 64), (300, 1000)])
def test_quantize_bytes_match_the_format(dev, R, Kd):
    rng = np.random.default_rng(R + Kd)
    X = np.concatenate([rng.uniform(-500, 500, R * Kd // 2 + 1), rng.uniform(-0.05, 0.05, R * Kd)])
    X = X[:R * Kd].astype(np.float32).reshape(R, Kd)
    X.ravel()[:4] = [448.0, 449.0, 1e9, -3e-4][:min(4, X.size)]
    for scale in (1.0, 4.0):
        Q = host(K.fp8_quantize(cu(X), False, one(scale, dev)))
        rows, ld = K.fp8_quantized_shape(R, Kd)
        assert Q.shape == (rows, ld) and rows % 256 == 0 and ld % 64 == 0 and ld >= Kd
        want = e4m3_round(X * np.float32(scale))
        assert np.array_equal(e4m3_decode(Q[:R, :Kd]), want.astype(np.float64))
        clamped = np.clip(X * np.float32(scale), -448.0, 448.0)
        tq = torch.from_numpy(clamped).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(Q[:R, :Kd], tq)
        assert not Q[R:].any() and not Q[:, Kd:].any()


def test_quantize_nan_stays_nan(dev):
    X = np.array([[np.nan, 1.0, -np.nan, 2.0]], np.float32)
    Q = host(K.fp8_quantize(cu(X), False, one(1.0, dev)))
    d = e4m3_decode(Q[0, :4])
    assert np.isnan(d[0]) and np.isnan(d[2]) and d[1] == 1.0 and d[3] == 2.0


@pytest.mark.parametrize("R,Kd", [(1, 5), (130, 70), (512, 256)])
def test_quantize_transposed_read(dev, R, Kd):
    X = O.uniform(R * Kd, 7).reshape(Kd, R) * 50.0  # op(X) = X^T is [R, Kd]
    Qt = host(K.fp8_quantize(cu(X), True, one(2.0, dev)))
    Qn = host(K.fp8_quantize(cu(np.ascontiguousarray(X.T)), False, one(2.0, dev)))
    assert np.array_equal(Qt, Qn)


def _product(dev, X, Y, scales=None, alpha=1.0, beta=0.0, C0=None):
    """C = alpha * X.Y (+ beta C0) through quantize + the narrow product"""
    M, Kd = X.shape
    N = Y.shape[1]
    sc = torch.ones(2, device=dev) if scales is None else scales
    dX, dY = cu(X), cu(Y)
    A8 = K.fp8_quantize(dX, False, sc[0:1])
    B8 = K.fp8_quantize(dY, True, sc[1:2])
    C = torch.full((M, N), float("nan"), device=dev) if C0 is None else cu(C0)
    K.gemm_fp8q(M, N, Kd, A8, B8, sc, C, alpha=alpha, beta=beta)
    return host(C)


SHAPES = [(256, 256, 64), (512, 768, 320), (1, 1, 1), (300, 257, 65), (1000, 333, 1000),
          (64, 4096, 128), (4096, 4096, 512), (2048, 768, 4096), (257, 511, 4095)]


@pytest.mark.parametrize("M,N,Kd", SHAPES)
def test_fp8q_gemm_integers_bitexact(dev, M, N, Kd):
    rng = np.random.default_rng(M * 7 + N + Kd)
    X = rng.integers(-16, 17, (M, Kd)).astype(np.float32)
    Y = rng.integers(-16, 17, (Kd, N)).astype(np.float32)
    ref = (X.astype(np.float64) @ Y.astype(np.float64)).astype(np.float32)
    assert np.array_equal(_product(dev, X, Y), ref)
    # C = -X.Y + C0 = 0 exactly
    assert not np.any(_product(dev, X, Y, alpha=-1.0, beta=1.0, C0=ref))


@pytest.mark.parametrize("M,N,Kd", [(1024, 1024, 1024), (300, 257, 70), (4096, 768, 768)])
def test_fp8q_gemm_equals_product_of_rounded_operands(dev, M, N, Kd):
    X = O.uniform(M * Kd, M + 1).reshape(M, Kd)
    Y = O.uniform(Kd * N, N + 2).reshape(Kd, N)
    C = _product(dev, X, Y)
    assert gemm_err(C, e4m3_round(X), e4m3_round(Y)) <= TOL
    assert 1e-3 < gemm_err(C, X, Y) < 2 ** -3  # fp8-sized
    # the fp32-operand fp8 product rounds the same operands: equal up to summation order
    C2 = torch.empty(M, N, device=dev)
    K.gemm_fp8("N", "N", cu(X), cu(Y), C2)
    assert gemm_err(C, e4m3_round(X), e4m3_round(Y), C_ref=host(C2).astype(np.float64)) <= TOL


def test_fp8q_gemm_with_operand_scales(dev):
    """gradient-sized operands: quantized with pk_fp8_scales_f32's powers of two
    and descaled in the epilogue, the result is the product of the rounded
    scaled operands divided by the scales, and not flushed to zero"""
    M, N, Kd = 512, 320, 448
    X = O.uniform(M * Kd, 31).reshape(M, Kd) * 2e-5
    Y = O.uniform(Kd * N, 32).reshape(Kd, N) * 0.02
    sc = K.fp8_scales(cu(X), cu(Y), torch.empty(2, device=dev))
    sa, sb = host(sc)
    C = _product(dev, X, Y, scales=sc, alpha=0.5)
    Xr = e4m3_round(X * sa).astype(np.float64) / sa
    Yr = e4m3_round(Y * sb).astype(np.float64) / sb
    assert gemm_err(C, 0.5 * Xr, Yr) <= TOL
    assert 1e-3 < gemm_err(C, 0.5 * X, Y) < 2 ** -3


def test_fp8q_gemm_empty_k_scales_c(dev):
    C0 = O.uniform(40 * 30, 5).reshape(40, 30)
    C = cu(C0)
    K.gemm_fp8q(40, 30, 0, torch.zeros(256, 0, dtype=torch.uint8, device=dev),
                torch.zeros(256, 0, dtype=torch.uint8, device=dev), torch.ones(2, device=dev), C,
                beta=2.0)
    assert np.array_equal(host(C), 2.0 * C0)


def test_fp8q_refusals(dev):
    from pico_amd import _lib

    L = _lib.hip_lib()
    Q = torch.zeros(256, 128, dtype=torch.uint8, device=dev)
    C = torch.zeros(4, 4, device=dev)
    sc = torch.ones(2, device=dev)
    X = torch.zeros(4, 100, device=dev)
    # row stride below K rounded up to 64
    assert L.pk_gemm_fp8q_f32(4, 4, 100, 1.0, Q.data_ptr(), 64, Q.data_ptr(), 128, sc.data_ptr(),
                              0.0, C.data_ptr(), 4, None) != 0
    assert L.pk_fp8_quantize_f32(4, 100, X.data_ptr(), 100, 0, sc.data_ptr(), Q.data_ptr(), 100,
                                 None) != 0
    # misaligned operand
    assert L.pk_gemm_fp8q_f32(4, 4, 64, 1.0, Q.data_ptr() + 8, 128, Q.data_ptr(), 128,
                              sc.data_ptr(), 0.0, C.data_ptr(), 4, None) != 0
    with pytest.raises(PkError):  # K rounded up to 64 is 128: ldq 100 refused by the library
        from pico_amd._lib import check
        check("pk_fp8_quantize_f32", L.pk_fp8_quantize_f32(
            4, 100, X.data_ptr(), 100, 0, sc.data_ptr(), Q.data_ptr(), 100, None))
    with pytest.raises(ValueError):
        K.gemm_fp8q(4, 4, 100, Q[:, :64], Q, sc, C)


# ---- MX8: e4m3 with an E8M0 scale per 32 values of a row -------------------

def mx8_decode(Q, R, Kd):
    """an MX8 buffer (pk_mx8_bytes layout) -> float64 [R, Kd], plus the scale
    bytes [Rp, Kp / 32] and the raw values [Rp, Kp]"""
    Rp, Kp = -(-R // 256) * 256, -(-Kd // 128) * 128
    Q = np.asarray(Q)
    vals = Q[:Rp * Kp].reshape(Rp, Kp)
    S = Q[Rp * Kp:Rp * Kp + Rp * Kp // 32].reshape(Kp // 64, Rp, 2)
    S = S.transpose(1, 0, 2).reshape(Rp, Kp // 32).astype(np.int64)
    X = e4m3_decode(vals) * np.exp2(np.repeat(S - 127, 32, axis=1).astype(np.float64))
    return X[:R, :Kd], S, vals


def _mixed(R, Kd, seed):
    """rows of uniform values whose 32-value blocks have magnitudes 2^-40..2^40"""
    rng = np.random.default_rng(seed)
    X = rng.uniform(-1, 1, (R, Kd)).astype(np.float32)
    nb = -(-Kd // 32)
    mag = np.exp2(rng.integers(-40, 41, (R, nb))).astype(np.float32)
    return (X * np.repeat(mag, 32, axis=1)[:, :Kd]).astype(np.float32)


@pytest.mark.parametrize("R,Kd", [(1, 1), (70, 130), (256, 128), (300, 1000)])
def test_mx8_quantize_scales_and_values(dev, R, Kd):
    X = _mixed(R, Kd, R + Kd)
    X.ravel()[:3] = [448.0, -449.0, 0.0][:min(3, X.size)]
    if R > 1:
        X[1, :] = 0.0  # all-zero blocks: scale 2^0
    Q = host(K.mx8_quantize(cu(X), False))
    Xd, S, vals = mx8_decode(Q, R, Kd)
    Rp, Kp = vals.shape
    Xp = np.zeros((Rp, Kp), np.float64)
    Xp[:R, :Kd] = X
    amax = np.abs(Xp).reshape(Rp, Kp // 32, 32).max(axis=2)
    e = S - 127
    # the defining property: the smallest power of two that brings the block within 448
    nz = amax > 0
    assert np.all(amax[nz] * np.exp2(-e[nz].astype(np.float64)) <= 448.0)
    assert np.all(amax[nz] * np.exp2(-(e[nz] - 1).astype(np.float64)) > 448.0)
    assert np.all(e[~nz] == 0)
    # each value is e4m3 of x * 2^-e (nearest even), byte for byte as torch encodes it
    scaled = (Xp * np.exp2(-np.repeat(e, 32, axis=1).astype(np.float64))).astype(np.float32)
    assert np.array_equal(e4m3_decode(vals), e4m3_round(scaled).astype(np.float64))
    tq = torch.from_numpy(np.clip(scaled, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8)
    assert np.array_equal(vals, tq.numpy())
    assert not vals[R:].any() and not vals[:, Kd:].any()
    # each block keeps e4m3's relative precision, whatever its magnitude
    big = np.abs(Xp[:R, :Kd]) >= np.repeat(amax, 32, axis=1)[:R, :Kd] / 8
    assert np.all(np.abs(Xd - X)[big] <= np.abs(X)[big] * 2.0 ** -4 + 1e-300)


@pytest.mark.parametrize("R,Kd", [(1, 5), (130, 70), (512, 256)])
def test_mx8_quantize_transposed_read(dev, R, Kd):
    X = _mixed(Kd, R, 9)  # op(X) = X^T is [R, Kd]
    Qt = host(K.mx8_quantize(cu(X), True))
    Qn = host(K.mx8_quantize(cu(np.ascontiguousarray(X.T)), False))
    assert np.array_equal(Qt, Qn)


def _mx_product(dev, X, Y, alpha=1.0, beta=0.0, Xadd=None, C0=None):
    M, Kd = X.shape
    N = Y.shape[1]
    A8 = K.mx8_quantize(cu(X), False)
    B8 = K.mx8_quantize(cu(Y), True)
    C = torch.full((M, N), float("nan"), device=dev) if C0 is None else cu(C0)
    K.gemm_mx8(M, N, Kd, A8, B8, C, alpha=alpha, beta=beta,
               X=None if Xadd is None else cu(Xadd))
    return host(C), host(A8), host(B8)


@pytest.mark.parametrize("M,N,Kd", SHAPES)
def test_mx8_gemm_integers_bitexact(dev, M, N, Kd):
    """integers of magnitude <= 16 have at most 4 significant bits: exact in
    e4m3 under any power-of-two block scale, so the product is exact"""
    rng = np.random.default_rng(M * 5 + N + Kd)
    X = rng.integers(-16, 17, (M, Kd)).astype(np.float32)
    Y = rng.integers(-16, 17, (Kd, N)).astype(np.float32)
    ref = (X.astype(np.float64) @ Y.astype(np.float64)).astype(np.float32)
    C, _, _ = _mx_product(dev, X, Y)
    assert np.array_equal(C, ref)
    C, _, _ = _mx_product(dev, X, Y, alpha=-1.0, beta=1.0, C0=ref)
    assert not np.any(C)


@pytest.mark.parametrize("M,N,Kd", [(1024, 1024, 1024), (300, 257, 70), (512, 768, 2048)])
def test_mx8_gemm_mixed_magnitudes(dev, M, N, Kd):
    """blocks of magnitude 2^-40..2^40: the product equals the float64 product
    of the decoded operands within fp32 summation error, where one tensor-wide
    scale would flush all but the largest blocks to zero"""
    X = _mixed(M, Kd, 3 * M + Kd)
    Y = _mixed(N, Kd, 5 * N + Kd).T.copy()
    C, A8, B8 = _mx_product(dev, X, Y)
    Xd, _, _ = mx8_decode(A8, M, Kd)
    Yd, _, _ = mx8_decode(B8, N, Kd)
    assert gemm_err(C, Xd, Yd.T) <= TOL
    assert gemm_err(C, X, Y) < 2 ** -3


def test_mx8_gemm_epilogue_adds_x(dev):
    M, N, Kd = 300, 520, 200
    X = O.uniform(M * Kd, 1).reshape(M, Kd)
    Y = O.uniform(Kd * N, 2).reshape(Kd, N)
    A8, B8 = K.mx8_quantize(cu(X), False), K.mx8_quantize(cu(Y), True)
    P = torch.empty(M, N, device=dev)
    K.gemm_mx8(M, N, Kd, A8, B8, P)
    Pn = host(P)
    R = O.uniform(M * N, 3).reshape(M, N)
    b = O.uniform(N, 4)
    for Xadd, want in ((R, 2.0 * Pn + 0.5 * R), (b, 2.0 * Pn + 0.5 * b[None, :])):
        C = torch.full((M, N), float("nan"), device=dev)
        K.gemm_mx8(M, N, Kd, A8, B8, C, alpha=2.0, beta=0.5, X=cu(Xadd))
        got = host(C)
        assert np.max(np.abs(got - want)) <= 1e-6 * np.max(np.abs(want))
    C = cu(R)
    K.gemm_mx8(M, N, Kd, A8, B8, C, beta=1.0)  # accumulate into C
    assert np.max(np.abs(host(C) - (Pn + R))) <= 1e-6 * np.max(np.abs(Pn + R))
    # beta 0: X is not read (NaN there stays out of C)
    C = torch.empty(M, N, device=dev)
    K.gemm_mx8(M, N, Kd, A8, B8, C, beta=0.0,
               X=torch.full((M, N), float("nan"), device=dev))
    assert np.array_equal(host(C), Pn)


def test_mx8_refusals(dev):
    from pico_amd import _lib

    L = _lib.hip_lib()
    Q = torch.zeros(K.mx8_bytes(256, 128) + 16, dtype=torch.uint8, device=dev)
    C = torch.zeros(4, 4, device=dev)
    X = torch.zeros(4, 100, device=dev)
    assert L.pk_mx8_quantize_f32(4, 100, X.data_ptr(), 100, 0, Q.data_ptr() + 8, None) != 0
    assert L.pk_mx8_quantize_f32(4, 100, X.data_ptr(), 99, 0, Q.data_ptr(), None) != 0
    assert L.pk_gemm_mx8_f32(4, 4, 100, 1.0, Q.data_ptr() + 4, Q.data_ptr(), 0.0, None, 0,
                             C.data_ptr(), 4, None) != 0
    assert L.pk_gemm_mx8_f32(4, 4, 100, 1.0, Q.data_ptr(), Q.data_ptr(), 1.0, None, 0,
                             C.data_ptr(), 4, None) != 0
    assert L.pk_gemm_mx8_f32(4, 4, 100, 1.0, Q.data_ptr(), Q.data_ptr(), 0.0, None, 0,
                             C.data_ptr(), 3, None) != 0


@pytest.mark.parametrize("M,N,Kd", [(768, 768, 8192), (2048, 768, 8192), (768, 2304, 8192),
                                    (8192, 768, 32000), (300, 200, 5000)])
def test_mx8_gemm_k_split(dev, M, N, Kd):
    """a split K (the planes summed in order by a second kernel, the last split
    taking the slices that remain): integers exact, and uniform operands equal
    to the unsplit product within fp32 summation error"""
    tm, tn, splits = K.mx8_plan(M, N, Kd)
    assert (tm, tn) in ((256, 256), (256, 128), (128, 256), (128, 128))
    ws = torch.empty(K.mx8_workspace(M, N, Kd) // 4 + 1, device=dev)
    assert (splits > 1) == (K.mx8_workspace(M, N, Kd) > 0)
    rng = np.random.default_rng(M + N + Kd)
    X = rng.integers(-16, 17, (M, Kd)).astype(np.float32)
    Y = rng.integers(-16, 17, (Kd, N)).astype(np.float32)
    A8, B8 = K.mx8_quantize(cu(X), False), K.mx8_quantize(cu(Y), True)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm_mx8(M, N, Kd, A8, B8, C, ws=ws)
    ref = (X.astype(np.float64) @ Y.astype(np.float64)).astype(np.float32)
    assert np.array_equal(host(C), ref)
    # alpha, beta and a row X through the split's reduction
    b = O.uniform(N, 12)
    K.gemm_mx8(M, N, Kd, A8, B8, C, alpha=0.5, beta=2.0, X=cu(b), ws=ws)
    want = (0.5 * ref.astype(np.float64) + 2.0 * b[None, :].astype(np.float64))
    assert np.max(np.abs(host(C) - want)) <= 1e-6 * np.max(np.abs(want))
    Xu = O.uniform(M * Kd, 13).reshape(M, Kd)
    Yu = O.uniform(Kd * N, 14).reshape(Kd, N)
    A8, B8 = K.mx8_quantize(cu(Xu), False), K.mx8_quantize(cu(Yu), True)
    Cs, Cu = torch.empty(M, N, device=dev), torch.empty(M, N, device=dev)
    K.gemm_mx8(M, N, Kd, A8, B8, Cs, ws=ws)
    K.gemm_mx8(M, N, Kd, A8, B8, Cu)  # no workspace: unsplit
    Xd, _, _ = mx8_decode(host(A8), M, Kd)
    Yd, _, _ = mx8_decode(host(B8), N, Kd)
    assert gemm_err(host(Cs), Xd, Yd.T) <= TOL
    assert gemm_err(host(Cs), Xd, Yd.T, C_ref=host(Cu).astype(np.float64)) <= TOL


@pytest.mark.parametrize("M,N", [(1, 1), (70, 130), (256, 128), (300, 1000), (8192, 768), (130, 2304)])
def test_mx8_dual_cast_equals_two_casts(dev, M, N):
    """one read, both casts: byte for byte the row cast of X and the cast of
    X^T, padding and scales included"""
    X = _mixed(M, N, M + 3 * N)
    dX = cu(X)
    QR, QT = K.mx8_quantize2(dX)
    assert np.array_equal(host(QR), host(K.mx8_quantize(dX, False)))
    assert np.array_equal(host(QT), host(K.mx8_quantize(dX, True)))
    # a strided view: the row stride is honoured
    wide = cu(np.concatenate([X, X[:, :N // 2 + 1] * 3.0], axis=1))
    QR2, QT2 = K.mx8_quantize2(wide[:, :N])
    assert np.array_equal(host(QR2), host(QR)) and np.array_equal(host(QT2), host(QT))
