"""fp8 matrix products (pk_gemm_fp8_f32, PICO_MATMUL_FP8): outside the fp32
parity contract, so pinned against what the arithmetic fixes, as the bf16
products are (tests/test_bf16_gpu.py).

* e4m3 is OCP FP8 E4M3 (exponent bias 7, 3 mantissa bits, largest finite 448,
  subnormals down to 2^-9).  The kernel clamps to +-448 and rounds to nearest
  even; `e4m3_round` below restates that from the format's definition, and is
  pinned by known values (ties to even, subnormals, clamping).  A product with
  K = 1 against a ones row returns each rounded operand exactly, which checks
  the GPU conversion against that restatement value by value.
* A product of two e4m3 values is exact in fp32, so the GPU result must equal
  the float64 product of the host-rounded operands up to fp32 summation error
  (the fp32 GEMM's 1e-4 normalised bound), and sit measurably away from the
  unrounded product (an fp8-sized error).
* Integers of magnitude <= 16 are exact in e4m3: bit-exact, every tile shape,
  layout and edge path.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import kernels as K
from pico_amd.pico import Pico
from tests._util import gemm_err

pytestmark = pytest.mark.gpu
TOL = 1e-4


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def e4m3_round(x):
    """float32 -> e4m3 (clamped to +-448, nearest even) -> float32"""
    x = np.clip(np.asarray(x, np.float64), -448.0, 448.0)
    ax = np.abs(x)
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(ax > 0, ax, 1.0)))
    e = np.maximum(e, -6.0)  # below 2^-6 the spacing stays 2^-9 (subnormals)
    q = np.exp2(e - 3.0)
    r = np.rint(x / q) * q  # rint: half to even
    return np.clip(r, -448.0, 448.0).astype(np.float32)


def test_e4m3_rounding_helper_known_values():
    x = np.array([1.0, 1.0625, 1.07, 1.1875, -3.3, 448.0, 460.0, -1e6, 240.0, 2 ** -9,
                  2 ** -10, 0.75 * 2 ** -9, 2 ** -7 + 2 ** -10, 0.0], np.float32)
    want = [1.0, 1.0, 1.125, 1.25, -3.25, 448.0, 448.0, -448.0, 240.0, 2 ** -9,
            0.0, 2 ** -9, 2 ** -7, 0.0]
    assert e4m3_round(x).tolist() == want


def test_fp8_conversion_matches_the_format(dev):
    """C = A . ones(1, 1): each output is the kernel's e4m3 rounding of A"""
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.uniform(-500, 500, 2000), rng.uniform(-1, 1, 2000), rng.uniform(-0.02, 0.02, 1000),
        np.array([0.0, 1.0625, 1.1875, 2 ** -10, 0.75 * 2 ** -9, 448.0, 449.0, 1e9, -1e9])])
    vals = vals.astype(np.float32)
    A = vals.reshape(-1, 1)
    C = torch.full((A.shape[0], 1), float("nan"), device=dev)
    K.gemm_fp8("N", "N", cu(A), cu(np.ones((1, 1))), C)
    assert np.array_equal(host(C)[:, 0], e4m3_round(vals))


def _ops(ta, tb, M, N, Kd, seed, integer=False):
    if integer:
        rng = np.random.default_rng(seed)
        A = rng.integers(-16, 17, (M, Kd)).astype(np.float32)
        B = rng.integers(-16, 17, (Kd, N)).astype(np.float32)
    else:
        A = O.uniform(M * Kd, seed).reshape(M, Kd)
        B = O.uniform(Kd * N, seed + 1).reshape(Kd, N)
    return A, B, (np.ascontiguousarray(A.T) if ta == "T" else A), \
        (np.ascontiguousarray(B.T) if tb == "T" else B)


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,Kd", [(4096, 4096, 512), (1000, 1376, 516), (8192, 768, 768),
                                    (200, 136, 70), (64, 128, 784)])
def test_fp8_gemm_equals_product_of_rounded_operands(dev, ta, tb, M, N, Kd):
    A, B, As, Bs = _ops(ta, tb, M, N, Kd, seed=M + N + Kd)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm_fp8(ta, tb, cu(As), cu(Bs), C)
    Cn = host(C)
    assert gemm_err(Cn, e4m3_round(A), e4m3_round(B)) <= TOL
    e = gemm_err(Cn, A, B)
    assert 1e-3 < e < 2 ** -3  # fp8-sized, not bf16- or fp32-sized


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,Kd", [(4096, 4096, 256), (4000, 4000, 200), (8192, 768, 768),
                                    (1024, 1024, 1024), (130, 257, 70), (64, 10, 784)])
def test_fp8_gemm_integers_bitexact(dev, ta, tb, M, N, Kd):
    A, B, As, Bs = _ops(ta, tb, M, N, Kd, seed=3 * M + N + Kd, integer=True)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm_fp8(ta, tb, cu(As), cu(Bs), C)
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    assert np.array_equal(host(C), ref)
    C = cu(ref.copy())
    K.gemm_fp8(ta, tb, cu(As), cu(Bs), C, alpha=-1.0, beta=1.0)
    assert not np.any(host(C))


def test_fp8_gemm_split_k_workspace(dev):
    M, N, Kd = 768, 768, 8192
    A, B, As, Bs = _ops("T", "N", M, N, Kd, seed=11)
    ws = torch.empty(K.gemm_workspace(M, N, Kd) // 4 + 1, device=dev)
    C1 = torch.empty(M, N, device=dev)
    C2 = torch.empty(M, N, device=dev)
    K.gemm_fp8("T", "N", cu(As), cu(Bs), C1, ws=ws)
    K.gemm_fp8("T", "N", cu(As), cu(Bs), C2, ws=ws)
    assert np.array_equal(host(C1), host(C2))
    assert gemm_err(host(C1), e4m3_round(A), e4m3_round(B)) <= TOL


def test_fp8_scales_are_the_largest_safe_powers_of_two(dev):
    from pico_amd import _lib

    L = _lib.hip_lib()
    A = cu(O.uniform(300 * 70, 3).reshape(300, 70) * 3e-5)
    B = cu(O.normal(80 * 50, 4).reshape(80, 50) * 1000.0)
    Z = torch.zeros(7, 9, device=dev)
    sc = torch.full((2,), float("nan"), device=dev)
    for X, Y in ((A, B), (B, Z)):
        _lib.check("pk_fp8_scales_f32", L.pk_fp8_scales_f32(
            X.shape[0], X.shape[1], X.data_ptr(), X.shape[1], Y.shape[0], Y.shape[1],
            Y.data_ptr(), Y.shape[1], sc.data_ptr(), None))
        got = host(sc)
        for s_, M_ in zip(got, (X, Y)):
            amax = float(M_.abs().max())
            if amax == 0.0:
                assert s_ == 1.0
            else:
                assert np.log2(s_) == np.floor(np.log2(s_))  # a power of two
                assert 224.0 < amax * s_ <= 448.0


def test_fp8_scales_of_extreme_magnitudes_stay_finite(dev):
    """The scale's exponent is held to [-63, 63]: operands of magnitude 1e-37
    (448 / amax overflows float), 1e-20 and near float's largest (1e38) all get
    finite power-of-two scales whose product and its reciprocal are finite
    normals, and a scaled product of two tiny operands is neither NaN nor
    flushed to zero by the descale."""
    from pico_amd import _lib

    L = _lib.hip_lib()
    sc = torch.full((2,), float("nan"), device=dev)
    cases = [(1e-37, 1e-37), (1e-20, 3e-21), (2.0, 5e-38), (1e38, 1e38), (3e21, 1e-30)]
    for amax_a, amax_b in cases:
        A = cu(np.full((4, 8), amax_a, np.float32))
        B = cu(np.full((8, 4), amax_b, np.float32))
        _lib.check("pk_fp8_scales_f32", L.pk_fp8_scales_f32(
            4, 8, A.data_ptr(), 8, 8, 4, B.data_ptr(), 4, sc.data_ptr(), None))
        got = host(sc).astype(np.float64)
        amax = (float(np.float32(amax_a)), float(np.float32(amax_b)))
        for s_, m_ in zip(got, amax):
            e = np.log2(s_)
            assert np.isfinite(s_) and e == np.floor(e) and -63 <= e <= 63, (amax_a, amax_b)
            # the largest power of two keeping amax within e4m3, unless clamped
            want = min(max(np.floor(np.log2(448.0 / m_)), -63), 63)
            assert e == want, (m_, e, want)
        prod = np.float32(got[0]) * np.float32(got[1])
        assert np.isfinite(prod) and prod > 0 and np.isfinite(np.float32(1.0) / prod)
    # two operands of 1e-17: scaled by 2^63 each (448 / 1e-17 would want 2^65),
    # their product, 32 * 1e-34 (a normal float), comes back through the
    # descale 2^-126 exactly, not as 0 or NaN
    A = cu(np.full((32, 32), 1e-17, np.float32))
    _lib.check("pk_fp8_scales_f32", L.pk_fp8_scales_f32(
        32, 32, A.data_ptr(), 32, 32, 32, A.data_ptr(), 32, sc.data_ptr(), None))
    C = torch.full((32, 32), float("nan"), device=dev)
    _lib.check("pk_gemm_add_f32", L.pk_gemm_add_f32(
        b"N", b"N", 32, 32, 32, 1.0, A.data_ptr(), 32, A.data_ptr(), 32, 0.0, None, 32,
        C.data_ptr(), 32, 3, sc.data_ptr(), None, 0, None))
    s0 = float(host(sc)[0])
    assert s0 == 2.0 ** 63
    a8 = float(e4m3_round(np.array([np.float32(1e-17) * s0], np.float32))[0]) / s0
    want = np.float32(32 * a8 * a8)
    got = host(C)
    assert np.isfinite(got).all() and np.all(got > 0)
    assert np.max(np.abs(got - want)) <= 1e-4 * want


def test_fp8_scaled_product_keeps_small_operands(dev):
    """gradient-sized operands (|x| ~ 1e-5, below e4m3's smallest subnormal)
    through the scaled fp8 product: the result equals the product of the
    host-rounded scaled operands, divided by the scales, within the fp32
    summation bound -- and is not flushed to zero"""
    from pico_amd import _lib

    L = _lib.hip_lib()
    M, N, Kd = 256, 192, 384
    A = O.uniform(M * Kd, 21).reshape(M, Kd) * 2e-5
    B = O.uniform(Kd * N, 22).reshape(Kd, N) * 0.02
    dA, dB = cu(A), cu(B)
    sc = torch.empty(2, device=dev)
    _lib.check("pk_fp8_scales_f32", L.pk_fp8_scales_f32(M, Kd, dA.data_ptr(), Kd, Kd, N,
                                                        dB.data_ptr(), N, sc.data_ptr(), None))
    C = torch.full((M, N), float("nan"), device=dev)
    _lib.check("pk_gemm_add_f32", L.pk_gemm_add_f32(
        b"N", b"N", M, N, Kd, 1.0, dA.data_ptr(), Kd, dB.data_ptr(), N, 0.0, None, N,
        C.data_ptr(), N, 3, sc.data_ptr(), None, 0, None))
    sa, sb = host(sc)
    Ar = e4m3_round(A * sa).astype(np.float64) / sa
    Br = e4m3_round(B * sb).astype(np.float64) / sb
    Cn = host(C)
    assert gemm_err(Cn, Ar, Br) <= TOL
    assert 1e-3 < gemm_err(Cn, A, B) < 2 ** -3  # fp8-sized, and not all zero
    # unscaled, the same operands mostly flush to zero
    C0 = torch.empty(M, N, device=dev)
    K.gemm_fp8("N", "N", dA, dB, C0)
    assert np.mean(host(C0) == 0.0) > 0.9


def _cos(a, b):
    return float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30))


def test_pico_matmul_fp8_precision(dev):
    """a transformer step with PICO_MATMUL_FP8 (operands scaled per product):
    the loss stays near the fp32 one, every gradient points the same way
    (e4m3 keeps 4 significant bits), and bf16 (8 bits) stays closer to fp32
    than fp8 does"""
    P = Pico()
    cfg = dict(vocab=96, d_model=64, n_layers=2, n_heads=2, d_ff=160, batch=2, seq_len=64)
    seq = O.labels(cfg["batch"] * (cfg["seq_len"] + 1), 78, cfg["vocab"]).reshape(2, -1)
    tok, tgt = seq[:, :-1].ravel(), seq[:, 1:].ravel()
    out = {}
    for prec in (0, 1, 3):
        assert P.lib.pico_set_matmul_precision(prec) == 0
        model = P.gpt_init(cfg, 4)
        with P.arena(1 << 26):
            loss = P.gpt_loss(model, tok, tgt)
            P.backward(loss)
            out[prec] = (float(P.data(loss)[0]), [P.grad(t) for t in P.gpt_params(model)])
        P.gpt_free(model)
    assert P.lib.pico_set_matmul_precision(0) == 0
    (l32, g32), (l16, g16), (l8, g8) = out[0], out[1], out[3]
    assert l8 != l32 and abs(l8 - l32) <= 5e-2 * abs(l32)
    cos8 = [_cos(a, b) for a, b in zip(g32, g8)]
    cos16 = [_cos(a, b) for a, b in zip(g32, g16)]
    assert min(cos8) > 0.9, cos8
    assert np.mean(cos16) > np.mean(cos8)
