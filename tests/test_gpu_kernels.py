"""GPU parity of every pk_* launcher against the CPU oracle (seeded inputs).

Bar: bit-exact where the arithmetic is exact or order-free (integer-valued
GEMMs, add/sub/mul and their gradients, relu, SGD, gathers, argmax); otherwise
the north-star tolerance, max relative error <= 1e-4 (GEMM: the
componentwise-normalised error of tests/_util.gemm_err).
"""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import kernels as K
from tests._util import gemm_err, max_rel, row_err

pytestmark = pytest.mark.gpu
TOL = 1e-4
GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_ops.npz"))


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _op(x, t):
    return x.T if t == "T" else x


def _operands(ta, tb, M, N, Kd, seed, integer=False):
    if integer:
        rng = np.random.default_rng(seed)
        A = rng.integers(-8, 9, (M, Kd)).astype(np.float32)
        B = rng.integers(-8, 9, (Kd, N)).astype(np.float32)
    else:
        A = O.uniform(M * Kd, seed).reshape(M, Kd)
        B = O.uniform(Kd * N, seed + 1).reshape(Kd, N)
    As = np.ascontiguousarray(A.T) if ta == "T" else A
    Bs = np.ascontiguousarray(B.T) if tb == "T" else B
    return A, B, As, Bs


# ----------------------------------------------------------------- GEMM
def test_gemm_reference_kats(dev):
    A = cu(np.array([[1, 2, 3], [4, 5, 6]], np.float32))
    B = cu(np.array([[7, 8], [9, 10], [11, 12]], np.float32))
    C = torch.zeros(2, 2, device=dev)
    assert host(K.gemm("N", "N", A, B, C)).tolist() == [[58, 64], [139, 154]]
    # pico_matmul_backward with dC = ones (tests/test_autograd.c:382)
    dC = torch.ones(2, 2, device=dev)
    dA = torch.zeros(2, 3, device=dev)
    dB = torch.zeros(3, 2, device=dev)
    K.gemm("N", "T", dC, B, dA, beta=1.0)
    K.gemm("T", "N", A, dC, dB, beta=1.0)
    assert host(dA).ravel().tolist() == [15, 19, 23, 15, 19, 23]
    assert host(dB).ravel().tolist() == [5, 5, 7, 7, 9, 9]


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,Kd", [(64, 128, 784), (64, 10, 128), (130, 257, 70), (256, 256, 256),
                                    (1, 1, 1), (3, 5, 0)])
def test_gemm_integer_bitexact(dev, ta, tb, M, N, Kd):
    A, B, As, Bs = _operands(ta, tb, M, N, Kd, seed=M + N + Kd, integer=True)
    C = torch.full((M, N), float("nan"), device=dev)  # beta = 0 must not read C
    K.gemm(ta, tb, cu(As), cu(Bs), C)
    ref = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)
    assert np.array_equal(host(C), ref)


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,Kd", [(512, 512, 512), (512, 512, 1024), (256, 256, 256),
                                    (512, 256, 1536), (256, 512, 384), (96, 64, 128),
                                    (32, 480, 2048)])
def test_gemm_small_products(dev, ta, tb, M, N, Kd):
    """Outputs of at most 256 tiles of 32 x 32 (and fewer 64 x 64 tiles than
    CUs) run one tile per workgroup with K split over its waves: sixteen when
    K is 1024 (two slices of 32 per wave, both in flight), eight when K/256 is
    whole (2, 1, 6 and 8 slices per wave here, 2, 1, 2 and 4 in flight), else
    four (3 and 1 slices, 1 in flight).  Integer operands bit for
    bit, the beta accumulate exact, a separate X (pk_gemm_add_f32), and uniform
    operands within the fp64 bound"""
    from pico_amd import _lib
    A, B, As, Bs = _operands(ta, tb, M, N, Kd, seed=M + 13 * N + Kd, integer=True)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm(ta, tb, cu(As), cu(Bs), C)
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    assert np.array_equal(host(C), ref)
    C = cu(ref.copy())
    K.gemm(ta, tb, cu(As), cu(Bs), C, alpha=-1.0, beta=1.0)  # C - A.B = 0 exactly
    assert not np.any(host(C))
    if (ta, tb) == ("N", "N"):  # a separate X is built for A.B only
        X = O.uniform(M * N, 17).reshape(M, N)
        C = torch.full((M, N), float("nan"), device=dev)
        dA, dB, dX = cu(As), cu(Bs), cu(X)
        _lib.check("pk_gemm_add_f32", _lib.hip_lib().pk_gemm_add_f32(
            b"N", b"N", M, N, Kd, 0.5, dA.data_ptr(), Kd, dB.data_ptr(), N, 2.0, dX.data_ptr(), N,
            C.data_ptr(), N, 0, None, None, 0, None))
        assert np.array_equal(host(C), (0.5 * ref).astype(np.float32) + 2.0 * X)
    A, B, As, Bs = _operands(ta, tb, M, N, Kd, seed=M + N + 3 * Kd)
    C = torch.empty(M, N, device=dev)
    K.gemm(ta, tb, cu(As), cu(Bs), C)
    assert gemm_err(host(C), A, B) <= TOL


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,Kd", [(64, 128, 784), (64, 10, 128), (784, 128, 64), (64, 784, 128),
                                    (37, 45, 1001), (1, 1, 1), (130, 257, 70), (500, 33, 3)])
def test_gemm_small_edge_products(dev, ta, tb, M, N, Kd):
    """Small products whose sizes or strides are not whole tiles (the MLP's
    784 / 10 widths, K 784 = 24.5 slices, K 1 and 3) run on the edge kernel:
    masked 32-bit loads, waves taking slices w, w + W, ... (sixteen waves from
    12 slices up, else four), predicated stores.  Integer operands bit for bit
    with beta 0 (C starts NaN), the beta accumulate exact, a bias row added by
    pk_gemm_add_f32 with ldx 0, and uniform operands within the fp64 bound"""
    from pico_amd import _lib
    L = _lib.hip_lib()
    A, B, As, Bs = _operands(ta, tb, M, N, Kd, seed=M + 19 * N + Kd, integer=True)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm(ta, tb, cu(As), cu(Bs), C)
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    assert np.array_equal(host(C), ref)
    C = cu(ref.copy())
    K.gemm(ta, tb, cu(As), cu(Bs), C, alpha=-1.0, beta=1.0)
    assert not np.any(host(C))
    if (ta, tb) == ("N", "N"):
        x = np.random.default_rng(M + N).integers(-50, 50, N).astype(np.float32)
        C = torch.full((M, N), float("nan"), device=dev)
        dA, dB, dx = cu(As), cu(Bs), cu(x)
        _lib.check("pk_gemm_add_f32", L.pk_gemm_add_f32(
            b"N", b"N", M, N, Kd, 1.0, dA.data_ptr(), Kd, dB.data_ptr(), N, 1.0, dx.data_ptr(), 0,
            C.data_ptr(), N, 0, None, None, 0, None))
        assert np.array_equal(host(C), ref + x)
    A, B, As, Bs = _operands(ta, tb, M, N, Kd, seed=M + N + 5 * Kd)
    C = torch.empty(M, N, device=dev)
    K.gemm(ta, tb, cu(As), cu(Bs), C)
    assert gemm_err(host(C), A, B) <= TOL


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N")])
@pytest.mark.parametrize("n", [512, 1024, 2048])
def test_gemm_uniform_vs_fp64(dev, ta, tb, n):
    A, B, As, Bs = _operands(ta, tb, n, n, n, seed=100 + n)
    C = torch.empty(n, n, device=dev)
    K.gemm(ta, tb, cu(As), cu(Bs), C)
    assert gemm_err(host(C), A, B) <= TOL


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N")])
@pytest.mark.parametrize("n", [4096, 8192])
def test_gemm_large_sampled_rows(dev, ta, tb, n):
    # full-size product on the GPU; 32 sampled rows checked against fp64
    gen = torch.Generator(device="cpu").manual_seed(n)
    As = (torch.rand(n, n, generator=gen) * 2 - 1)
    Bs = (torch.rand(n, n, generator=gen) * 2 - 1)
    C = torch.empty(n, n, device=dev)
    K.gemm(ta, tb, As.cuda(), Bs.cuda(), C)
    Cn = host(C)
    A = As.numpy().T if ta == "T" else As.numpy()
    B = Bs.numpy().T if tb == "T" else Bs.numpy()
    rows = np.random.default_rng(n).choice(n, 32, replace=False)
    assert gemm_err(Cn[rows], A[rows], B) <= TOL


@pytest.mark.parametrize("ta,tb", [("T", "N"), ("N", "T"), ("N", "N")])
@pytest.mark.parametrize("M,N,Kd,split", [(768, 768, 8192, True), (768, 2048, 8192, True),
                                          (200, 136, 4000, True), (64, 128, 784, True),
                                          (64, 10, 256, False), (1024, 512, 768, False),
                                          (2048, 1024, 4096, True)])
def test_gemm_splitk(dev, ta, tb, M, N, Kd, split):
    # weight-gradient shapes and a tiny output with a long K: K split into
    # slices summed in a fixed order; short K, or an output the 64 x 64 tiles
    # already spread over the chip, stays unsplit.  2048 x 1024 with K 4096
    # splits as A^T.B only: A.B and A.B^T have two 64 x 64 tiles per CU and run
    # unsplit (the workspace size is the largest over layouts)
    need = K.gemm_workspace(M, N, Kd)
    assert (need > 0) == split
    A, B, As, Bs = _operands(ta, tb, M, N, Kd, seed=M + N, integer=True)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm_ex(ta, tb, cu(As), cu(Bs), C)
    # |entries| <= 8 and K <= 8192 keep every partial sum below 2^19, exact in
    # fp32 and in the float64 BLAS product used as the reference
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    assert np.array_equal(host(C), ref)
    A, B, As, Bs = _operands(ta, tb, M, N, Kd, seed=M + N + 1)
    C0 = O.uniform(M * N, 3).reshape(M, N)
    C = cu(C0.copy())
    K.gemm_ex(ta, tb, cu(As), cu(Bs), C, alpha=0.5, beta=1.0)
    Cn = host(C)
    assert gemm_err(Cn - C0, 0.5 * A, B) <= TOL
    C2 = cu(C0.copy())  # deterministic: the same call gives the same bits
    K.gemm_ex(ta, tb, cu(As), cu(Bs), C2, alpha=0.5, beta=1.0)
    assert np.array_equal(host(C2), Cn)
    small = torch.empty(1, device=dev)  # a workspace too small runs the product unsplit
    C3 = torch.empty(M, N, device=dev)
    K.gemm_ex(ta, tb, cu(As), cu(Bs), C3, ws=small)
    assert gemm_err(host(C3), A, B) <= TOL


def test_gemm_alpha_beta_accumulate(dev):
    M, N, Kd = 200, 136, 96
    A, B, As, Bs = _operands("N", "N", M, N, Kd, seed=5)
    C0 = O.uniform(M * N, 77).reshape(M, N)
    C = cu(C0.copy())
    K.gemm("N", "N", cu(As), cu(Bs), C, alpha=0.5, beta=1.0)
    ref = 0.5 * (A.astype(np.float64) @ B) + C0
    assert max_rel(host(C), ref) <= TOL
    # a pico_transpose_2d view maps to 'T': A^T stored contiguously as [K, M]
    C2 = torch.empty(M, N, device=dev)
    K.gemm("T", "N", cu(np.ascontiguousarray(A.T)), cu(B), C2)
    assert gemm_err(host(C2), A, B) <= TOL


@pytest.mark.parametrize("causal", [0, 1, 2, 3])
def test_gemm_batched_causal(dev, causal):
    # two-level batch (2 sequences x 3 heads) addressed inside token-major buffers
    Bn, H, T, hd = 2, 3, 256, 64
    D = H * hd
    q = O.uniform(Bn * T * D, 1).reshape(Bn * T, D)
    k = O.uniform(Bn * T * D, 2).reshape(Bn * T, D)
    S = torch.zeros(Bn * H * T * T, device=dev)
    if causal in (0, 1):
        K.gemm_batched("N", "T", T, T, hd, 0.5, cu(q), D, T * D, hd, cu(k), D, T * D, hd, 0.0, S,
                       T, H * T * T, T * T, Bn * H, H, causal)
        Sn = host(S).reshape(Bn, H, T, T)
        for b in range(Bn):
            for h in range(H):
                Q = q[b * T:(b + 1) * T, h * hd:(h + 1) * hd].astype(np.float64)
                Kh = k[b * T:(b + 1) * T, h * hd:(h + 1) * hd].astype(np.float64)
                ref = 0.5 * Q @ Kh.T
                got = Sn[b, h]
                if causal == 1:
                    keep = np.tril(np.ones((T, T), bool))
                    got, ref = got[keep], ref[keep]
                assert max_rel(got, ref) <= TOL
    else:
        # op(A) triangular: lower for mode 2 (stored as is), upper for mode 3 (stored
        # transposed, read with 'T'); out = op(A) . V per head
        X = O.uniform(T * T, 3).reshape(T, T)
        Amat = np.tril(X) if causal == 2 else np.triu(X)
        store = Amat if causal == 2 else np.ascontiguousarray(Amat.T)
        Pb = np.broadcast_to(store, (Bn * H, T, T)).copy()
        out = torch.zeros(Bn * T, D, device=dev)
        ta = "N" if causal == 2 else "T"
        K.gemm_batched(ta, "N", T, hd, T, 1.0, cu(Pb), T, H * T * T, T * T, cu(q), D, T * D,
                       hd, 0.0, out, D, T * D, hd, Bn * H, H, causal)
        on = host(out)
        for b in range(Bn):
            for h in range(H):
                Vh = q[b * T:(b + 1) * T, h * hd:(h + 1) * hd].astype(np.float64)
                ref = Amat @ Vh
                assert max_rel(on[b * T:(b + 1) * T, h * hd:(h + 1) * hd], ref) <= TOL


def test_gemm_rejects_bad_arguments(dev):
    from pico_amd._lib import PkError

    A = torch.zeros(4, 4, device=dev)
    with pytest.raises(PkError):
        K.gemm_batched("X", "N", 4, 4, 4, 1.0, A, 4, 0, 0, A, 4, 0, 0, 0.0, A, 4, 0, 0, 1, 1)
    with pytest.raises(PkError):  # lda < K
        K.gemm_batched("N", "N", 4, 4, 8, 1.0, A, 4, 0, 0, A, 4, 0, 0, 0.0, A, 4, 0, 0, 1, 1)


# ---------------------------------------------------------- elementwise
# same shapes (float4 and per-element paths), biases broadcast over leading rows,
# broadcasts over trailing or interleaved dims (the general path), config-sized ones
BCAST_CASES = [((3, 5), (3, 5)), ((4, 6), (6,)), ((4, 6), (4, 1)), ((2, 3, 4), (3, 1)),
               ((7,), (1,)), ((5, 1, 3), (1, 4, 1)), ((16,), (16,)), ((19,), (19,)),
               ((64, 128), (128,)), ((3, 64, 10), (1, 10)), ((256, 768), (256, 768))]


@pytest.mark.parametrize("accumulate", [True, False])
@pytest.mark.parametrize("op", [0, 1, 2])
@pytest.mark.parametrize("sa,sb", BCAST_CASES)
def test_binary_and_grad_bitexact(dev, op, sa, sb, accumulate):
    a = O.normal(int(np.prod(sa)), 1).reshape(sa)
    b = O.normal(int(np.prod(sb)), 2).reshape(sb)
    name = ["add", "sub", "mul"][op]
    out = K.binary(name, cu(a), cu(b))
    assert np.array_equal(host(out), O.binary(op, a, b))
    g = O.normal(out.numel(), 3).reshape(out.shape)
    g.ravel()[::5] = -0.0  # a fresh grad is 0 + g: -0.0 becomes +0.0, as in pico
    if accumulate:  # += onto a nonzero grad
        ga0 = O.normal(a.size, 4).reshape(sa)
        gb0 = O.normal(b.size, 5).reshape(sb)
    else:
        ga0, gb0 = np.zeros(sa, np.float32), np.zeros(sb, np.float32)
    ga_ref, gb_ref = O.binary_bwd(op, a, b, g, ga0.copy(), gb0.copy())
    ga = cu(ga0.copy()) if accumulate else torch.full(sa, float("nan"), device=dev)
    gb = cu(gb0.copy()) if accumulate else torch.full(sb, float("nan"), device=dev)
    K.binary_bwd(name, 0, out.shape, sa, sb, cu(g), cu(b), ga, accumulate=accumulate)
    K.binary_bwd(name, 1, out.shape, sb, sa, cu(g), cu(a), gb, accumulate=accumulate)
    assert np.array_equal(np.signbit(host(ga)), np.signbit(ga_ref))
    assert np.array_equal(host(ga), ga_ref)
    assert np.array_equal(host(gb), gb_ref)


@pytest.mark.parametrize("op", range(6))
def test_unary_and_grad(dev, op):
    n = 1000
    x = O.uniform(n, 9, 0.05, 1.4)  # in every op's domain
    y = K.unary(list(K.UNARY_OPS)[op], cu(x), torch.empty(n, device=dev))
    assert row_err(host(y), O.unary(op, x)) <= 1e-6
    gy = O.normal(n, 10)
    gx0 = O.normal(n, 11)
    yref = O.unary(op, x)
    ref = O.unary_bwd(op, x, yref, gy, gx0.copy())
    gx = cu(gx0.copy())
    K.unary_bwd(list(K.UNARY_OPS)[op], cu(x), cu(yref), cu(gy), gx)
    assert max_rel(host(gx), ref) <= 1e-6


def test_relu_fill_sgd_bitexact(dev):
    x = O.normal(5003, 1)
    x[:4] = [np.nan, -0.0, 0.0, -1.0]
    y = K.relu(cu(x), torch.empty(5003, device=dev))
    assert np.array_equal(host(y), O.relu(x))
    gy, gx0 = O.normal(5003, 2), O.normal(5003, 3)
    gx = cu(gx0.copy())
    K.relu_bwd(cu(O.relu(x)), cu(gy), gx)
    assert np.array_equal(host(gx), O.relu_bwd(O.relu(x), gy, gx0.copy()))
    f = K.fill(torch.empty(777, device=dev), 1.0)
    assert np.all(host(f) == 1.0)
    p, g = O.normal(4099, 4), O.normal(4099, 5)
    pt = cu(p.copy())
    K.sgd(pt, cu(g), 0.01)
    assert np.array_equal(host(pt), O.sgd(p.copy(), g, 0.01))


def test_axpy_and_sum(dev):
    x, y0 = O.normal(3001, 1), O.normal(3001, 2)
    s = cu(np.array([0.25], np.float32))
    y = cu(y0.copy())
    K.axpy(2.0, cu(x), y, alpha_dev=s)
    assert max_rel(host(y), y0 + 0.5 * x) <= 1e-6
    out = torch.zeros(1, device=dev)
    K.reduce_sum(cu(x), out, scale=0.5)
    assert abs(host(out)[0] - 0.5 * x.astype(np.float64).sum()) <= 1e-4 * np.abs(x).sum()


def test_adamw_vs_oracle_and_golden(dev):
    lr, b1, b2, eps, wd = (float(v) for v in GOLD["adamw_hparams"])
    p = cu(GOLD["adamw_p0"].copy())
    m, v = torch.zeros_like(p), torch.zeros_like(p)
    for s in range(3):
        K.adamw(p, cu(GOLD["adamw_g"][s]), m, v, lr, b1, b2, eps, wd, s + 1)
        assert max_rel(host(p), GOLD["adamw_p"][s]) <= 1e-6
    n = 10007
    p0, g = O.normal(n, 1), O.normal(n, 2)
    ref = O.adamw(p0.copy(), g, np.zeros(n, np.float32), np.zeros(n, np.float32), 1e-3, 0.9,
                  0.999, 1e-8, 0.01, 1)
    pt = cu(p0.copy())
    K.adamw(pt, cu(g), torch.zeros_like(pt), torch.zeros_like(pt), 1e-3, 0.9, 0.999, 1e-8, 0.01, 1)
    assert np.array_equal(host(pt), ref)


# ------------------------------------------------------------ row kernels
@pytest.mark.parametrize("R,V", [(7, 37), (64, 10), (16, 8192), (8, 32000), (3, 40000),
                                 (4, 33000)])
def test_xent_vs_oracle(dev, R, V):
    z = O.normal(R * V, R + V, 0.0, 2.0).reshape(R, V)
    y = O.labels(R, 7, V)
    loss_ref, dz_ref = O.xent(z, y, scale=1.0 / R)
    rows = torch.empty(R, device=dev)
    dz = torch.empty(R, V, device=dev)
    K.xent_fwd_bwd(cu(z), cu(y), rows, dz, scale=1.0 / R)
    assert row_err(host(rows), loss_ref) <= TOL
    assert max_rel(host(dz), dz_ref) <= TOL
    dz2 = cu(dz_ref.copy())  # accumulate mode adds onto the existing gradient
    K.xent_fwd_bwd(cu(z), cu(y), None, dz2, scale=1.0 / R, accumulate=True)
    assert max_rel(host(dz2), 2 * dz_ref) <= TOL


def test_xent_golden_and_bad_labels(dev):
    z, y = GOLD["xent_z"], GOLD["xent_y"]
    rows = torch.empty(z.shape[0], device=dev)
    dz = torch.empty(z.shape, device=dev)
    K.xent_fwd_bwd(cu(z), cu(y), rows, dz, scale=1.0 / z.shape[0])
    assert row_err(host(rows), GOLD["xent_rows"]) <= TOL
    assert max_rel(host(dz), GOLD["xent_dz"]) <= TOL
    bad = y.copy()
    bad[0], bad[1] = -1, z.shape[1]
    K.xent_fwd_bwd(cu(z), cu(bad), rows, dz)
    r, d = host(rows), host(dz)
    assert np.isnan(r[0]) and np.isnan(r[1]) and not np.any(d[:2])


@pytest.mark.parametrize("R,V", [(64, 10), (1, 1), (7, 37), (1024, 64), (1000, 63), (64, 16),
                                 (1025, 10), (16, 8192)])
def test_xent_mean_equals_rows_then_sum(dev, R, V):
    """pk_xent_mean_f32 (one launch up to 1024 rows of 64 classes) gives the
    rows, gradient and mean of pk_xent_fwd_bwd_f32 + pk_reduce_sum_f32 bit for
    bit where those run the same per-row arithmetic (V not a multiple of 4, or
    above the one-launch sizes), and within the oracle's bound otherwise"""
    z = O.normal(R * V, R + 2 * V, 0.0, 2.0).reshape(R, V)
    y = O.labels(R, 9, V)
    y[0] = -1 if R > 1 else y[0]  # a bad label: NaN row, zero gradient
    rows0, dz0, out0 = torch.empty(R, device=dev), torch.empty(R, V, device=dev), torch.empty(1, device=dev)
    K.xent_fwd_bwd(cu(z), cu(y), rows0, dz0, scale=1.0 / R)
    K.reduce_sum(rows0, out0, 1.0 / R)
    rows1, dz1, out1 = torch.empty(R, device=dev), torch.empty(R, V, device=dev), torch.empty(1, device=dev)
    K.xent_mean(cu(z), cu(y), out1, rows1, dz1, scale=1.0 / R, mean_scale=1.0 / R)
    r0, r1, d0, d1 = host(rows0), host(rows1), host(dz0), host(dz1)
    if V % 4 or R > 1024 or V > 64:
        assert np.array_equal(r0, r1, equal_nan=True) and np.array_equal(d0, d1)
        assert np.array_equal(host(out0), host(out1), equal_nan=True)
    else:
        ok = ~np.isnan(r0)
        assert np.array_equal(np.isnan(r0), np.isnan(r1))
        assert row_err(r1[ok], r0[ok]) <= TOL and max_rel(d1, d0) <= TOL
    # accumulate: gradient and mean added onto what is there
    K.xent_mean(cu(z), cu(y), out1, None if R <= 1024 and V <= 64 else rows1, dz1, scale=1.0 / R,
                mean_scale=1.0 / R, accumulate=True, accumulate_out=True)
    assert max_rel(host(dz1), 2 * d1) <= TOL
    if R > 1:  # a NaN row makes the mean NaN
        assert np.isnan(host(out1)[0])


def test_xent_mean_refusals(dev):
    from pico_amd import _lib

    L = _lib.hip_lib()
    z = torch.zeros(2000, 10, device=dev)
    y = torch.zeros(2000, dtype=torch.int32, device=dev)
    out = torch.zeros(1, device=dev)
    # no out; rows above the one-launch sizes need loss_rows; a row stride below V
    assert L.pk_xent_mean_f32(64, 10, z.data_ptr(), 10, y.data_ptr(), None, None, 10, 1.0, 0, 1.0,
                              None, None) != 0
    assert L.pk_xent_mean_f32(2000, 10, z.data_ptr(), 10, y.data_ptr(), None, None, 10, 1.0, 0, 1.0,
                              out.data_ptr(), None) != 0
    assert L.pk_xent_mean_f32(64, 10, z.data_ptr(), 9, y.data_ptr(), None, None, 10, 1.0, 0, 1.0,
                              out.data_ptr(), None) != 0
    # R = 0: the mean of nothing is 0
    out.fill_(5.0)
    assert L.pk_xent_mean_f32(0, 10, z.data_ptr(), 10, y.data_ptr(), None, None, 10, 1.0, 0, 1.0,
                              out.data_ptr(), None) == 0
    assert host(out)[0] == 0.0


@pytest.mark.parametrize("R,V", [(6, 13), (100, 32000), (9, 7)])
def test_argmax_bitexact(dev, R, V):
    if (R, V) == (6, 13):
        x = GOLD["argmax_x"]
        ref = GOLD["argmax_idx"]
    else:
        x = O.normal(R * V, 5).reshape(R, V)
        x[0, V // 2] = x[0, V // 3] = 100.0  # tie: first wins
        ref = O.argmax(x)
    idx = torch.empty(R, dtype=torch.int32, device=dev)
    K.argmax(cu(x), idx)
    assert np.array_equal(host(idx), ref)


@pytest.mark.parametrize("R,C", [(5, 24), (64, 512), (33, 768), (16, 4096), (7, 10001), (3, 9000),
                                 (1030, 2048), (9, 2052), (5, 3072), (600, 8192)])
def test_rmsnorm_vs_oracle(dev, R, C):
    x = O.normal(R * C, 1).reshape(R, C)
    g = O.normal(C, 2, 1.0, 0.02)
    dy = O.normal(R * C, 3).reshape(R, C)
    y_ref, rstd_ref = O.rmsnorm_fwd(x, g, 1e-6)
    y, rstd = torch.empty(R, C, device=dev), torch.empty(R, device=dev)
    K.rmsnorm_fwd(cu(x), cu(g), y, rstd, 1e-6)
    assert max_rel(host(y), y_ref) <= TOL and row_err(host(rstd), rstd_ref) <= TOL
    dx0, dg0 = O.normal(R * C, 4).reshape(R, C), O.normal(C, 5)
    dx_ref, dg_ref = O.rmsnorm_bwd(x, g, rstd_ref, dy, dx0.copy(), dg0.copy())
    dx, dg = cu(dx0.copy()), cu(dg0.copy())
    K.rmsnorm_bwd(cu(x), cu(g), cu(rstd_ref), cu(dy), dx, dg, accum_dx=True, accum_dg=True)
    assert max_rel(host(dx), dx_ref) <= TOL and max_rel(host(dg), dg_ref) <= TOL
    # the accumulated term read from another buffer: the same bits, the source untouched
    src = cu(dx0.copy())
    dx2, dg2 = torch.full((R, C), float("nan"), device=dev), cu(dg0.copy())
    K.rmsnorm_bwd(cu(x), cu(g), cu(rstd_ref), cu(dy), dx2, dg2, accum_dg=True, dx_in=src)
    assert np.array_equal(host(dx2), host(dx)) and np.array_equal(host(dg2), host(dg))
    assert np.array_equal(host(src), dx0)
    # dg's reduction as a second call (the partial sums kept in the workspace)
    dx3, dg3 = torch.full((R, C), float("nan"), device=dev), cu(dg0.copy())
    ws = K.rmsnorm_bwd(cu(x), cu(g), cu(rstd_ref), cu(dy), dx3, None, dx_in=src,
                       keep_partials=True)
    assert np.array_equal(host(dg3), dg0)  # not touched yet
    K.rmsnorm_dg_reduce(R, C, ws, dg3, accum=True)
    assert np.array_equal(host(dx3), host(dx)) and np.array_equal(host(dg3), host(dg))
    dx, dg = torch.empty(R, C, device=dev), torch.empty(C, device=dev)  # overwrite mode
    K.rmsnorm_bwd(cu(x), cu(g), cu(rstd_ref), cu(dy), dx, dg)
    dx_ref, dg_ref = O.rmsnorm_bwd(x, g, rstd_ref, dy)
    assert max_rel(host(dx), dx_ref) <= TOL and max_rel(host(dg), dg_ref) <= TOL


@pytest.mark.parametrize("R,F", [(4, 33), (64, 1376), (128, 2048)])
def test_swiglu_vs_oracle(dev, R, F):
    a, u, dh = (O.normal(R * F, s).reshape(R, F) for s in (1, 2, 3))
    h = torch.empty(R, F, device=dev)
    K.swiglu_fwd(cu(a), cu(u), h)
    assert max_rel(host(h), O.swiglu_fwd(a, u)) <= TOL
    da0, du0 = O.normal(R * F, 4).reshape(R, F), O.normal(R * F, 5).reshape(R, F)
    da_ref, du_ref = O.swiglu_bwd(a, u, dh, da0.copy(), du0.copy())
    da, du = cu(da0.copy()), cu(du0.copy())
    K.swiglu_bwd(cu(a), cu(u), cu(dh), da, du, accum_da=True, accum_du=True)
    assert max_rel(host(da), da_ref) <= TOL and max_rel(host(du), du_ref) <= TOL


def _attn_case(dev, B, H, T, hd, q, k, v, do):
    D = H * hd
    o = torch.empty(B * T, D, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    P = torch.empty(B * H * T * T, device=dev)
    K.attn_fwd(B, H, cu(q), cu(k), cu(v), o, lse, P)
    o_ref, lse_ref = O.attn_fwd(B, H, q, k, v)
    assert max_rel(host(o), o_ref) <= TOL and max_rel(host(lse), lse_ref) <= TOL
    dq, dk, dv = (torch.empty(B * T, D, device=dev) for _ in range(3))
    ws = torch.empty(B * H * T * T, device=dev)
    K.attn_bwd(B, H, cu(q), cu(k), cu(v), P, cu(do), dq, dk, dv, ws)
    refs = O.attn_bwd(B, H, q, k, v, o_ref, lse_ref, do)
    for got, ref in zip((dq, dk, dv), refs):
        assert max_rel(host(got), ref) <= TOL


def test_attention_golden(dev):
    B, H = int(GOLD["att_B"]), int(GOLD["att_H"])
    _attn_case(dev, B, H, GOLD["att_q"].shape[0] // B, GOLD["att_q"].shape[1] // H,
               GOLD["att_q"], GOLD["att_k"], GOLD["att_v"], GOLD["att_do"])


@pytest.mark.parametrize("B,H,T,hd", [(2, 2, 128, 64), (1, 3, 256, 64), (1, 2, 200, 32)])
def test_attention_vs_oracle(dev, B, H, T, hd):
    D = H * hd
    q, k, v, do = (O.normal(B * T * D, s).reshape(B * T, D) for s in (1, 2, 3, 4))
    _attn_case(dev, B, H, T, hd, q, k, v, do)


@pytest.mark.parametrize("V,d,n", [(50, 6, 5000), (32000, 768, 8192), (7, 3, 1), (3, 64, 4097),
                                   (32000, 64, 100000), (1000, 16, 200000), (1 << 20, 8, 5000),
                                   (1, 4, 3000)])
def test_embedding_backward_deterministic_order(dev, V, d, n):
    # many repeats per id (n >> V), one id only (V = 1), keys of 1 to 3 radix
    # digits and sizes crossing the sort's 2048-key blocks: the same bits as the
    # position-ordered loop, every time; an accumulating call adds onto the
    # existing rows; out-of-range ids add nothing
    ids = O.labels(n, V + n, V)
    if n > 4:
        ids[::97] = -1
        ids[1::89] = V
    dout = O.normal(n * d, 7 + n).reshape(n, d)
    base = O.normal(V * d, 8).reshape(V, d)
    ref = O.embed_bwd(np.where((ids >= 0) & (ids < V), ids, 0)[(ids >= 0) & (ids < V)],
                      dout[(ids >= 0) & (ids < V)], base.copy())
    for _ in range(2):
        dt = cu(base.copy())
        K.embed_bwd(cu(ids), cu(dout), dt)
        assert np.array_equal(host(dt), ref)


def test_embedding(dev):
    V, d, n = 1000, 64, 513
    table = O.normal(V * d, 1).reshape(V, d)
    ids = O.labels(n, 2, V)
    out = torch.empty(n, d, device=dev)
    K.embed_fwd(cu(ids), cu(table), out)
    assert np.array_equal(host(out), O.embed_fwd(ids, table))
    dout = O.normal(n * d, 3).reshape(n, d)
    dt = torch.zeros(V, d, device=dev)
    K.embed_bwd(cu(ids), cu(dout), dt)
    # each row's contributions are added in position order, as the sequential loop does
    assert np.array_equal(host(dt), O.embed_bwd(ids, dout, np.zeros((V, d), np.float32)))
    out = torch.empty(GOLD["emb_ids"].size, GOLD["emb_table"].shape[1], device=dev)
    K.embed_fwd(cu(GOLD["emb_ids"]), cu(GOLD["emb_table"]), out)
    assert np.array_equal(host(out), GOLD["emb_out"].astype(np.float32))


# ------------------------------------------------------- fused attention (hd 64)
@pytest.mark.parametrize("B,H,T", [(2, 2, 128), (1, 3, 256), (2, 2, 384), (1, 2, 1024),
                                   (2, 2, 1), (2, 2, 50), (1, 3, 200), (2, 1, 1000)])
def test_flash_attention_vs_oracle(dev, B, H, T):
    """any T (the last 128-row block padded: rows past T read as zeros, get no
    probability and are never stored), against the oracle"""
    hd, D = 64, H * 64
    assert K.flash_supported(T, hd) and not K.flash_supported(T, 32)
    q, k, v, do = (O.normal(B * T * D, s).reshape(B * T, D) for s in (11, 12, 13, 14))
    o = torch.empty(B * T, D, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o, lse)
    o_ref, lse_ref = O.attn_fwd(B, H, q, k, v)
    assert max_rel(host(o), o_ref) <= TOL and max_rel(host(lse), lse_ref) <= TOL
    dq, dk, dv = (torch.full((B * T, D), float("nan"), device=dev) for _ in range(3))
    K.flash_bwd(B, H, cu(q), cu(k), cu(v), cu(o_ref), cu(lse_ref), cu(do), dq, dk, dv)
    refs = O.attn_bwd(B, H, q, k, v, o_ref, lse_ref, do)

    def close(got, ref):
        # at T = 1 dq and dk are exactly 0 (one key: dS = P*(dP - D) = 0), and
        # the kernels return rounding residue of dO's scale
        if not np.any(ref):
            return np.max(np.abs(got)) <= TOL * np.max(np.abs(do))
        return max_rel(got, ref) <= TOL
    for got, ref in zip((dq, dk, dv), refs):
        assert close(host(got), ref)
    # accumulate bits: each output adds onto what it holds
    base = [O.normal(B * T * D, 20 + i).reshape(B * T, D) for i in range(3)]
    acc = [cu(b.copy()) for b in base]
    K.flash_bwd(B, H, cu(q), cu(k), cu(v), cu(o_ref), cu(lse_ref), cu(do), *acc, flags=7)
    for got, ref, b0 in zip(acc, refs, base):
        assert close(host(got) - b0, ref)


@pytest.mark.parametrize("B,T", [(2, 200), (1, 999)])
def test_flash_attention_padding_rows_are_not_read(dev, B, T):
    """A T that is not a multiple of 128 pads the last 128-row block; its rows
    past T must load as zeros without reading memory.  Here q, k, v, dout and o
    are the first B*T rows of larger buffers whose further rows are NaN
    (inside the allocation, past the last sequence).  Every output must be
    finite and equal bit for bit to the same call on zero-padded buffers, for
    the fp32 kernels (stored and recomputed dQ) and the bf16 ones; the fp32
    outputs also match the oracle."""
    H, hd = 2, 64
    D = H * hd
    q, k, v, do = (O.normal(B * T * D, 171 + i).reshape(B * T, D) for i in range(4))

    def padded(x, fill):
        buf = torch.full((B * T + 128, D), fill, device=dev)
        buf[:B * T] = cu(x)
        return buf[:B * T]

    runs = {}
    for fill in ("zero", "nan"):
        val = 0.0 if fill == "zero" else float("nan")
        qv, kv, vv, dov = (padded(x, val) for x in (q, k, v, do))
        for mode in ("fp32", "recompute", "bf16"):
            o = padded(np.zeros_like(q), val)
            lse = torch.empty(B * H * T, device=dev)
            K.flash_fwd(B, H, qv, kv, vv, o, lse, bf16=mode == "bf16")
            dq, dk, dv = (torch.full((B * T, D), float("nan"), device=dev) for _ in range(3))
            K.flash_bwd(B, H, qv, kv, vv, o, lse, dov, dq, dk, dv, bf16=mode == "bf16",
                        recompute=mode == "recompute")
            runs[(fill, mode)] = [host(x) for x in (o, lse, dq, dk, dv)]
    for mode in ("fp32", "recompute", "bf16"):
        for got, want in zip(runs[("nan", mode)], runs[("zero", mode)]):
            assert np.isfinite(got).all(), mode
            assert np.array_equal(got, want), mode
    o, lse, dq, dk, dv = runs[("nan", "fp32")]
    o_ref, lse_ref = O.attn_fwd(B, H, q, k, v)
    assert max_rel(o, o_ref) <= TOL and max_rel(lse, lse_ref) <= TOL
    for got, ref in zip((dq, dk, dv), O.attn_bwd(B, H, q, k, v, o_ref, lse_ref, do)):
        assert max_rel(got, ref) <= TOL


@pytest.mark.parametrize("trend", ["rising", "falling"])
def test_flash_attention_running_max_raises_and_underflow(dev, trend):
    """The forward keeps a stale running max, raised only when a key block's
    scores exceed it by 2^8 (in log2 units).  Keys whose scale grows along the
    sequence (scores up to ~100 log2 units) take that raise on most blocks;
    keys whose scale shrinks leave the first block dominant, so later blocks'
    exponentials underflow as in the exact online softmax.  Both against the
    float64 oracle, forward and backward."""
    B, H, T, hd = 1, 2, 1024, 64
    D = H * hd
    t = np.arange(B * T, dtype=np.float64).reshape(-1, 1)
    ramp = 1 + 16 * t / T if trend == "rising" else 17 - 16 * t / T
    q = O.normal(B * T * D, 61).reshape(B * T, D)
    k = (O.normal(B * T * D, 62).reshape(B * T, D) * ramp).astype(np.float32)
    v, do = (O.normal(B * T * D, s).reshape(B * T, D) for s in (63, 64))
    o, lse = torch.empty(B * T, D, device=dev), torch.empty(B * H * T, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o, lse)
    o_ref, lse_ref = O.attn_fwd(B, H, q, k, v)
    assert max_rel(host(o), o_ref) <= TOL and max_rel(host(lse), lse_ref) <= TOL
    dq, dk, dv = (torch.empty(B * T, D, device=dev) for _ in range(3))
    K.flash_bwd(B, H, cu(q), cu(k), cu(v), o, lse, cu(do), dq, dk, dv)
    for got, ref in zip((dq, dk, dv), O.attn_bwd(B, H, q, k, v, o_ref, lse_ref, do)):
        assert max_rel(host(got), ref) <= TOL


@pytest.mark.parametrize("B,T", [(5, 1664), (10, 1152)])
def test_flash_attention_beyond_dispatch_plan(dev, B, T):
    """Launches with more workgroups than the dispatch plans place (the
    forward plans 768 = 3 per CU, the dQ kernel 1024 = 4 per CU): 780 and 1080
    query blocks of 12 heads; the later workgroups take the remaining blocks
    in order.  Every head's output is written (NaN-filled before), and
    sampled heads match the oracle."""
    H, hd = 12, 64
    D = H * hd
    q, k, v, do = (O.normal(B * T * D, 151 + i).reshape(B * T, D) for i in range(4))
    o = torch.full((B * T, D), float("nan"), device=dev)
    lse = torch.empty(B * H * T, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o, lse)
    dq, dk, dv = (torch.full((B * T, D), float("nan"), device=dev) for _ in range(3))
    K.flash_bwd(B, H, cu(q), cu(k), cu(v), o, lse, cu(do), dq, dk, dv)
    o, lse, dq, dk, dv = (host(x) for x in (o, lse, dq, dk, dv))
    for x in (o, lse, dq, dk, dv):
        assert np.isfinite(x).all()
    for b, h in ((0, 0), (B - 1, H - 1), (B // 2, 5)):
        rows, cols = slice(b * T, (b + 1) * T), slice(h * hd, (h + 1) * hd)
        qh, kh, vh, doh = (np.ascontiguousarray(x[rows, cols]) for x in (q, k, v, do))
        o_ref, lse_ref = O.attn_fwd(1, 1, qh, kh, vh)
        assert max_rel(o[rows, cols], o_ref) <= TOL, (b, h)
        assert max_rel(lse[(b * H + h) * T:(b * H + h + 1) * T], lse_ref) <= TOL, (b, h)
        for got, ref in zip((dq, dk, dv), O.attn_bwd(1, 1, qh, kh, vh, o_ref, lse_ref, doh)):
            assert max_rel(got[rows, cols], ref) <= TOL, (b, h)


@pytest.mark.parametrize("B,H,T", [(2, 2, 128), (1, 3, 256), (2, 2, 384), (8, 12, 1024),
                                   (2, 2, 200)])
def test_flash_attention_recompute_dq_equals_stored_ds(dev, B, H, T):
    """PK_FLASH_RECOMPUTE (dQ from recomputed scores, no dS tiles) against the
    stored-dS backward: dq, dk and dv bit for bit, plain and accumulating, and
    within the tolerance of the oracle; q, k, v as column views of one fused
    projection"""
    hd, D = 64, H * 64
    q, k, v, do = (O.normal(B * T * D, s).reshape(B * T, D) for s in (31, 32, 33, 34))
    qkv = cu(np.concatenate([q, k, v], 1))
    qv, kv, vv = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
    o = torch.empty(B * T, D, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    K.flash_fwd(B, H, qv, kv, vv, o, lse)
    outs = []
    for rc in (False, True):
        g = torch.full((B * T, 3 * D), float("nan"), device=dev)
        K.flash_bwd(B, H, qv, kv, vv, o, lse, cu(do), g[:, :D], g[:, D:2 * D], g[:, 2 * D:],
                    recompute=rc)
        base = O.normal(B * T * 3 * D, 40).reshape(B * T, 3 * D)
        a = cu(base.copy())
        K.flash_bwd(B, H, qv, kv, vv, o, lse, cu(do), a[:, :D], a[:, D:2 * D], a[:, 2 * D:],
                    flags=7, recompute=rc)
        outs.append((host(g), host(a)))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])
    if T <= 384:
        refs = O.attn_bwd(B, H, q, k, v, host(o), host(lse), do)
        for i, ref in enumerate(refs):
            assert max_rel(outs[1][0][:, i * D:(i + 1) * D], ref) <= TOL


def test_flash_attention_recompute_workspace_and_refusal(dev):
    from pico_amd import _lib
    L = _lib.hip_lib()
    B, H, T = 2, 3, 256
    assert L.pk_flash_attn_bwd_workspace_recompute(B, H, T) == 8 * B * H * T
    assert L.pk_flash_attn_bwd_workspace_recompute(B, H, 200) == 8 * B * H * 256
    assert L.pk_flash_attn_bwd_workspace(B, H, T) > 8 * B * H * T
    D = H * 64
    x = torch.zeros(B * T, D, device=dev)
    lse = torch.zeros(B * H * T, device=dev)
    ws = torch.empty(2 * B * H * T, device=dev)
    for bf16 in (False, True):
        name = "pk_flash_attn_bwd_bf16_f32" if bf16 else "pk_flash_attn_bwd_f32"
        # the row-constant workspace is enough for the recompute path only
        st = getattr(L, name)(B, H, T, 64, D, 0.125, *([x.data_ptr()] * 3), x.data_ptr(),
                              lse.data_ptr(), x.data_ptr(), *([x.data_ptr()] * 3),
                              ws.data_ptr(), ws.numel() * 4, 0, None)
        assert st == -1 and b"workspace" in L.pk_last_error()
    st = L.pk_flash_attn_bwd_bf16_f32(B, H, T, 64, D, 0.125, *([x.data_ptr()] * 3), x.data_ptr(),
                                      lse.data_ptr(), x.data_ptr(), *([x.data_ptr()] * 3),
                                      ws.data_ptr(), ws.numel() * 4, 16, None)
    assert st == -1 and b"fp32" in L.pk_last_error()


@pytest.mark.parametrize("flash", [True, False])
def test_attention_strided_qkv_views(dev, flash):
    # q, k, v (and dq, dk, dv) as the column blocks of one [B*T, 3*H*hd]
    # projection: row stride 3*H*hd; o and dout contiguous
    B, H, T = 2, 2, 128
    hd = 64 if flash else 32
    D = H * hd
    q, k, v, do = (O.normal(B * T * D, s).reshape(B * T, D) for s in (81, 82, 83, 84))
    qkv = cu(np.concatenate([q, k, v], 1))
    qv, kv, vv = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
    assert qv.stride(0) == 3 * D
    o = torch.empty(B * T, D, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    o_ref, lse_ref = O.attn_fwd(B, H, q, k, v)
    g = torch.full((B * T, 3 * D), float("nan"), device=dev)
    gq, gk, gv = g[:, :D], g[:, D:2 * D], g[:, 2 * D:]
    if flash:
        K.flash_fwd(B, H, qv, kv, vv, o, lse)
        K.flash_bwd(B, H, qv, kv, vv, cu(o_ref), cu(lse_ref), cu(do), gq, gk, gv)
    else:
        P = torch.empty(B * H * T * T, device=dev)
        K.attn_fwd(B, H, qv, kv, vv, o, lse, P)
        K.attn_bwd(B, H, qv, kv, vv, P, cu(do), gq, gk, gv, torch.empty_like(P))
    assert max_rel(host(o), o_ref) <= TOL and max_rel(host(lse), lse_ref) <= TOL
    refs = O.attn_bwd(B, H, q, k, v, o_ref, lse_ref, do)
    for got, ref in zip((gq, gk, gv), refs):
        assert max_rel(host(got), ref) <= TOL


def test_flash_attention_causality(dev):
    # a change to the last key/value of each sequence leaves every earlier
    # query's output unchanged (bit for bit) and changes the last one
    B, H, T, D = 2, 2, 256, 128
    q, k, v = (O.normal(B * T * D, s).reshape(B * T, D) for s in (1, 2, 3))
    o1, o2 = torch.empty(B * T, D, device=dev), torch.empty(B * T, D, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o1, lse)
    k2, v2 = k.copy(), v.copy()
    for b in range(B):
        k2[b * T + T - 1] += 1.0
        v2[b * T + T - 1] -= 1.0
    K.flash_fwd(B, H, cu(q), cu(k2), cu(v2), o2, lse)
    a, c = host(o1).reshape(B, T, D), host(o2).reshape(B, T, D)
    assert np.array_equal(a[:, :-1], c[:, :-1]) and not np.array_equal(a[:, -1], c[:, -1])


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,Kd", [(8192, 768, 768), (1000, 768, 200), (4096, 2304, 256),
                                    (8192, 768, 2048), (8000, 768, 772), (8001, 768, 37)])
def test_gemm_96_wide_tiles(dev, ta, tb, M, N, Kd):
    # N a multiple of 96: [8192, 768] (a d_model-768 transformer's
    # projections) and 8000 / 8001 rows take the 256 x 96 tiles, one per CU,
    # except as A.B, which takes 128 x 96 -- 8000 x 772 on the float4 edge
    # path, 8001 x 37 on the scalar one; 1000 x 768 and 4096 x 2304 the 128 x 96
    # ones, two per CU
    A, B, As, Bs = _operands(ta, tb, M, N, Kd, seed=M + 3 * N + Kd, integer=True)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm(ta, tb, cu(As), cu(Bs), C)
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    assert np.array_equal(host(C), ref)
    A, B, As, Bs = _operands(ta, tb, M, N, Kd, seed=M + N + Kd + 1)
    C0 = O.uniform(M * N, 9).reshape(M, N)
    C = cu(C0.copy())
    K.gemm(ta, tb, cu(As), cu(Bs), C, alpha=2.0, beta=1.0)
    assert gemm_err(host(C) - C0, 2.0 * A, B) <= TOL


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,Kd", [(4096, 4096, 256), (4000, 4000, 200), (4096, 8192, 1088),
                                    (4352, 3840, 1)])
def test_gemm_256_tiles(dev, ta, tb, M, N, Kd):
    # outputs of >= 256 tiles of 256 x 256 take the one-workgroup-per-CU shape
    # (two rounds of them only with K > 1024: a shorter K takes 128 x 128);
    # 4000 and Kd = 200 / 1 exercise its edge path
    A, B, As, Bs = _operands(ta, tb, M, N, Kd, seed=M + 5 * N + Kd, integer=True)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm(ta, tb, cu(As), cu(Bs), C)
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    assert np.array_equal(host(C), ref)
    C0 = ref.copy()
    C = cu(C0)
    K.gemm(ta, tb, cu(As), cu(Bs), C, alpha=-1.0, beta=1.0)  # C - A.B = 0 exactly
    assert not np.any(host(C))


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,Kd", [(4352, 4096, 1056), (3072, 3072, 64), (768, 32000, 64),
                                    (8192, 2304, 128), (4096, 2304, 64), (6144, 4096, 160)])
def test_gemm_tile_rounds(dev, ta, tb, M, N, Kd):
    # whole tiles, more of them than resident workgroups, so later tiles run
    # on workgroups dispatched as earlier ones finish: 4352 x 4096 (K 1056) is
    # 272 tiles of 256 x 256 for 256 slots (16 in a second round); 3072^2 and
    # the LM head's weight gradient [768, 32000] 576 and 1500 tiles of
    # 128 x 128 for 512; 8192 x 2304 768 of 256 x 96 for 256; 4096 x 2304 768
    # of 128 x 96 for 512; 6144 x 4096 with K 160, two rounds of 256 x 256 with
    # a short K, 1536 of 128 x 128
    A, B, As, Bs = _operands(ta, tb, M, N, Kd, seed=M + 11 * N + Kd, integer=True)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm(ta, tb, cu(As), cu(Bs), C)
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    assert np.array_equal(host(C), ref)
    C = cu(ref.copy())
    K.gemm(ta, tb, cu(As), cu(Bs), C, alpha=-1.0, beta=1.0)  # C - A.B = 0 exactly
    assert not np.any(host(C))
    C0 = O.uniform(M * N, 13).reshape(M, N)
    C = cu(C0.copy())
    K.gemm(ta, tb, cu(As), cu(Bs), C, alpha=0.5, beta=2.0)
    assert np.array_equal(host(C), (0.5 * ref).astype(np.float32) + 2.0 * C0)


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,Kd", [(4096, 1376, 512), (1000, 1376, 516), (516, 960, 100),
                                    (8192, 768, 772), (1024, 1024, 1024), (200, 64, 36)])
def test_gemm_vector_edge_tiles(dev, ta, tb, M, N, Kd):
    # sizes that are multiples of 4 but not of the tile: partial tiles load
    # whole float4 under a predicate (d_ff = 1376 in the 1-layer config);
    # 8192 x 768 takes 256 x 96 tiles, 1024^2 and 200 x 64 the 64 x 64 ones
    A, B, As, Bs = _operands(ta, tb, M, N, Kd, seed=M + 7 * N + Kd, integer=True)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm(ta, tb, cu(As), cu(Bs), C)
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    assert np.array_equal(host(C), ref)
    C = cu(ref.copy())
    K.gemm(ta, tb, cu(As), cu(Bs), C, alpha=-1.0, beta=1.0)
    assert not np.any(host(C))


def test_sgd_multi_equals_per_tensor(dev):
    """pk_sgd_multi_f32 over 40 tensors (two launches of up to 32; sizes 0 to
    100000, odd ones included) equals pk_sgd_f32 on each, bit for bit"""
    from pico_amd import _lib
    import ctypes
    L = _lib.hip_lib()
    sizes = [0, 1, 3, 10, 128, 1000, 100352, 4097] * 5
    ps = [cu(O.normal(n, 60 + i)) if n else torch.empty(1, device=dev) for i, n in enumerate(sizes)]
    gs = [cu(O.normal(n, 160 + i)) if n else torch.empty(1, device=dev) for i, n in enumerate(sizes)]
    ref = [p.clone() for p in ps]
    st = torch.cuda.current_stream().cuda_stream
    for p, g, n in zip(ref, gs, sizes):
        _lib.check("pk_sgd_f32", L.pk_sgd_f32(n, 0.01, p.data_ptr(), g.data_ptr(), st))
    k = len(sizes)
    parr = (ctypes.c_void_p * k)(*[p.data_ptr() for p in ps])
    garr = (ctypes.c_void_p * k)(*[g.data_ptr() for g in gs])
    narr = (ctypes.c_int64 * k)(*sizes)
    _lib.check("pk_sgd_multi_f32", L.pk_sgd_multi_f32(k, parr, garr, narr, 0.01, st))
    torch.cuda.synchronize()
    for p, r in zip(ps, ref):
        assert torch.equal(p, r)
