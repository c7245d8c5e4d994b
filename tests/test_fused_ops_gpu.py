"""Fused epilogues: pk_gemm_add_f32 / pk_gemm_swiglu_bwd_f32 /
pk_gemm_swiglu_fwd_f32 (launcher layer) and the ops built on them,
pico_matmul_add, pico_swiglu_matmul_add and pico_matmul_gate_up.

Each fused path must equal the composition of the kernels it replaces bit for
bit: the product is accumulated identically, and the epilogue applies the same
single rounding (c + a.b) or the same SwiGLU-gradient expression the row
kernels use.  The compositions themselves are pinned against the CPU oracle
elsewhere; here the composed ops' results are also compared with the oracle
within 1e-4, so an error shared by both GPU paths would show.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import _lib
from pico_amd import kernels as kern
from pico_amd.pico import TP, Pico
from tests._util import max_rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def P():
    return Pico()


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)


def _same_or_small(got, ref, small):
    """bit for bit, unless the plain fp32 product of the shape runs on the
    small-product kernels (pk_gemm_small_product_f32), whose K split rounds
    differently from the tiled kernels the fused epilogues use: then within
    fp32 rounding of the sum (pico's fused ops use the composition there)"""
    if not small:
        assert torch.equal(got, ref)
    else:
        assert max_rel(got.cpu().numpy(), ref.cpu().numpy()) <= 2e-6


# ---------------------------------------------------------------- launchers
@pytest.mark.parametrize("M,N,K", [(512, 768, 768), (200, 136, 96), (768, 768, 8192),
                                   (97, 33, 1030)])
@pytest.mark.parametrize("prec", [0, 1, 2])
def test_gemm_add_equals_product_then_add(dev, M, N, K, prec):
    """C = A.B + X with X != C against the product written to C and X added
    by the elementwise kernel (the split-K reduction carries X when K splits)"""
    L = _lib.hip_lib()
    A = _t(O.uniform(M * K, 1).reshape(M, K), dev)
    B = _t(O.uniform(K * N, 2).reshape(K, N), dev)
    X = _t(O.uniform(M * N, 3).reshape(M, N), dev)
    need = L.pk_gemm_workspace_f32(M, N, K)
    ws = torch.empty(max(need, 4) // 4, device=dev)
    got = torch.full((M, N), 7.0, device=dev)
    _lib.check("pk_gemm_add_f32", L.pk_gemm_add_f32(
        b"N", b"N", M, N, K, 1.0, A.data_ptr(), K, B.data_ptr(), N, 1.0, X.data_ptr(), N,
        got.data_ptr(), N, prec, None, ws.data_ptr(), need, None))
    prod = torch.empty(M, N, device=dev)
    fn = {0: L.pk_gemm_ex_f32, 1: L.pk_gemm_ex_bf16_f32, 2: L.pk_gemm_ex_bf16x3_f32}[prec]
    _lib.check("pk_gemm_ex", fn(b"N", b"N", M, N, K, 1.0, A.data_ptr(), K, B.data_ptr(), N, 0.0,
                                prod.data_ptr(), N, ws.data_ptr(), need, None))
    ref = torch.empty(M, N, device=dev)
    kern.binary("add", prod, X, ref)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)
    if prec == 0:
        want = O.gemm_ref_f64("N", "N", A.cpu().numpy(), B.cpu().numpy()) + X.cpu().numpy()
        assert max_rel(got.cpu().numpy(), want) <= 1e-5


@pytest.mark.parametrize("M,F,N", [(256, 512, 128), (300, 200, 136), (1024, 512, 128),
                                   (8192, 2048, 768)])
@pytest.mark.parametrize("flags", [0, 1, 2, 3])
def test_gemm_swiglu_bwd_equals_product_then_swiglu_bwd(dev, M, F, N, flags):
    L = _lib.hip_lib()
    ld = 2 * F  # gate and up as the two halves of one [M, 2F] projection
    gu = _t(O.normal(M * ld, 11).reshape(M, ld), dev)
    dY = _t(O.normal(M * N, 12).reshape(M, N), dev)
    W = _t(O.normal(F * N, 13, 0.0, 0.05).reshape(F, N), dev)
    g0 = _t(O.normal(M * ld, 14).reshape(M, ld), dev)
    gate, up = gu[:, :F], gu[:, F:]
    got = g0.clone()
    _lib.check("pk_gemm_swiglu_bwd_f32", L.pk_gemm_swiglu_bwd_f32(
        b"N", b"T", M, F, N, 1.0, dY.data_ptr(), N, W.data_ptr(), N, gate.data_ptr(), ld,
        up.data_ptr(), ld, got.data_ptr(), got.data_ptr() + 4 * F, ld, flags, 0, None, None))
    dh = torch.empty(M, F, device=dev)
    _lib.check("pk_gemm_f32", L.pk_gemm_f32(b"N", b"T", M, F, N, 1.0, dY.data_ptr(), N,
                                            W.data_ptr(), N, 0.0, dh.data_ptr(), F, None))
    ref = g0.clone()
    _lib.check("pk_swiglu_bwd_f32", L.pk_swiglu_bwd_f32(
        M, F, gate.data_ptr(), ld, up.data_ptr(), ld, dh.data_ptr(), F, ref.data_ptr(),
        ref.data_ptr() + 4 * F, ld, flags, None))
    torch.cuda.synchronize()
    _same_or_small(got, ref, L.pk_gemm_small_product_f32(M, F, N))
    if M <= 300:
        a, u = gate.cpu().numpy(), up.cpu().numpy()
        dh_ref = dY.cpu().numpy().astype(np.float64) @ W.cpu().numpy().astype(np.float64).T
        da, du = O.swiglu_bwd(a, u, dh_ref.astype(np.float32))
        base = g0.cpu().numpy()
        want_a = da + (base[:, :F] if flags & 1 else 0)
        want_u = du + (base[:, F:] if flags & 2 else 0)
        out = got.cpu().numpy()
        assert max_rel(out[:, :F], want_a) <= 1e-4
        assert max_rel(out[:, F:], want_u) <= 1e-4


@pytest.mark.parametrize("M,K,F", [(512, 768, 2048), (300, 96, 160), (200, 64, 96), (64, 40, 32),
                                   (1000, 256, 384)])
@pytest.mark.parametrize("prec", [0, 1, 2, 3])
def test_gemm_swiglu_fwd_equals_product_then_swiglu(dev, M, K, F, prec):
    """C = A.[W1 | W3] and h = silu(C[:, :F]) * C[:, F:] from one product,
    against the plain product (pk_gemm_ex_*, the same multiplies) and the
    SwiGLU row kernel on its two column views: C and h bit for bit (the
    paired tiles -- 256x256, 128x96, 64x64 ... by F -- accumulate k in the
    same order as every other tile)"""
    L = _lib.hip_lib()
    A = _t(O.uniform(M * K, 51).reshape(M, K), dev)
    W = _t(O.uniform(K * 2 * F, 52).reshape(K, 2 * F) * 0.2, dev)
    C = torch.full((M, 2 * F), float("nan"), device=dev)
    h = torch.full((M, F), float("nan"), device=dev)
    _lib.check("pk_gemm_swiglu_fwd_f32", L.pk_gemm_swiglu_fwd_f32(
        b"N", b"N", M, 2 * F, K, 1.0, A.data_ptr(), K, W.data_ptr(), 2 * F, C.data_ptr(), 2 * F,
        h.data_ptr(), F, prec, None, None))
    ref = torch.empty(M, 2 * F, device=dev)
    fn = {0: L.pk_gemm_ex_f32, 1: L.pk_gemm_ex_bf16_f32, 2: L.pk_gemm_ex_bf16x3_f32,
          3: L.pk_gemm_ex_fp8_f32}[prec]
    _lib.check("pk_gemm_ex", fn(b"N", b"N", M, 2 * F, K, 1.0, A.data_ptr(), K, W.data_ptr(),
                                2 * F, 0.0, ref.data_ptr(), 2 * F, None, 0, None))
    href = torch.empty(M, F, device=dev)
    _lib.check("pk_swiglu_fwd_f32", L.pk_swiglu_fwd_f32(
        M, F, ref.data_ptr(), 2 * F, ref.data_ptr() + 4 * F, 2 * F, href.data_ptr(), F, None))
    torch.cuda.synchronize()
    small = prec == 0 and L.pk_gemm_small_product_f32(M, 2 * F, K)
    _same_or_small(C, ref, small)
    _same_or_small(h, href, small)
    if prec == 0 and M <= 512:
        c64 = O.gemm_ref_f64("N", "N", A.cpu().numpy(), W.cpu().numpy())
        assert max_rel(C.cpu().numpy(), c64) <= 1e-5
        want = O.swiglu_fwd(c64[:, :F].astype(np.float32), c64[:, F:].astype(np.float32))
        assert max_rel(h.cpu().numpy(), want) <= 1e-4


def test_gemm_swiglu_fwd_strided_h_and_refusals(dev):
    L = _lib.hip_lib()
    M, K, F = 96, 64, 128
    A = _t(O.uniform(M * K, 61).reshape(M, K), dev)
    W = _t(O.uniform(K * 2 * F, 62).reshape(K, 2 * F), dev)
    C = torch.empty(M, 2 * F, device=dev)
    hbuf = torch.full((M, F + 36), -7.0, device=dev)  # h with row stride F + 36
    _lib.check("pk_gemm_swiglu_fwd_f32", L.pk_gemm_swiglu_fwd_f32(
        b"N", b"N", M, 2 * F, K, 1.0, A.data_ptr(), K, W.data_ptr(), 2 * F, C.data_ptr(), 2 * F,
        hbuf.data_ptr(), F + 36, 0, None, None))
    href = torch.empty(M, F, device=dev)
    _lib.check("pk_swiglu_fwd_f32", L.pk_swiglu_fwd_f32(
        M, F, C.data_ptr(), 2 * F, C.data_ptr() + 4 * F, 2 * F, href.data_ptr(), F, None))
    torch.cuda.synchronize()
    assert torch.equal(hbuf[:, :F], href)
    assert bool((hbuf[:, F:] == -7.0).all())  # the padding is untouched

    def call(ta, tb, N, ldh):
        return L.pk_gemm_swiglu_fwd_f32(ta, tb, M, N, K, 1.0, A.data_ptr(), K, W.data_ptr(),
                                        2 * F, C.data_ptr(), 2 * F, hbuf.data_ptr(), ldh, 0, None,
                                        None)
    assert call(b"N", b"T", 2 * F, F) == -1 and b"N','N'" in L.pk_last_error()
    assert call(b"N", b"N", 2 * F - 4, F) == -1  # N not 2F with F a multiple of 4
    assert call(b"N", b"N", 200, 100) == -1 and b"multiple of 32" in L.pk_last_error()
    assert call(b"N", b"N", 2 * F, F - 1) == -1 and b"ldh" in L.pk_last_error()


def test_gemm_swiglu_bwd_refuses_other_layouts(dev):
    L = _lib.hip_lib()
    x = torch.zeros(64, 64, device=dev)
    st = L.pk_gemm_swiglu_bwd_f32(b"N", b"N", 64, 64, 64, 1.0, x.data_ptr(), 64, x.data_ptr(), 64,
                                  x.data_ptr(), 64, x.data_ptr(), 64, x.data_ptr(),
                                  x.data_ptr() + 4, 64, 0, 0, None, None)
    assert st == -1 and b"layout" in L.pk_last_error()


# ------------------------------------------------------------------- ops
def _grads(P, ts):
    return [P.grad(t).copy() for t in ts]


def _run_matmul_add(P, fused, av, bv, cv, seed_grad, b_param):
    with P.arena(1 << 26):
        a = P.tensor(list(av.shape), av)
        b = (P.param if b_param else P.tensor)(list(bv.shape), bv)
        c = P.tensor(list(cv.shape), cv)
        out = P.matmul_add(a, b, c) if fused else P.add(c, P.matmul(a, b))
        loss = P.mul(out, P.tensor(list(seed_grad.shape), seed_grad))
        P.backward(loss)
        res = (P.data(out), *_grads(P, [a, b, c]))
        if b_param:
            P.free(b)
        return res


@pytest.mark.parametrize("M,K,N", [(64, 48, 40), (512, 768, 768), (37, 100, 65)])
@pytest.mark.parametrize("b_param", [False, True])
def test_matmul_add_equals_composition(P, M, K, N, b_param):
    av = O.uniform(M * K, 21).reshape(M, K)
    bv = O.uniform(K * N, 22).reshape(K, N)
    cv = O.uniform(M * N, 23).reshape(M, N)
    sg = O.uniform(M * N, 24).reshape(M, N)
    fused = _run_matmul_add(P, True, av, bv, cv, sg, b_param)
    plain = _run_matmul_add(P, False, av, bv, cv, sg, b_param)
    for x, y in zip(fused, plain):
        assert np.array_equal(x, y)
    # and the values, against the oracle's loops
    out_ref = O.binary(0, cv, O.matmul_scalar(av, bv))
    assert max_rel(fused[0], out_ref.ravel()) <= 1e-5
    dA, dB = O.matmul_backward(av, bv, sg)
    assert max_rel(fused[1], dA.ravel()) <= 1e-4 and max_rel(fused[2], dB.ravel()) <= 1e-4
    assert np.array_equal(fused[3], sg.ravel())


def _run_swiglu_mm(P, fused, xv, w13v, w2v, cv, seed_grad, split, gate_up=False):
    M, d = xv.shape
    F = w2v.shape[0]
    with P.arena(1 << 27):
        x = P.tensor([M, d], xv)
        w13 = P.param([d, 2 * F], w13v)
        w2 = P.param([F, w2v.shape[1]], w2v)
        c = P.tensor(list(cv.shape), cv) if cv is not None else None
        if split:
            gu = P.matmul_gate_up(x, w13) if gate_up else P.matmul(x, w13)
            gate, up = P.split_cols(gu, 2)
        else:
            g_ = P.tensor([M, F], (xv @ w13v)[:, :F])
            u_ = P.tensor([M, F], (xv @ w13v)[:, F:])
            gate, up = g_, u_
        if fused:
            out = P.swiglu_matmul_add(gate, up, w2, c)
        else:
            out = P.matmul(P.swiglu(gate, up), w2)
            if c is not None:
                out = P.add(c, out)
        P.backward(P.mul(out, P.tensor(list(seed_grad.shape), seed_grad)))
        ts = [x, w13, w2] + ([c] if c is not None else []) + ([] if split else [gate, up])
        res = (P.data(out), *_grads(P, ts))
        P.free(w13)
        P.free(w2)
        return res


@pytest.mark.parametrize("M,d,F,N", [(128, 64, 160, 64), (300, 96, 200, 72), (1024, 768, 2048, 768)])
@pytest.mark.parametrize("resid", [False, True])
@pytest.mark.parametrize("split,gate_up", [(True, False), (True, True), (False, False)])
def test_swiglu_matmul_add_equals_composition(P, M, d, F, N, resid, split, gate_up):
    """the fused path (gate_up: the projection by pico_matmul_gate_up, whose h
    pico_swiglu_matmul_add then takes -- F = 200 is not a multiple of 32, so
    there it is a plain product) against matmul, swiglu, matmul, add: outputs
    and every gradient bit for bit"""
    xv = O.normal(M * d, 31).reshape(M, d)
    w13v = O.normal(d * 2 * F, 32, 0.0, 0.05).reshape(d, 2 * F)
    w2v = O.normal(F * N, 33, 0.0, 0.05).reshape(F, N)
    cv = O.normal(M * N, 34).reshape(M, N) if resid else None
    sg = O.normal(M * N, 35).reshape(M, N)
    fused = _run_swiglu_mm(P, True, xv, w13v, w2v, cv, sg, split, gate_up)
    plain = _run_swiglu_mm(P, False, xv, w13v, w2v, cv, sg, split)
    assert len(fused) == len(plain)
    for i, (x, y) in enumerate(zip(fused, plain)):
        assert np.array_equal(x, y), i


def test_swiglu_matmul_add_values_against_oracle(P):
    M, F, N = 96, 160, 80
    gv = O.normal(M * F, 41).reshape(M, F)
    uv = O.normal(M * F, 42).reshape(M, F)
    wv = O.normal(F * N, 43, 0.0, 0.1).reshape(F, N)
    cv = O.normal(M * N, 44).reshape(M, N)
    sg = O.normal(M * N, 45).reshape(M, N)
    with P.arena(1 << 24):
        gate, up = P.tensor([M, F], gv), P.tensor([M, F], uv)
        w, c = P.tensor([F, N], wv), P.tensor([M, N], cv)
        out = P.swiglu_matmul_add(gate, up, w, c)
        P.backward(P.mul(out, P.tensor([M, N], sg)))
        got = [P.data(out), P.grad(gate), P.grad(up), P.grad(w), P.grad(c)]
    h = O.swiglu_fwd(gv, uv)
    want_out = O.binary(0, cv, O.matmul_scalar(h, wv))
    dh, dw = O.matmul_backward(h, wv, sg)
    da, du = O.swiglu_bwd(gv, uv, dh)
    for g, w_ in zip(got, [want_out, da, du, dw, sg]):
        assert max_rel(g, w_.ravel()) <= 1e-4


def test_fused_ops_refuse_bad_shapes(P):
    with P.arena(1 << 20):
        a = P.tensor([4, 3], np.ones(12))
        b = P.tensor([3, 5], np.ones(15))
        bad = P.tensor([4, 6], np.ones(24))
        assert not P.lib.pico_matmul_add(a, b, bad)
        g = P.tensor([4, 3], np.ones(12))
        assert not P.lib.pico_swiglu_matmul_add(g, g, b, None)  # gate == up
        assert not P.lib.pico_swiglu_matmul_add(g, a, P.tensor([4, 5], np.ones(20)), None)


# ------------------------------------------------------------------ Linear
def _linear_layer(P, K, N, wv, bv):
    layer = P.lib.pico_nn_linear_init(K, N, True)
    w = ctypes.cast(layer + 8, ctypes.POINTER(TP)).contents
    b = ctypes.cast(layer + 16, ctypes.POINTER(TP)).contents
    P.set(w, wv)
    P.set(b, bv)
    return layer, w, b


@pytest.mark.parametrize("M,K,N", [(64, 784, 128), (64, 128, 10), (512, 512, 512), (300, 96, 200),
                                   (4096, 512, 1376)])
@pytest.mark.parametrize("x_param", [False, True])
def test_linear_equals_matmul_then_add(P, M, K, N, x_param):
    """pico_nn_linear_forward is one node, x.W + b with the bias row added in
    the product's epilogue (pk_gemm_add_f32, ldx 0).  It equals pico_matmul
    then pico_add (src/nn/linear.c:57-64) bit for bit: the output and the
    gradients of x, W and b, with x an activation (the weight and bias
    gradients then run on the side stream) or a parameter.  The shapes take the
    split-K product (64 x 784 . 784 x 128), the scalar edge path (N 10), the
    small-product kernel (512^3) and the tiled kernel."""
    xv = O.normal(M * K, 51).reshape(M, K)
    wv = O.normal(K * N, 52, 0.0, 0.1).reshape(K, N)
    bv = O.normal(N, 53)
    sg = O.normal(M * N, 54).reshape(M, N)
    runs = []
    for fused in (True, False):
        with P.arena(1 << 26):
            layer, w, b = _linear_layer(P, K, N, wv, bv)
            x = P.param([M, K], xv) if x_param else P.tensor([M, K], xv)
            out = (P.lib.pico_nn_linear_forward(layer, x) if fused
                   else P.add(P.matmul(x, w), b))
            assert out
            P.backward(P.mul(out, P.tensor([M, N], sg)))
            runs.append([P.data(out), P.grad(x), P.grad(w), P.grad(b)])
            if x_param:
                P.free(x)
            P.lib.pico_nn_linear_free(layer)
    for i, (f, c) in enumerate(zip(*runs)):
        assert np.array_equal(f, c), i
    want = O.gemm_ref_f64("N", "N", xv, wv) + bv
    assert max_rel(runs[0][0], want.ravel()) <= 1e-5
    assert max_rel(runs[0][3], sg.astype(np.float64).sum(0)) <= 1e-5


def test_linear_bias_row_epilogue_launcher(dev):
    """pk_gemm_add_f32 with ldx 0 adds one row to every row of C, for the
    tiled, small-product and split-K paths: integer operands, bit for bit"""
    L = _lib.hip_lib()
    rng = np.random.default_rng(7)
    for M, N, K in ((256, 256, 256), (1024, 768, 256), (64, 128, 4096), (100, 36, 20)):
        A = rng.integers(-8, 9, (M, K)).astype(np.float32)
        B = rng.integers(-8, 9, (K, N)).astype(np.float32)
        x = rng.integers(-100, 100, N).astype(np.float32)
        need = L.pk_gemm_workspace_f32(M, N, K)
        ws = torch.empty(max(need, 4) // 4, device=dev)
        C = torch.full((M, N), float("nan"), device=dev)
        dA, dB, dx = _t(A, dev), _t(B, dev), _t(x, dev)
        _lib.check("pk_gemm_add_f32", L.pk_gemm_add_f32(
            b"N", b"N", M, N, K, 1.0, dA.data_ptr(), K, dB.data_ptr(), N, 1.0, dx.data_ptr(), 0,
            C.data_ptr(), N, 0, None, ws.data_ptr(), need, None))
        ref = (A.astype(np.float64) @ B.astype(np.float64) + x).astype(np.float32)
        torch.cuda.synchronize()
        assert np.array_equal(C.cpu().numpy(), ref), (M, N, K)
