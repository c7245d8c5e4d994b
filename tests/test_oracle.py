"""Pins the CPU oracle (CPU-only tests).

The oracle is checked against (1) the reference's own known-answer tests,
(2) the reference itself compiled from its sources (oracle/_ref, bit-exact,
where it was built), (3) torch-CPU float64 golden vectors for the ops the
reference lacks, and (4) closed forms and invariants chosen so a dropped term,
wrong sign or transposed operand fails.
"""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests._util import gemm_err, max_rel, row_err

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_ops.npz"))


# --------------------------------------------------- reference KATs: matmul
def test_matmul_forward_kats():
    # tests/test_autograd.c:286 (2x3 . 3x2) and :318 (square)
    A = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    B = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    for f in (O.matmul_scalar, O.matmul_avx):
        assert f(A, B).tolist() == [[58, 64], [139, 154]]
        assert f([[1, 2], [3, 4]], [[5, 6], [7, 8]]).tolist() == [[19, 22], [43, 50]]
    # :482 dot product (1x3 . 3x1) = 32
    assert O.matmul_scalar([[1, 2, 3]], [[4], [5], [6]]).tolist() == [[32]]


def test_matmul_avx_all_edges_kat():
    # tests/kernels/test_avx_matmul.c:266-303: 3x3 . 3x10 covers 2x8 tile, 1x8 tile,
    # right-edge and bottom-right scalar cells
    A = np.arange(1, 10, dtype=np.float32).reshape(3, 3)
    B = np.arange(1, 31, dtype=np.float32).reshape(3, 10)
    expect = A.astype(np.float64) @ B.astype(np.float64)
    assert np.array_equal(O.matmul_avx(A, B), expect.astype(np.float32))


def test_matmul_backward_kats():
    # tests/test_autograd.c:348 square, :382 non-square, seed dC = ones
    dA, dB = O.matmul_backward([[1, 2], [3, 4]], [[5, 6], [7, 8]], np.ones((2, 2), np.float32))
    assert dA.ravel().tolist() == [11, 15, 11, 15] and dB.ravel().tolist() == [4, 4, 6, 6]
    A = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    B = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    dA, dB = O.matmul_backward(A, B, np.ones((2, 2), np.float32))
    assert dA.ravel().tolist() == [15, 19, 23, 15, 19, 23]
    assert dB.ravel().tolist() == [5, 5, 7, 7, 9, 9]


def test_matmul_shared_parent_through_graph():
    # tests/test_autograd.c:559: C = A.A with A shared -> dA = dC.A^T + A^T.dC
    L = O.api()
    ar = L.arena_init(1 << 20)
    L.arena_ctx_push(ar)
    a = O.param([2, 2], [1, 2, 3, 4])
    c = L.pico_matmul(a, a)
    L.pico_backward(ar, c)
    assert O.grad(a).tolist() == [7, 11, 9, 13]
    L.arena_ctx_pop()
    L.arena_destroy(ar)
    L.pico_free(a)


def test_matmul_then_add_graph():
    # tests/test_autograd.c:517 pattern: (A.B) + bias, bias broadcast down the rows
    L = O.api()
    ar = L.arena_init(1 << 20)
    L.arena_ctx_push(ar)
    a = O.param([2, 2], [1, 2, 3, 4])
    b = O.param([2, 2], [5, 6, 7, 8])
    bias = O.param([2], [10, 20])
    out = L.pico_add(L.pico_matmul(a, b), bias)
    L.pico_backward(ar, out)
    assert O.data(out).tolist() == [29, 42, 53, 70]
    assert O.grad(bias).tolist() == [2, 2]
    assert O.grad(a).tolist() == [11, 15, 11, 15]
    L.arena_ctx_pop()
    L.arena_destroy(ar)


# ------------------------------------------------ reference KATs: broadcast
def test_broadcast_kats():
    g = np.array([[1, 2], [3, 4]], np.float32)
    a = np.zeros((2, 2), np.float32)
    # add_row (test_autograd.c:592): b [2] -> b.grad = column sums
    ga, gb = O.binary_bwd(0, a, np.zeros(2, np.float32), g, np.zeros((2, 2), np.float32),
                          np.zeros(2, np.float32))
    assert ga.ravel().tolist() == [1, 2, 3, 4] and gb.tolist() == [4, 6]
    # add_col (:627): b [2,1] -> row sums
    _, gb = O.binary_bwd(0, a, np.zeros((2, 1), np.float32), g, np.zeros((2, 2), np.float32),
                         np.zeros((2, 1), np.float32))
    assert gb.ravel().tolist() == [3, 7]
    # sub_row (:654): negated column sums
    _, gb = O.binary_bwd(1, a, np.zeros(2, np.float32), g, np.zeros((2, 2), np.float32),
                         np.zeros(2, np.float32))
    assert gb.tolist() == [-4, -6]
    # mul forward broadcast (:713) and mul_row backward (:828)
    av = np.array([[1, 2], [3, 4]], np.float32)
    bv = np.array([10, 20], np.float32)
    assert O.binary(2, av, bv).ravel().tolist() == [10, 40, 30, 80]
    ga, gb = O.binary_bwd(2, av, bv, g, np.zeros((2, 2), np.float32), np.zeros(2, np.float32))
    assert ga.ravel().tolist() == [10, 40, 30, 80] and gb.tolist() == [10, 20]


def test_unary_kats():
    # tests/test_unary.c:18-129 forward, :165-289 backward with upstream 2
    pi = np.float32(np.pi)
    assert O.unary(0, [0, 4, 9, 16]).tolist() == [0, 2, 3, 4]
    near = lambda a, b: np.allclose(a, b, atol=1e-5)  # the reference's NEAR
    assert near(O.unary(1, [0, pi / 2]), [0, 1]) and near(O.unary(2, [0, pi]), [1, -1])
    assert near(O.unary(3, [0, pi / 4]), [0, 1]) and near(O.unary(4, [0, 20]), [0, 1])
    assert O.unary(5, [1])[0] == 0 and near(O.unary(5, [np.e]), [1])
    for op, x, want in ((0, 4.0, 0.5), (1, pi, -2.0), (2, pi / 2, -2.0), (3, 0.0, 2.0),
                        (4, 0.0, 2.0), (5, 2.0, 1.0)):
        xs = np.array([x], np.float32)
        g = O.unary_bwd(op, xs, O.unary(op, xs), np.array([2.0], np.float32),
                        np.zeros(1, np.float32))
        assert near(g, [want]), op


@pytest.mark.skipif(not O.ref_available(), reason="reference build absent")
@pytest.mark.parametrize("op", range(6))
def test_unary_bitexact_vs_reference(op):
    # libm-dependent values and the backward expressions as the reference
    # evaluates them (tanh's g*1 - y^2 precedence included), bit for bit
    import ctypes

    x = O.uniform(4099, 30 + op, 0.05, 1.4)
    y = np.empty_like(x)
    O.ref().picoref_unary(ctypes.c_int(op), ctypes.c_int64(x.size), O.p(x), O.p(y))
    assert np.array_equal(O.unary(op, x), y)
    gy, gx0 = O.normal(x.size, 40 + op), O.normal(x.size, 50 + op)
    gref = gx0.copy()
    O.ref().picoref_unary_bwd(ctypes.c_int(op), ctypes.c_int64(x.size), O.p(x), O.p(y), O.p(gy),
                              O.p(gref))
    assert np.array_equal(O.unary_bwd(op, x, y, gy, gx0.copy()), gref)


def test_relu_kats():
    # tests/act/test_activations.c:12 (clamp), :75 (gate at 0 closed), NaN -> 0
    x = np.array([-2, -0.5, 0, 0.5, 3, np.nan, -0.0], np.float32)
    y = O.relu(x)
    assert y.tolist() == [0, 0, 0, 0.5, 3, 0, 0]
    gx = O.relu_bwd(y, np.full(7, 2.0, np.float32), np.zeros(7, np.float32))
    assert gx.tolist() == [0, 0, 0, 2, 2, 0, 0]


def test_sgd_kat():
    # tests/optim/test_optim.c:16: 10 - 0.5*4 = 8
    p = np.array([10.0], np.float32)
    assert O.sgd(p, np.array([4.0], np.float32), 0.5).tolist() == [8.0]


def test_linear_grads_kat():
    # tests/nn/test_linear.c:262 pattern: W.grad = x^T . 1, b.grad = batch size
    L = O.api()
    ar = L.arena_init(1 << 20)
    L.arena_ctx_push(ar)
    x = O.param([1, 2], [10, 20])
    W = O.param([2, 1], [0, 0])
    b = O.param([1], [0])
    out = L.pico_add(L.pico_matmul(x, W), b)
    neg = O.param([1], [-1])
    loss = L.pico_mul(out, neg)
    L.pico_backward(ar, loss)
    assert O.grad(W).tolist() == [-10, -20] and O.grad(b).tolist() == [-1]
    L.arena_ctx_pop()
    L.arena_destroy(ar)


# ---------------------------------------- bit-equality with the reference
needs_ref = pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built here")


@needs_ref
@pytest.mark.parametrize("M,K,N", [(3, 3, 10), (17, 31, 23), (64, 784, 128), (520, 64, 37),
                                   (9, 1, 8)])
def test_matmul_bitexact_vs_reference(M, K, N):
    import ctypes

    R = O.ref()
    A = O.uniform(M * K, 11 + M).reshape(M, K)
    B = O.uniform(K * N, 12 + N).reshape(K, N)
    for ours, theirs in ((O.matmul_scalar, R.picoref_matmul_scalar),
                         (O.matmul_avx, R.picoref_matmul_avx)):
        Cr = np.zeros((M, N), np.float32)
        theirs(ctypes.c_int(M), ctypes.c_int(N), ctypes.c_int(K), O.p(A), O.p(B), O.p(Cr))
        assert np.array_equal(ours(A, B).view(np.uint32), Cr.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("M,K,N", [(5, 7, 3), (33, 16, 40), (64, 128, 10)])
def test_matmul_backward_bitexact_vs_reference(M, K, N):
    import ctypes

    R = O.ref()
    A = O.uniform(M * K, 3).reshape(M, K)
    B = O.uniform(K * N, 4).reshape(K, N)
    dC = O.uniform(M * N, 5).reshape(M, N)
    dA0 = O.uniform(M * K, 6).reshape(M, K)  # nonzero start: += semantics
    dB0 = O.uniform(K * N, 7).reshape(K, N)
    dA, dB = O.matmul_backward(A, B, dC, dA0.copy(), dB0.copy())
    dAr, dBr = dA0.copy(), dB0.copy()
    R.picoref_matmul_backward(ctypes.c_int(M), ctypes.c_int(K), ctypes.c_int(N), O.p(A), O.p(B),
                              O.p(dC), O.p(dAr), O.p(dBr))
    assert np.array_equal(dA.view(np.uint32), dAr.view(np.uint32))
    assert np.array_equal(dB.view(np.uint32), dBr.view(np.uint32))
    # the pico-order GEMM is the same arithmetic in GEMM form
    dA2 = O.gemm_pico_order("N", "T", dC, B, dA0.copy())
    dB2 = O.gemm_pico_order("T", "N", A, dC, dB0.copy())
    assert np.array_equal(dA2, dAr) and np.array_equal(dB2, dBr)


@needs_ref
def test_pico_rand_stream_matches_reference():
    import ctypes

    # xorshift32 -> [0,1) from src/tensor.c:249-273, via the reference's pico_rand
    theirs = np.empty(50, np.float32)
    O.ref().picoref_rand(ctypes.c_uint32(12345), ctypes.c_int64(50), O.p(theirs))
    assert np.array_equal(O.pico_rand(50, 12345), theirs)


# ---------------- the op API, graph walk and optimizer vs the reference's own
# The same call sequence runs on the oracle (O.api()) and on the compiled
# reference's exported pico API (O.ref_api(): src/ops.c, act/activations.c,
# autograd.h through pico_backward, optim/SGD.c, nn/linear.c), on seeded random
# values with random upstream gradients, so the order of every sum over
# stretched dims and every accumulation into a shared parent's grad shows.
def _pv(L, shape, values):
    arr = (ctypes.c_int64 * len(shape))(*shape)
    t = L.pico_param(arr, len(shape))
    O.set_data(t, values)
    return t


def _on_both(build, simd=3):
    """build(L, arena) -> list of tensors; their data and grads, oracle then
    reference, as uint32 bit patterns"""
    outs = []
    for L in (O.api(), O.ref_api()):
        O.set_simd(L, simd)
        ar = L.arena_init(1 << 24)
        L.arena_ctx_push(ar)
        try:
            ts, owned = build(L, ar)
            outs.append([np.concatenate([O.data(t), O.grad(t)]).view(np.uint32) for t in ts])
            for t in owned:
                L.pico_free(t)
        finally:
            L.arena_ctx_pop()
            L.arena_destroy(ar)
    O.set_simd(O.api(), 3)  # pico_init's level
    return outs


BCAST = [((5, 1, 3), (1, 4, 1)), ((2, 3, 4), (3, 1)), ((3, 64, 10), (1, 10)), ((4, 5), (5,)),
         ((7, 1), (1, 6)), ((16, 19), (16, 19)), ((2, 1, 3, 1), (5, 1, 4)), ((6,), (1,)),
         ((1,), (3, 2))]


@needs_ref
@pytest.mark.parametrize("simd", [0, 3])
@pytest.mark.parametrize("sa,sb", BCAST)
def test_broadcast_graph_bitexact_vs_reference(sa, sb, simd):
    """add, sub and mul with numpy-style broadcasting, forward and backward
    through pico_backward: s = a + b, d = s - b, m = d * b, y = m * w (b feeds
    three ops, w random so every upstream gradient is random)"""
    so = np.broadcast_shapes(sa, sb)
    a0, b0 = O.normal(int(np.prod(sa)), 1), O.normal(int(np.prod(sb)), 2)
    w0 = O.normal(int(np.prod(so)), 3)

    def build(L, ar):
        a, b, w = _pv(L, sa, a0), _pv(L, sb, b0), _pv(L, so, w0)
        s = L.pico_add(a, b)
        d = L.pico_sub(s, b)
        m = L.pico_mul(d, b)
        y = L.pico_mul(m, w)
        L.pico_backward(ar, y)
        return [a, b, w, s, d, m, y], [a, b, w]

    ours, theirs = _on_both(build, simd)
    for i, (x, r) in enumerate(zip(ours, theirs)):
        assert np.array_equal(x, r), i


@needs_ref
def test_transposed_view_graph_bitexact_vs_reference():
    """a pico_transpose_2d view (swapped shape and strides) as an operand of a
    broadcast add and a same-shape mul, and its grad written at the view's
    strides, against the reference's scalar kernels (cpu_scalar.h:12-30, which
    index both operands through map_index).

    The reference's AVX2 level differs here: its same-shape fast path
    (cpu_avx_2.h:15-33) reads both operands in storage order and ignores a
    view's strides, so w * a^T comes out as w * a elementwise in memory order.
    The oracle (and the GPU library) keep the strided semantics of the scalar
    path and of every backward hook; the second half pins that the AVX2
    difference is exactly that flat read."""
    a0, b0, w0 = O.normal(15, 4), O.normal(3, 5), O.normal(15, 6)

    def build(L, ar):
        a, b, w = _pv(L, [3, 5], a0), _pv(L, [3], b0), _pv(L, [5, 3], w0)
        L.pico_transpose_2d(a)
        wa = L.pico_mul(w, a)
        y = L.pico_mul(L.pico_add(a, b), wa)
        L.pico_backward(ar, y)
        return [a, b, w, wa, y], [a, b, w]

    ours, theirs = _on_both(build, simd=0)
    for i, (x, r) in enumerate(zip(ours, theirs)):
        assert np.array_equal(x, r), i
    # the strided product, as the oracle computes it at any level
    wa_ours = ours[3][:15].view(np.float32)
    assert np.array_equal(wa_ours, (w0.reshape(5, 3) * a0.reshape(3, 5).T).ravel())
    # the reference's AVX2 same-shape path: the flat storage-order product
    _, avx2 = _on_both(build, simd=3)
    assert np.array_equal(avx2[3][:15].view(np.float32), w0 * a0)


@needs_ref
def test_relu_graph_bitexact_vs_reference():
    """relu forward (NaN -> 0, -0.0, exact zeros) and its gate y > 0"""
    x0 = O.normal(64 * 33, 7)
    x0[::17] = 0.0
    x0[5::23] = -0.0
    x0[3::31] = np.nan
    w0 = O.normal(64 * 33, 8)

    def build(L, ar):
        x, w = _pv(L, [64, 33], x0), _pv(L, [64, 33], w0)
        r = L.pico_relu(x)
        y = L.pico_mul(r, w)
        L.pico_backward(ar, y)
        return [r, y, w], [x, w]

    ours, theirs = _on_both(build)
    for i, (x, r) in enumerate(zip(ours, theirs)):
        assert np.array_equal(x, r), i


@needs_ref
def test_graph_walk_shared_parents_bitexact_vs_reference():
    """a diamond-rich graph (a and b feed several ops, c feeds two): the
    post-order walk fixes the order of the += into each shared grad, hence its
    rounding; a second pico_backward over the same graph accumulates again"""
    a0, b0, w0 = O.normal(6 * 5, 9), O.normal(6 * 5, 10), O.normal(6 * 5, 11)
    bias0 = O.normal(5, 12)

    def build(L, ar):
        a, b, w, bias = (_pv(L, [6, 5], a0), _pv(L, [6, 5], b0), _pv(L, [6, 5], w0),
                         _pv(L, [5], bias0))
        c = L.pico_mul(a, b)
        d = L.pico_add(c, a)
        e = L.pico_mul(d, c)
        f = L.pico_sub(e, L.pico_add(b, bias))
        g = L.pico_mul(L.pico_add(f, a), w)
        L.pico_backward(ar, g)
        L.pico_backward(ar, g)
        return [a, b, w, bias, c, d, e, f, g], [a, b, w, bias]

    ours, theirs = _on_both(build)
    for i, (x, r) in enumerate(zip(ours, theirs)):
        assert np.array_equal(x, r), i


@needs_ref
def test_linear_and_sgd_steps_bitexact_vs_reference():
    """PicoLinear (x.W + b, bias broadcast over the batch) through a two-layer
    graph with relu, backward, then SGD steps (p -= lr*g, two roundings) and
    zero_grad, three times: every weight, bias and activation bit for bit"""
    x0 = O.normal(8 * 7, 13)
    w10, b10 = O.normal(7 * 5, 14, 0.0, 0.5), O.normal(5, 15)
    w20, b20 = O.normal(5 * 3, 16, 0.0, 0.5), O.normal(3, 17)
    gy0 = O.normal(8 * 3, 18)

    def build(L, ar):
        l1 = L.pico_nn_linear_init(7, 5, True)
        l2 = L.pico_nn_linear_init(5, 3, True)
        for lin, wv, bv in ((l1, w10, b10), (l2, w20, b20)):
            O.set_data(lin.contents.weights, wv)
            O.set_data(lin.contents.bias, bv)
        opt = L.pico_optim_sgd_init(ctypes.c_float(0.05))
        params = [l1.contents.weights, l1.contents.bias, l2.contents.weights, l2.contents.bias]
        for t in params:
            L.pico_optim_sgd_add(opt, t)
        x, gy = _pv(L, [8, 7], x0), _pv(L, [8, 3], gy0)
        acts = []
        for _ in range(3):
            h = L.pico_relu(L.pico_nn_linear_forward(l1, x))
            out = L.pico_nn_linear_forward(l2, h)
            y = L.pico_mul(out, gy)
            L.pico_backward(ar, y)
            acts += [h, out]
            L.pico_optim_sgd_step(opt)
            grads = [O.grad(t).copy() for t in params]
            L.pico_optim_sgd_zero_grad(opt)
            assert not any(np.any(O.grad(t)) for t in params)
            acts.append(_pv(L, [sum(g.size for g in grads)], np.concatenate(grads)))
        L.pico_optim_sgd_free(opt)
        snap = [_pv(L, [t.contents.numel], O.data(t)) for t in params]
        L.pico_nn_linear_free(l1)
        L.pico_nn_linear_free(l2)
        return snap + acts, [x, gy] + snap + acts[2::3]

    ours, theirs = _on_both(build)
    for i, (x, r) in enumerate(zip(ours, theirs)):
        assert np.array_equal(x, r), i


# ------------------------------------------------------- math pins (GEMM)
@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N")])
def test_gemm_f64_reference_vs_numpy(ta, tb):
    rng = np.random.default_rng(1)
    A = rng.uniform(-1, 1, (37, 29)).astype(np.float32)
    B = rng.uniform(-1, 1, (29 if tb == "N" else 41, 41 if tb == "N" else 29)).astype(np.float32)
    if ta == "T":
        A = np.ascontiguousarray(A.T)
    C0 = rng.uniform(-1, 1, (37, 41)).astype(np.float32)
    C = O.gemm_ref_f64(ta, tb, A, B, alpha=0.5, beta=2.0, C=C0.copy())
    Aop = A.T if ta == "T" else A
    Bop = B.T if tb == "T" else B
    ref = 0.5 * (Aop.astype(np.float64) @ Bop) + 2.0 * C0
    assert np.allclose(C, ref, rtol=1e-6, atol=1e-6)


def test_integer_matmul_is_exact_any_order():
    # integer-valued inputs with |partial sums| < 2^24 are exact in any order
    rng = np.random.default_rng(2)
    A = rng.integers(-8, 9, (40, 70)).astype(np.float32)
    B = rng.integers(-8, 9, (70, 33)).astype(np.float32)
    ref = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)
    assert np.array_equal(O.matmul_scalar(A, B), ref)
    assert np.array_equal(O.matmul_avx(A, B), ref)


def test_matmul_avx_matches_scalar_within_metric():
    A = O.uniform(130 * 300, 8).reshape(130, 300)
    B = O.uniform(300 * 77, 9).reshape(300, 77)
    assert gemm_err(O.matmul_avx(A, B), A, B) < 1e-6
    assert gemm_err(O.matmul_scalar(A, B), A, B) < 1e-6


# ------------------------------------------------- golden: ops pico lacks
def test_xent_golden():
    z, y = GOLD["xent_z"], GOLD["xent_y"]
    R = z.shape[0]
    rows, dz = O.xent(z, y, scale=1.0 / R)
    assert row_err(rows, GOLD["xent_rows"]) < 1e-5
    assert abs(rows.mean() - GOLD["xent_loss"]) < 1e-5
    assert max_rel(dz, GOLD["xent_dz"]) < 1e-5


def test_xent_invariants():
    R, V = 3, 50
    z = np.full((R, V), 0.7, np.float32)
    y = np.array([0, 49, 7], np.int32)
    rows, dz = O.xent(z, y)
    assert np.allclose(rows, np.log(V), rtol=1e-6)  # constant logits -> ln V
    assert np.allclose(dz.sum(1), 0.0, atol=1e-6)  # gradient rows sum to zero
    assert np.allclose(dz[np.arange(R), y], 1.0 / V - 1.0, atol=1e-6)
    rows, dz = O.xent(z, np.array([-1, 50, 3], np.int32))  # out-of-range labels
    assert np.isnan(rows[0]) and np.isnan(rows[1]) and not np.any(dz[:2])


def test_rmsnorm_golden_and_invariants():
    x, w, dy, eps = GOLD["rms_x"], GOLD["rms_w"], GOLD["rms_dy"], float(GOLD["rms_eps"])
    y, rstd = O.rmsnorm_fwd(x, w, eps)
    assert max_rel(y, GOLD["rms_y"]) < 1e-6
    dx, dw = O.rmsnorm_bwd(x, w, rstd, dy)
    assert max_rel(dx, GOLD["rms_dx"]) < 1e-5 and max_rel(dw, GOLD["rms_dw"]) < 1e-5
    y1, _ = O.rmsnorm_fwd(x, np.ones_like(w), eps)  # unit gain -> rms(y) = 1
    assert np.allclose(np.sqrt((y1.astype(np.float64) ** 2).mean(1)), 1.0, atol=1e-5)


def test_swiglu_golden_and_invariants():
    a, u, dh = GOLD["swi_a"], GOLD["swi_u"], GOLD["swi_dh"]
    assert max_rel(O.swiglu_fwd(a, u), GOLD["swi_h"]) < 1e-6
    da, du = O.swiglu_bwd(a, u, dh)
    assert max_rel(da, GOLD["swi_da"]) < 1e-6 and max_rel(du, GOLD["swi_du"]) < 1e-6
    assert not np.any(O.swiglu_fwd(np.zeros(5, np.float32), np.ones(5, np.float32)))


def test_attention_golden_and_invariants():
    B, H = int(GOLD["att_B"]), int(GOLD["att_H"])
    q, k, v, do = GOLD["att_q"], GOLD["att_k"], GOLD["att_v"], GOLD["att_do"]
    o, lse = O.attn_fwd(B, H, q, k, v)
    assert max_rel(o, GOLD["att_o"]) < 1e-5 and max_rel(lse, GOLD["att_lse"]) < 1e-5
    dq, dk, dv = O.attn_bwd(B, H, q, k, v, o, lse, do)
    for got, key in ((dq, "att_dq"), (dk, "att_dk"), (dv, "att_dv")):
        assert max_rel(got, GOLD[key]) < 1e-5, key
    # causal row 0 attends only to itself: o_0 = v_0 for every head and sequence
    T = q.shape[0] // B
    for b in range(B):
        assert np.allclose(o[b * T], v[b * T], atol=1e-6)


def test_embedding_golden():
    out = O.embed_fwd(GOLD["emb_ids"], GOLD["emb_table"])
    assert np.array_equal(out, GOLD["emb_out"].astype(np.float32))
    dt = O.embed_bwd(GOLD["emb_ids"], GOLD["emb_dout"], np.zeros_like(GOLD["emb_table"]))
    assert max_rel(dt, GOLD["emb_dtable"]) < 1e-6


def test_adamw_golden_and_first_step_closed_form():
    lr, b1, b2, eps, wd = (float(x) for x in GOLD["adamw_hparams"])
    p = GOLD["adamw_p0"].copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    for s in range(3):
        O.adamw(p, GOLD["adamw_g"][s], m, v, lr, b1, b2, eps, wd, s + 1)
        assert max_rel(p, GOLD["adamw_p"][s]) < 1e-6
    # first step from zero moments: p(1 - lr*wd) - lr * g/(|g| + eps)
    p0 = GOLD["adamw_p0"].astype(np.float64)
    g0 = GOLD["adamw_g"][0].astype(np.float64)
    closed = p0 * (1 - lr * wd) - lr * g0 / (np.abs(g0) + eps)
    assert max_rel(GOLD["adamw_p"][0], closed) < 1e-7


def test_argmax_golden():
    assert np.array_equal(O.argmax(GOLD["argmax_x"]), GOLD["argmax_idx"])


# ------------------------------------ finite differences on the new ops
def _fd_check(f, x, dfdx, eps=1e-3, n=6, seed=0):
    rng = np.random.default_rng(seed)
    for idx in rng.choice(x.size, size=min(n, x.size), replace=False):
        xp, xm = x.copy().ravel(), x.copy().ravel()
        xp[idx] += eps
        xm[idx] -= eps
        num = (f(xp.reshape(x.shape)) - f(xm.reshape(x.shape))) / (2 * eps)
        assert abs(num - dfdx.ravel()[idx]) < 2e-2 * max(1.0, abs(num)), (idx, num)


def test_fd_rmsnorm_and_xent():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 8)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(8)).astype(np.float32)
    dy = rng.standard_normal((3, 8)).astype(np.float32)
    y, rstd = O.rmsnorm_fwd(x, w, 1e-6)
    dx, _ = O.rmsnorm_bwd(x, w, rstd, dy)
    _fd_check(lambda xx: float((O.rmsnorm_fwd(xx, w, 1e-6)[0].astype(np.float64) * dy).sum()),
              x, dx)
    z = rng.standard_normal((4, 9)).astype(np.float32)
    y = rng.integers(0, 9, 4).astype(np.int32)
    _, dz = O.xent(z, y, scale=1.0)
    _fd_check(lambda zz: float(O.xent(zz, y, want_grad=False)[0].astype(np.float64).sum()), z, dz)
