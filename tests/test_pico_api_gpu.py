"""pico's C API over GPU tensors (libpico_amd.so), tested the way the
reference tests itself: its known-answer tests from tests/test_autograd.c,
tests/nn/test_linear.c, tests/optim/test_optim.c and tests/act/
test_activations.c run through the GPU library with exact comparisons, and
whole graphs (forward + pico_backward) compared with the CPU oracle's pico
API on the same seeded inputs.

Bar: bit-exact where the arithmetic is exact or order-free (the KATs,
broadcast add/sub/mul, relu, SGD); max relative error <= 1e-4 otherwise.
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as O
from pico_amd.pico import Pico, PicoError, TP
from tests._util import max_rel

pytestmark = pytest.mark.gpu
TOL = 1e-4
HOOK = ctypes.CFUNCTYPE(None, TP)


@pytest.fixture(scope="module")
def P():
    return Pico()


@pytest.fixture(scope="module")
def C():
    return Pico(O.lib(), device=False)


def hook(t):
    """call t->_backward(t) directly, as the reference's tests do"""
    HOOK(t.contents._backward)(t)


# ------------------------------------------------------------------ matmul
def test_matmul_forward_kats(P):
    # tests/test_autograd.c:286, :318, :482
    with P.arena():
        a = P.param([2, 3], [1, 2, 3, 4, 5, 6])
        b = P.param([3, 2], [7, 8, 9, 10, 11, 12])
        c = P.matmul(a, b)
        assert P.shape(c) == (2, 2)
        assert P.data(c).tolist() == [58, 64, 139, 154]
        s = P.matmul(P.param([2, 2], [1, 2, 3, 4]), P.param([2, 2], [5, 6, 7, 8]))
        assert P.data(s).tolist() == [19, 22, 43, 50]
        d = P.matmul(P.param([1, 3], [1, 2, 3]), P.param([3, 1], [4, 5, 6]))
        assert P.data(d).tolist() == [32]


def test_matmul_backward_kats(P):
    # tests/test_autograd.c:348 (square) and :382 (non-square), dC = ones
    with P.arena():
        a = P.param([2, 2], [1, 2, 3, 4])
        b = P.param([2, 2], [5, 6, 7, 8])
        c = P.matmul(a, b)
        P.backward(c)
        assert P.grad(a).tolist() == [11, 15, 11, 15]
        assert P.grad(b).tolist() == [4, 4, 6, 6]
        a = P.param([2, 3], [1, 2, 3, 4, 5, 6])
        b = P.param([3, 2], [7, 8, 9, 10, 11, 12])
        P.backward(P.matmul(a, b))
        assert P.grad(a).tolist() == [15, 19, 23, 15, 19, 23]
        assert P.grad(b).tolist() == [5, 5, 7, 7, 9, 9]


def test_matmul_shared_parent_and_chain(P):
    # tests/test_autograd.c:559: C = A.A -> dA = dC.A^T + A^T.dC = [7, 11, 9, 13]
    with P.arena():
        a = P.param([2, 2], [1, 2, 3, 4])
        P.backward(P.matmul(a, a))
        assert P.grad(a).tolist() == [7, 11, 9, 13]
    # :517 matmul then add: out = A.B + bias, seeded through pico_backward
    with P.arena():
        a = P.param([2, 2], [1, 2, 3, 4])
        b = P.param([2, 2], [5, 6, 7, 8])
        bias = P.param([2], [1, 1])
        out = P.add(P.matmul(a, b), bias)
        P.backward(out)
        assert P.data(out).tolist() == [20, 23, 44, 51]
        assert P.grad(a).tolist() == [11, 15, 11, 15]
        assert P.grad(bias).tolist() == [2, 2]


def test_weight_grad_side_stream_orders_with_main_stream_writes(P):
    # x.W with x an activation puts dW on the side stream; W*W feeding a
    # second product writes W's grad on the main stream.  Both contributions
    # land, whichever runs first: dW[i][k] = s_i (1 + 2 W[i][k]) with
    # s = column sums of x = (5, 7, 9).  A second graph over the same W then
    # adds the same again (its intermediates are fresh).
    w = [1, -2, 3, 0, 2, -1, 4, 1, -3]
    W = P.param([3, 3], w)
    want = [s * (1 + 2 * v) for s, v in zip([5] * 3 + [7] * 3 + [9] * 3, w)]
    for rep in (1, 2):
        with P.arena():
            x = P.tensor([2, 3], [1, 2, 3, 4, 5, 6])
            P.backward(P.add(P.matmul(x, W), P.matmul(x, P.mul(W, W))))
            assert P.grad(W).tolist() == [rep * v for v in want]
    P.free(W)


def test_split_cols_views_share_data_and_grad(P):
    # t = x.W [2, 6] split into three [2, 2] column views.  v0 feeds v0*v0, v2
    # feeds the sum directly and v1 feeds nothing, so dt = [2*v0 | 0 | 1] and
    # dW = x^T.dt; every value is a small integer, so the check is exact.
    x_v = [1, 2, 3, 4]
    w = [1, 0, 2, -1, 1, 3, 0, 1, -2, 1, 2, -1]
    with P.arena():
        x = P.tensor([2, 2], x_v)
        W = P.param([2, 6], w)
        t = P.matmul(x, W)
        v0, v1, v2 = P.split_cols(t, 3)
        tv = np.array(x_v, float).reshape(2, 2) @ np.array(w, float).reshape(2, 6)
        assert np.array_equal(P.value(t), tv)
        for i, v in enumerate((v0, v1, v2)):
            # the views are windows into t's storage: same data and grad, 2*i floats in
            assert P.shape(v) == (2, 2) and P.strides(v) == (6, 1)
            assert (ctypes.cast(v.contents.data, ctypes.c_void_p).value ==
                    ctypes.cast(t.contents.data, ctypes.c_void_p).value + 8 * i)
            assert (ctypes.cast(v.contents.grad, ctypes.c_void_p).value ==
                    ctypes.cast(t.contents.grad, ctypes.c_void_p).value + 8 * i)
        P.backward(P.add(P.mul(v0, v0), v2))
        dt = np.concatenate([2 * tv[:, 0:2], np.zeros((2, 2)), np.ones((2, 2))], 1)
        want = np.array(x_v, float).reshape(2, 2).T @ dt
        assert np.array_equal(P.grad_value(W), want)
        # a view of a view, a param and a non-divisible width are refused
        with pytest.raises(PicoError):
            P.split_cols(v0, 2)
        with pytest.raises(PicoError):
            P.split_cols(W, 2)
        with pytest.raises(PicoError):
            P.split_cols(t, 4)
    P.free(W)


def test_matmul_transposed_view_matches_oracle(P, C):
    # a pico_transpose_2d view (tensor.c:230-244) is read as 'T' and its grad
    # lands with the view's strides, as the reference's backward loops index it
    rng = np.random.default_rng(3)
    av = rng.integers(-4, 5, (5, 7)).astype(np.float32)
    bv = rng.integers(-4, 5, (5, 6)).astype(np.float32)
    res = []
    for L in (P, C):
        with L.arena():
            a = L.param([5, 7], av)
            b = L.param([5, 6], bv)
            L.transpose_2d(a)  # a is now a [7, 5] view
            c = L.matmul(a, b)
            L.backward(c)
            res.append((L.data(c), L.grad(a), L.grad(b)))
    for x, y in zip(*res):
        assert np.array_equal(x, y)


def test_matmul_refusals(P, capfd):
    with P.arena():
        a = P.param([2, 3])
        with pytest.raises(PicoError):
            P.matmul(a, P.param([2, 2]))  # K mismatch (ops.c:145-148)
        with pytest.raises(PicoError):
            P.matmul(P.param([2, 2, 2]), P.param([2, 2]))  # not 2-D (ops.c:150-153)
    with pytest.raises(PicoError):  # no arena in context (ops.c:160-164)
        P.matmul(P.param([2, 2]), P.param([2, 2]))
    assert "[Pico] Error:" in capfd.readouterr().err


# --------------------------------------------------------------- broadcast
def test_broadcast_backward_kats(P):
    g = [1, 2, 3, 4]
    with P.arena():
        # add_row (test_autograd.c:591): (2,2)+(2,)
        a, b = P.param([2, 2]), P.param([2])
        c = P.add(a, b)
        assert P.shape(c) == (2, 2)
        P.set_grad(c, g)
        hook(c)
        assert P.grad(a).tolist() == [1, 2, 3, 4] and P.grad(b).tolist() == [4, 6]
        # add_col (:627): (2,2)+(2,1)
        a, b = P.param([2, 2]), P.param([2, 1])
        c = P.add(a, b)
        P.set_grad(c, g)
        hook(c)
        assert P.grad(b).tolist() == [3, 7]
        # sub_row (:654)
        a, b = P.param([2, 2]), P.param([2])
        c = P.sub(a, b)
        P.set_grad(c, g)
        hook(c)
        assert P.grad(a).tolist() == [1, 2, 3, 4] and P.grad(b).tolist() == [-4, -6]
        # mul forward (same shape and broadcast) and mul_row backward (:828)
        c = P.mul(P.param([3], [1, 2, 3]), P.param([3], [4, 5, 6]))
        assert P.data(c).tolist() == [4, 10, 18]
        a, b = P.param([2, 2], [1, 2, 3, 4]), P.param([2], [10, 20])
        c = P.mul(a, b)
        assert P.data(c).tolist() == [10, 40, 30, 80]
        P.set_grad(c, g)
        hook(c)
        assert P.grad(a).tolist() == [10, 40, 30, 80] and P.grad(b).tolist() == [10, 20]
        # mul backward_same_shape and backward_accumulates
        a, b = P.param([2], [2, 3]), P.param([2], [4, 5])
        c = P.mul(a, b)
        P.set_grad(c, [10, 100])
        hook(c)
        assert P.grad(a).tolist() == [40, 500] and P.grad(b).tolist() == [20, 300]
        a, b = P.param([1], [3]), P.param([1], [7])
        c = P.mul(a, b)
        P.set_grad(c, [1])
        hook(c)
        hook(c)
        assert P.grad(a).tolist() == [14] and P.grad(b).tolist() == [6]
        # add_row through pico_backward (:865)
        a, b = P.param([2, 2]), P.param([2])
        P.backward(P.add(a, b))
        assert P.grad(a).tolist() == [1, 1, 1, 1] and P.grad(b).tolist() == [2, 2]


@pytest.mark.parametrize("sa,sb", [((3, 5), (3, 5)), ((4, 6), (6,)), ((4, 6), (4, 1)),
                                   ((2, 3, 4), (3, 1)), ((5, 1, 3), (1, 4, 1)), ((7,), (1,))])
def test_broadcast_graph_bitexact_vs_oracle(P, C, sa, sb):
    """((a + b) * b - a) through pico_backward, GPU vs the CPU oracle"""
    av = O.normal(int(np.prod(sa)), 1).reshape(sa)
    bv = O.normal(int(np.prod(sb)), 2).reshape(sb)
    res = []
    for L in (P, C):
        with L.arena():
            a, b = L.param(list(sa), av), L.param(list(sb), bv)
            out = L.sub(L.mul(L.add(a, b), b), a)
            L.backward(out)
            res.append((L.data(out), L.grad(a), L.grad(b)))
    for x, y in zip(*res):
        assert np.array_equal(x, y)


# ------------------------------------------------------------ relu, unary
def test_relu_kats_and_gate(P):
    # tests/act/test_activations.c: relu(x) = max(x, 0); gate closed at x = 0
    with P.arena():
        x = P.param([5], [-2, -0.5, 0, 0.5, 3])
        y = P.relu(x)
        assert P.data(y).tolist() == [0, 0, 0, 0.5, 3]
        P.backward(y)
        assert P.grad(x).tolist() == [0, 0, 0, 1, 1]


@pytest.mark.parametrize("op", ["sqrt", "sin", "cos", "tan", "tanh", "log"])
def test_unary_graph_vs_oracle(P, C, op):
    xv = O.uniform(300, 4, 0.1, 1.3)
    res = []
    for L in (P, C):
        with L.arena():
            x = L.param([300], xv)
            y = getattr(L, op)(x)
            L.backward(y)
            res.append((L.data(y), L.grad(x)))
    assert max_rel(res[0][0], res[1][0]) <= 1e-6
    assert max_rel(res[0][1], res[1][1]) <= 1e-6


# ------------------------------------------------------------ SGD, Linear
def test_sgd_kats(P):
    # tests/optim/test_optim.c:16-92
    with P.arena():
        w = P.param([1], [10])
        P.set_grad(w, [4])
        opt = P.optim_sgd_init(0.5)
        P.optim_sgd_add(opt, w)
        P.optim_sgd_step(opt)
        assert P.data(w).tolist() == [8]
        w3 = P.param([3], [2, 4, 6])
        P.set_grad(w3, [2, 4, 6])
        o3 = P.optim_sgd_init(0.5)
        P.optim_sgd_add(o3, w3)
        P.optim_sgd_step(o3)
        assert P.data(w3).tolist() == [1, 2, 3]
        P.optim_sgd_zero_grad(o3)
        assert P.grad(w3).tolist() == [0, 0, 0]
        P.optim_sgd_free(opt)
        P.optim_sgd_free(o3)


def test_linear_backward_and_training(P):
    # tests/nn/test_linear.c:262 and :297 with the MSE of one sample written as
    # (out - t)^2 through pico ops: W.grad = [-10, -20], b.grad = -10, l1 = 25
    with P.arena():
        fc = P.nn_linear_init(2, 1, True)
        lin = ctypes.cast(fc, ctypes.POINTER(ctypes.c_int * 2))
        assert list(lin.contents) == [2, 1]
        x = P.param([1, 2], [1, 2])
        t = P.param([1, 1], [5])
        opt = P.optim_sgd_init(0.01)
        w = ctypes.cast(fc + 8, ctypes.POINTER(TP)).contents
        b = ctypes.cast(fc + 16, ctypes.POINTER(TP)).contents
        P.optim_sgd_add(opt, w)
        P.optim_sgd_add(opt, b)
        losses = []
        for step in range(5):
            d = P.sub(P.nn_linear_forward(fc, x), t)
            loss = P.mul(d, d)
            losses.append(float(P.data(loss)[0]))
            P.optim_sgd_zero_grad(opt)
            P.backward(loss)
            if step == 0:
                assert P.grad(w).tolist() == [-10, -20] and P.grad(b).tolist() == [-10]
            P.optim_sgd_step(opt)
        assert losses[0] == 25.0
        assert all(l2 < l1 for l1, l2 in zip(losses, losses[1:]))
        P.optim_sgd_free(opt)
        P.nn_linear_free(fc)


# ------------------------------------------------------- lazy-grad semantics
def test_grad_starts_zero_and_accumulates_across_backward_calls(P):
    with P.arena():
        a = P.param([3], [1, 2, 3])
        unused = P.param([3], [4, 5, 6])
        assert P.grad(a).tolist() == [0, 0, 0]
        out = P.mul(a, a)
        P.backward(out)
        P.backward(out)  # no zero_grad: contributions add (autograd.h:25-29)
        assert P.grad(a).tolist() == [4, 8, 12]
        assert P.grad(unused).tolist() == [0, 0, 0]
        t = P.tensor([4])  # pico_create_tensor zeroes data and grad
        assert P.data(t).tolist() == [0, 0, 0, 0] and P.grad(t).tolist() == [0, 0, 0, 0]


def _ptr(p):
    return ctypes.cast(p, ctypes.c_void_p).value


def test_add_backward_aliases_grads_and_second_backward_unaliases(P, C):
    # c = x*x + y*y, d = c*w: c's grad is w, and both operands of the add take
    # it as it is -- their grads point at c's -- so dx = 2 x w, dy = 2 y w.
    # Backward twice over the same graph (intermediate grads keep their values
    # and propagate again, as in the reference) and once more through a + a
    # must match the CPU library value for value; the GPU operands get their
    # own buffers back before anything accumulates into them.
    xv, yv, wv = [1, 2, 3, 4], [2, 0, -1, 3], [1, -2, 3, 5]
    runs = []
    for L in (P, C):
        seen = []
        with L.arena():
            x, y, w = L.param([4], xv), L.param([4], yv), L.param([4], wv)
            a, b = L.mul(x, x), L.mul(y, y)
            c = L.add(a, b)
            d = L.mul(c, w)
            L.backward(d)
            if L is P:
                assert _ptr(a.contents.grad) == _ptr(c.contents.grad) == _ptr(b.contents.grad)
            seen.append([L.grad(t).tolist() for t in (a, b, c, x, y, w)])
            L.backward(d)
            if L is P:
                assert len({_ptr(t.contents.grad) for t in (a, b, c)}) == 3
            seen.append([L.grad(t).tolist() for t in (a, b, c, x, y, w)])
            L.backward(L.add(a, a))
            seen.append([L.grad(t).tolist() for t in (a, b, c, x, y, w)])
        runs.append(seen)
    assert runs[0] == runs[1]
    first = runs[0][0]
    assert first[:3] == [wv] * 3
    assert first[3] == [2 * u * v for u, v in zip(xv, wv)]
    assert first[4] == [2 * u * v for u, v in zip(yv, wv)]


def _residual_graph(L, pv, gv, wv):
    # two pre-norm residual steps, c = a + matmul(rmsnorm(a), W): a's grad is
    # the sum of the add's (aliased) and RMSNorm's contributions
    p = [L.param(list(v.shape), v) for v in pv]
    g = [L.param(list(v.shape), v) for v in gv]
    W = [L.param(list(v.shape), v) for v in wv]
    a = L.mul(p[0], p[1])
    o1 = L.matmul(L.rmsnorm(a, g[0], 1e-6), W[0])
    c1 = L.add(a, o1)
    o2 = L.matmul(L.rmsnorm(c1, g[1], 1e-6), W[1])
    c2 = L.add(c1, o2)
    L.backward(c2)
    return [a, o1, c1, o2, c2] + p + g + W


def test_residual_add_grads_vs_oracle(P, C):
    R, D = 64, 96
    pv = [O.normal(R * D, 1).reshape(R, D), O.normal(R * D, 2).reshape(R, D)]
    gv = [O.normal(D, 3, 1.0, 0.02), O.normal(D, 4, 1.0, 0.02)]
    wv = [O.normal(D * D, 5, 0.0, 0.1).reshape(D, D), O.normal(D * D, 6, 0.0, 0.1).reshape(D, D)]
    out = []
    for L in (P, C):
        with L.arena(1 << 22):
            nodes = _residual_graph(L, pv, gv, wv)
            out.append([L.grad(t) for t in nodes])
    for i, (g, c) in enumerate(zip(*out)):
        assert max_rel(g, c) <= TOL, i


def test_backward_completes_without_split_k_scratch(P, C):
    """A matmul product runs unsplit when its optional split-K scratch cannot be
    had (pico_gpu_fail_next_workspaces refuses it as an out-of-memory would).
    That is no error: pico_backward carries on to the hooks after it, and every
    grad matches the oracle.  Weight gradients with K = 4096 rows and under 256
    output tiles take split-K scratch, on the side stream (W2, W1) and on the
    main stream (x . W1 with x a parameter too)."""
    R, D, F = 4096, 128, 96
    xv = O.normal(R * D, 1).reshape(R, D)
    w1 = O.normal(D * F, 2, 0.0, 0.1).reshape(D, F)
    w2 = O.normal(F * 64, 3, 0.0, 0.1).reshape(F, 64)
    out = []
    for L, fail in ((P, 0), (P, 8), (C, 0)):
        with L.arena(1 << 24):
            x = L.tensor([R, D], xv)
            W1, W2, X2 = L.param([D, F], w1), L.param([F, 64], w2), L.param([R, D], xv)
            y = L.add(L.matmul(L.matmul(x, W1), W2), L.matmul(L.matmul(X2, W1), W2))
            if fail:
                L.lib.pico_gpu_fail_next_workspaces(fail)
            L.backward(y)  # raises on a recorded error
            if fail:
                L.lib.pico_gpu_fail_next_workspaces(0)
                assert L.lib.pico_gpu_last_error() == b""
            out.append([L.grad(t) for t in (W1, W2, X2)])
            for t in (W1, W2, X2):
                L.free(t)
    for i in range(3):
        assert max_rel(out[0][i], out[2][i]) <= TOL, i
        assert max_rel(out[1][i], out[2][i]) <= TOL, i


# ------------------------------------------------------ new hot-path ops
def _new_ops_graph(L, gv, wv, ids, labels, table, B, H):
    x = L.embedding(L.param(list(table.shape), table), ids)
    n = L.rmsnorm(x, L.param([gv.size], gv), 1e-6)
    q = L.matmul(n, L.param(list(wv[0].shape), wv[0]))
    k = L.matmul(n, L.param(list(wv[1].shape), wv[1]))
    v = L.matmul(n, L.param(list(wv[2].shape), wv[2]))
    att = L.attention_causal(q, k, v, B, H)
    h = L.swiglu(att, L.add(att, x))
    logits = L.matmul(h, L.param(list(wv[3].shape), wv[3]))
    loss = L.xent(logits, labels)
    L.backward(loss)
    return loss, [x, n, q, k, v, att, h, logits]


@pytest.mark.parametrize("B,T,H,hd", [(2, 64, 2, 32), (2, 100, 2, 64), (1, 200, 1, 64)])
def test_new_ops_graph_vs_oracle(P, C, B, T, H, hd):
    # head size 32: the chain of GEMMs and softmax kernels; 64 at T 100 and 200:
    # the fused kernels with a padded last query block
    V = 50
    D = H * hd
    table = O.normal(V * D, 1).reshape(V, D)
    gv = O.normal(D, 2, 1.0, 0.02)
    wv = [O.normal(D * D, 3 + i, 0.0, 0.1).reshape(D, D) for i in range(3)]
    wv.append(O.normal(D * V, 9, 0.0, 0.1).reshape(D, V))
    ids = O.labels(B * T, 10, V)
    labels = O.labels(B * T, 11, V)
    out = []
    for L in (P, C):
        with L.arena(1 << 24):
            loss, nodes = _new_ops_graph(L, gv, wv, ids, labels, table, B, H)
            vals = [L.data(loss)] + [L.data(t) for t in nodes] + [L.grad(t) for t in nodes]
            out.append(vals)
    for i, (g, c) in enumerate(zip(*out)):
        assert max_rel(g, c) <= TOL, i


def test_xent_fused_path_matches_recompute(P):
    # loss as the pico_backward entry takes the fused gradient written by the
    # forward; loss * 1 (entry = the product) takes the recompute path scaled by
    # the upstream gradient on the device.  Both must agree.
    R, V = 16, 777
    z = O.normal(R * V, 1, 0.0, 2.0).reshape(R, V)
    y = O.labels(R, 2, V)
    grads = []
    for scaled in (False, True):
        with P.arena():
            zt = P.param([R, V], z)
            loss = P.xent(zt, y)
            entry = P.mul(loss, P.scalar(1.0)) if scaled else loss
            P.backward(entry)
            grads.append(P.grad(zt))
    _, dz = O.xent(z, y, scale=1.0 / R)
    assert max_rel(grads[0], dz.ravel()) <= TOL
    assert max_rel(grads[1], dz.ravel()) <= TOL


# ----------------------------------------------------- config 1: MLP loop
def _mlp_curve(L, steps, x, labels, w1, w2):
    """784 -> 128 -> 10 ReLU MLP, softmax cross-entropy, SGD lr 0.01
    (examples/02_relu_mlp/main.c:64-130 with CE in place of MSE)"""
    losses = []
    with L.arena(1 << 24) as ar:
        fc1 = L.nn_linear_init(784, 128, True)
        fc2 = L.nn_linear_init(128, 10, True)
        params = []
        for fc, w in ((fc1, w1), (fc2, w2)):
            wt = ctypes.cast(fc + 8, ctypes.POINTER(TP)).contents
            bt = ctypes.cast(fc + 16, ctypes.POINTER(TP)).contents
            L.set(wt, w)
            params += [wt, bt]
        opt = L.optim_sgd_init(0.01)
        for p in params:
            L.optim_sgd_add(opt, p)
        xt = L.param([64, 784], x)
        for _ in range(steps):
            h = L.relu(L.nn_linear_forward(fc1, xt))
            loss = L.xent(L.nn_linear_forward(fc2, h), labels)
            losses.append(float(L.data(loss)[0]))
            L.optim_sgd_zero_grad(opt)
            L.backward(loss)
            L.optim_sgd_step(opt)
            L.reset(ar)
        final = [L.data(p) for p in params]
        L.optim_sgd_free(opt)
        L.free(xt)
        L.nn_linear_free(fc1)
        L.nn_linear_free(fc2)
    return np.array(losses), final


def test_config1_mlp_loss_curve_matches_cpu(P, C):
    x = O.normal(64 * 784, 20261201).reshape(64, 784)
    labels = O.labels(64, 20261202, 10)
    w1 = O.uniform(784 * 128, 20261203, -784 ** -0.5, 784 ** -0.5).reshape(784, 128)
    w2 = O.uniform(128 * 10, 20261204, -128 ** -0.5, 128 ** -0.5).reshape(128, 10)
    gpu, gp = _mlp_curve(P, 100, x, labels, w1, w2)
    cpu, cp = _mlp_curve(C, 100, x, labels, w1, w2)
    # tests/test_train.c:22-193: the loss falls at every step
    assert np.all(np.isfinite(gpu)) and np.all(np.diff(gpu) < 0) and gpu[-1] < 0.5 * gpu[0]
    assert max_rel(gpu, cpu) <= TOL
    for g, c in zip(gp, cp):
        assert max_rel(g, c) <= TOL


def test_self_attention_shared_parent_vs_oracle(P, C):
    # attention(x, x, x) through the fused kernels (T 128, head size 64): the
    # three gradient contributions land in one grad buffer
    B, T, H, hd = 2, 128, 2, 64
    D = H * hd
    xv = O.normal(B * T * D, 5).reshape(B * T, D)
    res = []
    for L in (P, C):
        with L.arena(1 << 24):
            x = L.param([B * T, D], xv)
            out = L.attention_causal(x, x, x, B, H)
            L.backward(L.mul(out, out))
            res.append((L.data(out), L.grad(x)))
    assert max_rel(res[0][0], res[1][0]) <= TOL
    assert max_rel(res[0][1], res[1][1]) <= TOL

