"""pico_matmul's fp8 products (PICO_MATMUL_FP8) run through MX8 operands
(pk_mx8_quantize_f32 + pk_gemm_mx8_f32), with a parameter's casts kept and
redone after the parameter changes.  Outside the fp32 parity contract; what
is pinned here is the routing, the kept casts and graph replay:

* a matmul's forward, input gradient and weight gradient equal, bit for bit,
  the same products run straight on the kernels (the MX8 kernels are pinned
  against the format and exact arithmetic in tests/test_fp8q_gpu.py);
* after an SGD step, a host write or a graph replay changes a weight, the
  next product uses the new weight: bit for bit the product of freshly cast
  values, never a stale cast;
* a captured AdamW step of the transformer, replayed, gives bit for bit the
  losses and parameters of the same steps run eagerly.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import kernels as K
from pico_amd.pico import Pico

pytestmark = pytest.mark.gpu


@pytest.fixture
def P():
    P = Pico()
    assert P.lib.pico_set_matmul_precision(3) == 0
    yield P
    assert P.lib.pico_set_matmul_precision(0) == 0


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def mx_product(X, Y):
    """X [M, K] . Y [K, N] through the kernels directly (numpy in and out)"""
    M, Kd = X.shape
    N = Y.shape[1]
    C = torch.empty(M, N, device="cuda")
    K.gemm_mx8(M, N, Kd, K.mx8_quantize(cu(X), False), K.mx8_quantize(cu(Y), True), C)
    torch.cuda.synchronize()
    return C.cpu().numpy()


@pytest.mark.parametrize("M,Kd,N", [(256, 768, 512), (300, 70, 130), (1, 5, 3), (1000, 256, 96)])
def test_pico_matmul_fp8_runs_the_mx8_products(P, M, Kd, N):
    av = O.uniform(M * Kd, 1).reshape(M, Kd)
    wv = O.uniform(Kd * N, 2).reshape(Kd, N) * 0.1
    gv = O.uniform(M * N, 3).reshape(M, N)
    with P.arena(1 << 26):
        a = P.tensor([M, Kd], av)
        w = P.param([Kd, N], wv)
        out = P.matmul(a, w)
        P.backward(P.mul(out, P.tensor([M, N], gv)))
        got = (P.data(out).reshape(M, N), P.grad(a).reshape(M, Kd), P.grad(w).reshape(Kd, N))
        P.free(w)
    assert np.array_equal(got[0], mx_product(av, wv))
    assert np.array_equal(got[1], mx_product(gv, wv.T))      # dA = g . W^T
    assert np.array_equal(got[2], mx_product(av.T, gv))      # dW = A^T . g


def test_pico_matmul_fp8_transposed_view_and_add(P):
    """a transposed view operand and the fused residual add take the same
    MX8 products"""
    M, Kd, N = 192, 160, 288
    av = O.uniform(M * Kd, 4).reshape(M, Kd)
    wtv = O.uniform(N * Kd, 5).reshape(N, Kd) * 0.1   # stored [N, K]; used as its transpose
    cv = O.uniform(M * N, 6).reshape(M, N)
    with P.arena(1 << 26):
        a = P.tensor([M, Kd], av)
        wt = P.param([N, Kd], wtv)
        P.lib.pico_transpose_2d(wt)
        c = P.tensor([M, N], cv)
        out = P.matmul_add(a, wt, c)
        got = P.data(out).reshape(M, N)
        P.lib.pico_transpose_2d(wt)
        P.free(wt)
    prod = mx_product(av, wtv.T)
    assert np.array_equal(got, prod + cv)


def test_fp8_weight_casts_follow_parameter_changes(P):
    M, Kd, N = 256, 384, 256
    av = O.uniform(M * Kd, 7).reshape(M, Kd)
    wv = O.uniform(Kd * N, 8).reshape(Kd, N) * 0.1
    gv = O.uniform(M * N, 9).reshape(M, N)
    opt = P.optim_sgd_init(0.5)
    w = P.param([Kd, N], wv)
    P.optim_sgd_add(opt, w)
    with P.arena(1 << 26) as ar:
        a = P.tensor([M, Kd], av)
        out = P.matmul(a, w)
        assert np.array_equal(P.data(out).reshape(M, N), mx_product(av, wv))
        P.backward(P.mul(out, P.tensor([M, N], gv)))
        P.optim_sgd_step(opt)  # w changes on the device
        w1 = P.data(w).reshape(Kd, N)
        assert not np.array_equal(w1, wv)
        P.reset(ar)
        a = P.tensor([M, Kd], av)
        assert np.array_equal(P.data(P.matmul(a, w)).reshape(M, N), mx_product(av, w1))
        w2 = wv[::-1].copy()
        P.set(w, w2)  # a host write
        assert np.array_equal(P.data(P.matmul(a, w)).reshape(M, N), mx_product(av, w2))
        # the input gradient's layout of the weight follows too
        P.optim_sgd_zero_grad(opt)
        out = P.matmul(a, w)
        P.backward(P.mul(out, P.tensor([M, N], gv)))
        assert np.array_equal(P.grad(a).reshape(M, Kd), mx_product(gv, w2.T))
    P.optim_sgd_free(opt)
    P.free(w)


def _device_ids(P, arena, arr):
    a = np.ascontiguousarray(arr, dtype=np.int32)
    P.lib.arena_ctx_push(arena)
    try:
        d = P.lib.pico_ids_to_device(a.ctypes.data_as(ctypes.c_void_p), a.size)
    finally:
        P.lib.arena_ctx_pop()
    assert d
    return d


@pytest.mark.parametrize("cfg", [
    dict(vocab=96, d_model=64, n_layers=2, n_heads=2, d_ff=160, batch=2, seq_len=64),
    # the benchmark's 12-layer configuration (bench.py's fp8 step)
    pytest.param(dict(vocab=32000, d_model=768, n_layers=12, n_heads=12, d_ff=2048, batch=8,
                      seq_len=1024), marks=[pytest.mark.slow, pytest.mark.timeout(300)]),
])
def test_gpt_fp8_graph_replay_matches_eager(P, cfg):
    """weights change on the device inside every replay (the captured AdamW);
    each replay recasts them, so replays equal eager steps bit for bit"""
    batches = []
    for s in range(5):
        seq = O.labels(cfg["batch"] * (cfg["seq_len"] + 1), 90 + s, cfg["vocab"])
        seq = seq.reshape(cfg["batch"], cfg["seq_len"] + 1)
        batches.append((seq[:, :-1].ravel(), seq[:, 1:].ravel()))
    results = []
    for use_graph in (False, True):
        model = P.gpt_init(cfg, 6)
        opt = P.optim_adamw_init(1e-3, 0.9, 0.95, 1e-8, 0.1)
        params = P.gpt_params(model)
        for p in params:
            P.optim_adamw_add(opt, p)
        ids_arena = P.lib.arena_init(1 << 20)
        tok = _device_ids(P, ids_arena, batches[0][0])
        tgt = _device_ids(P, ids_arena, batches[0][1])

        def step():
            P.optim_adamw_zero_grad(opt)
            loss = P.gpt_loss(model, tok, tgt)
            P.backward(loss)
            P.optim_adamw_step(opt)
            return loss

        losses = []
        with P.arena(1 << 30) as ar:
            loss = step()
            losses.append(float(P.data(loss)[0]))
            P.reset(ar)
            graph = None
            if use_graph:
                assert P.lib.pico_graph_begin() == 0
                loss = step()
                graph = P.lib.pico_graph_end()
                assert graph, P.lib.pico_gpu_last_error()
            for s in range(1, len(batches)):
                for dev_ids, host_ids in ((tok, batches[s][0]), (tgt, batches[s][1])):
                    h = np.ascontiguousarray(host_ids, dtype=np.int32)
                    assert P.lib.pico_ids_update(dev_ids, h.ctypes.data_as(ctypes.c_void_p),
                                                 h.size) == 0
                if use_graph:
                    assert P.lib.pico_graph_launch(graph) == 0
                    losses.append(float(P.data(loss)[0]))
                else:
                    loss = step()
                    losses.append(float(P.data(loss)[0]))
                    P.reset(ar)
            # an eager forward after the replays sees the replayed weights
            P.reset(ar)
            after = float(P.data(P.gpt_loss(model, tok, tgt))[0])
            final = [P.data(p) for p in params]
            if graph:
                P.lib.pico_graph_free(graph)
        P.optim_adamw_free(opt)
        P.gpt_free(model)
        P.lib.arena_destroy(ids_arena)
        results.append((np.array(losses), final, after))
    (l0, p0, a0), (l1, p1, a1) = results
    # uniform random targets: the small model fits them, the 32000-way one stays
    # near ln(vocab) over five steps
    assert np.all(np.isfinite(l0)) and (l0[-1] < l0[0] or cfg["vocab"] > 1000)
    assert np.array_equal(l0, l1)
    assert a0 == a1
    for x, y in zip(p0, p1):
        assert np.array_equal(x, y)
