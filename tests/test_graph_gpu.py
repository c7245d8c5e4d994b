"""Device graphs (pico_graph_begin / end / launch): one training step recorded
once and replayed must give bit-for-bit the results of running the same steps
eagerly -- the replay launches the same kernels with the same arguments on the
same addresses -- and replayed curves must match the CPU oracle (config 1's 100
SGD steps) and the float64 transformer reference (AdamW steps) within 1e-4.  Each replay is read back and compared, with eager work and
synchronisations between replays.  Also: the multi-tensor AdamW that makes an
optimizer step replayable matches the per-tensor kernel bit for bit, and a
capture that would allocate or copy is refused with a clear error while the
library stays usable."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import kernels as K
from pico_amd.pico import TP, Pico, PicoError

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def P():
    return Pico()


def _device_ids(P, arena, arr):
    """int32 ids copied into `arena` (which must outlive the graph)"""
    a = np.ascontiguousarray(arr, dtype=np.int32)
    P.lib.arena_ctx_push(arena)
    try:
        d = P.lib.pico_ids_to_device(a.ctypes.data_as(ctypes.c_void_p), a.size)
    finally:
        P.lib.arena_ctx_pop()
    assert d
    return d


def _update_ids(P, dev, arr):
    a = np.ascontiguousarray(arr, dtype=np.int32)
    assert P.lib.pico_ids_update(dev, a.ctypes.data_as(ctypes.c_void_p), a.size) == 0


def _eager_noise(P):
    # unrelated eager work between replays, read back (synchronises)
    with P.arena(1 << 20):
        a = P.tensor([3, 5], np.arange(15.0))
        b = P.add(a, a)
        assert np.array_equal(P.data(b), 2.0 * np.arange(15.0, dtype=np.float32))


# ------------------------------------------------------------ multi AdamW
def test_adamw_multi_matches_per_tensor_kernel():
    dev = torch.device("cuda:0")
    sizes = [1, 3, 4, 65536, 65537, 200003, 131072]
    hp = dict(lr=3e-3, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.1)
    single, multi = [], []
    for i, n in enumerate(sizes):
        p = torch.from_numpy(O.normal(n, 100 + i)).to(dev)
        g = None if i == 2 else torch.from_numpy(O.normal(n, 200 + i)).to(dev)
        single.append([p.clone(), g, torch.zeros(n, device=dev), torch.zeros(n, device=dev)])
        multi.append([p.clone(), g, torch.zeros(n, device=dev), torch.zeros(n, device=dev)])
    state = torch.zeros(4, dtype=torch.int32, device=dev)
    keep = []
    for step in range(1, 4):
        for p, g, m, v in single:
            K.adamw(p, g, m, v, hp["lr"], hp["beta1"], hp["beta2"], hp["eps"], hp["wd"], step)
        keep.append(K.adamw_multi(multi, hp["lr"], hp["beta1"], hp["beta2"], hp["eps"], hp["wd"],
                                  state))
    torch.cuda.synchronize()
    assert int(state[0]) == 3
    for a, b in zip(single, multi):
        for x, y in ((a[0], b[0]), (a[2], b[2]), (a[3], b[3])):
            assert torch.equal(x, y)


# -------------------------------------------------------- config 1 (SGD)
def _mlp(P, x, w1, w2):
    fc1 = P.nn_linear_init(784, 128, True)
    fc2 = P.nn_linear_init(128, 10, True)
    params = []
    for fc, w in ((fc1, w1), (fc2, w2)):
        wt = ctypes.cast(fc + 8, ctypes.POINTER(TP)).contents
        bt = ctypes.cast(fc + 16, ctypes.POINTER(TP)).contents
        P.set(wt, w)
        params += [wt, bt]
    opt = P.optim_sgd_init(0.01)
    for p in params:
        P.optim_sgd_add(opt, p)
    return fc1, fc2, params, opt, P.param([64, 784], x)


def _mlp_step(P, fc1, fc2, opt, xt, labels_dev):
    P.optim_sgd_zero_grad(opt)
    h = P.relu(P.nn_linear_forward(fc1, xt))
    loss = P.softmax_xent(P.nn_linear_forward(fc2, h), labels_dev)
    P.backward(loss)
    P.optim_sgd_step(opt)
    return loss


def test_mlp_sgd_graph_replay_matches_eager(P):
    x = O.normal(64 * 784, 31).reshape(64, 784)
    w1 = O.uniform(784 * 128, 32, -784 ** -0.5, 784 ** -0.5).reshape(784, 128)
    w2 = O.uniform(128 * 10, 33, -128 ** -0.5, 128 ** -0.5).reshape(128, 10)
    batches = [O.labels(64, 40 + s, 10) for s in range(6)]
    results = []
    for use_graph in (False, True):
        ids_arena = P.lib.arena_init(1 << 16)
        losses = []
        with P.arena(1 << 24) as ar:
            fc1, fc2, params, opt, xt = _mlp(P, x, w1, w2)
            labels = _device_ids(P, ids_arena, batches[0])
            loss = _mlp_step(P, fc1, fc2, opt, xt, labels)  # eager warm-up step
            losses.append(float(P.data(loss)[0]))
            P.reset(ar)
            graph = None
            if use_graph:
                assert P.lib.pico_graph_begin() == 0
                loss = _mlp_step(P, fc1, fc2, opt, xt, labels)
                graph = P.lib.pico_graph_end()
                assert graph, P.lib.pico_gpu_last_error()
            for s in range(1, len(batches)):
                _update_ids(P, labels, batches[s])
                if use_graph:
                    assert P.lib.pico_graph_launch(graph) == 0
                    losses.append(float(P.data(loss)[0]))
                    _eager_noise(P)
                else:
                    loss = _mlp_step(P, fc1, fc2, opt, xt, labels)
                    losses.append(float(P.data(loss)[0]))
                    P.reset(ar)
            final = [P.data(p) for p in params]
            if graph:
                P.lib.pico_graph_free(graph)
            P.optim_sgd_free(opt)
            P.free(xt)
            P.nn_linear_free(fc1)
            P.nn_linear_free(fc2)
        P.lib.arena_destroy(ids_arena)
        results.append((np.array(losses), final))
    (l0, p0), (l1, p1) = results
    # fresh random labels every step: the losses move but need not fall
    assert np.all(np.isfinite(l0)) and len(set(l0.tolist())) == len(l0)
    assert np.array_equal(l0, l1)
    for a, b in zip(p0, p1):
        assert np.array_equal(a, b)


def test_mlp_graph_replay_loss_curve_matches_cpu_oracle(P):
    """Config 1's 100 SGD steps with the step captured once and replayed 99
    times, against the CPU oracle's pico API (pico's own loops restated) running
    the same 100 steps eagerly: every loss and the final weights within 1e-4.
    The replay is compared with the CPU here, not only with eager GPU steps,
    so an error shared by both GPU paths would show."""
    from tests._util import max_rel

    C = Pico(O.lib(), device=False)
    x = O.normal(64 * 784, 20261201).reshape(64, 784)
    labels = O.labels(64, 20261202, 10)
    w1 = O.uniform(784 * 128, 20261203, -784 ** -0.5, 784 ** -0.5).reshape(784, 128)
    w2 = O.uniform(128 * 10, 20261204, -128 ** -0.5, 128 ** -0.5).reshape(128, 10)
    steps = 100
    # CPU oracle, eager
    cpu = []
    with C.arena(1 << 24) as ar:
        fc1, fc2, params, opt, xt = _mlp(C, x, w1, w2)
        for _ in range(steps):
            loss = _mlp_step(C, fc1, fc2, opt, xt, C.ids(labels))
            cpu.append(float(C.data(loss)[0]))
            C.reset(ar)
        cpu_final = [C.data(p) for p in params]
        C.optim_sgd_free(opt)
        C.free(xt)
        C.nn_linear_free(fc1)
        C.nn_linear_free(fc2)
    # GPU: one eager step, then the captured step replayed
    ids_arena = P.lib.arena_init(1 << 16)
    gpu = []
    with P.arena(1 << 24) as ar:
        fc1, fc2, params, opt, xt = _mlp(P, x, w1, w2)
        dlab = _device_ids(P, ids_arena, labels)
        gpu.append(float(P.data(_mlp_step(P, fc1, fc2, opt, xt, dlab))[0]))
        P.reset(ar)
        assert P.lib.pico_graph_begin() == 0
        loss = _mlp_step(P, fc1, fc2, opt, xt, dlab)
        graph = P.lib.pico_graph_end()
        assert graph, P.lib.pico_gpu_last_error()
        for s in range(1, steps):
            assert P.lib.pico_graph_launch(graph) == 0
            gpu.append(float(P.data(loss)[0]))
            if s % 25 == 0:
                _eager_noise(P)
        gpu_final = [P.data(p) for p in params]
        P.lib.pico_graph_free(graph)
        P.optim_sgd_free(opt)
        P.free(xt)
        P.nn_linear_free(fc1)
        P.nn_linear_free(fc2)
    P.lib.arena_destroy(ids_arena)
    gpu, cpu = np.array(gpu), np.array(cpu)
    assert np.all(np.diff(gpu) < 0) and gpu[-1] < 0.5 * gpu[0]
    assert max_rel(gpu, cpu) <= 1e-4
    for g, c in zip(gpu_final, cpu_final):
        assert max_rel(g, c) <= 1e-4


def test_gpt_graph_replay_loss_curve_matches_float64_reference(P):
    """A small transformer's AdamW steps (one eager, then the captured step
    replayed 9 times on one batch) against the float64 reference's 10 steps
    (oracle/gpt_ref.py with its own AdamW): losses within 1e-4."""
    from oracle import gpt_ref as G
    from tests._util import max_rel

    cfg = dict(vocab=96, d_model=64, n_layers=2, n_heads=2, d_ff=160, batch=2, seq_len=64)
    hp = dict(lr=1e-3, b1=0.9, b2=0.95, eps=1e-8, wd=0.1)
    seq = O.labels(cfg["batch"] * (cfg["seq_len"] + 1), 91, cfg["vocab"])
    seq = seq.reshape(cfg["batch"], cfg["seq_len"] + 1)
    tokens, targets = seq[:, :-1].ravel().copy(), seq[:, 1:].ravel().copy()
    steps = 10
    model = P.gpt_init(cfg, 92)
    tensors = P.gpt_params(model)
    ref_params = [p.astype(np.float64) for p in
                  G.split_fused([P.value(t) for t in tensors], cfg)]
    opt = P.optim_adamw_init(hp["lr"], hp["b1"], hp["b2"], hp["eps"], hp["wd"])
    for t in tensors:
        P.optim_adamw_add(opt, t)
    ids_arena = P.lib.arena_init(1 << 20)
    tok = _device_ids(P, ids_arena, tokens)
    tgt = _device_ids(P, ids_arena, targets)

    def step():
        P.optim_adamw_zero_grad(opt)
        loss = P.gpt_loss(model, tok, tgt)
        P.backward(loss)
        P.optim_adamw_step(opt)
        return loss

    gpu = []
    with P.arena(1 << 26) as ar:
        gpu.append(float(P.data(step())[0]))
        P.reset(ar)
        assert P.lib.pico_graph_begin() == 0
        loss = step()
        graph = P.lib.pico_graph_end()
        assert graph, P.lib.pico_gpu_last_error()
        for _ in range(1, steps):
            assert P.lib.pico_graph_launch(graph) == 0
            gpu.append(float(P.data(loss)[0]))
        P.lib.pico_graph_free(graph)
    P.optim_adamw_free(opt)
    P.gpt_free(model)
    P.lib.arena_destroy(ids_arena)
    ref = []
    m = [np.zeros_like(p) for p in ref_params]
    v = [np.zeros_like(p) for p in ref_params]
    for s in range(1, steps + 1):
        loss, grads = G.loss_and_grads(ref_params, cfg, tokens, targets)
        ref.append(loss)
        for i, g in enumerate(grads):
            ref_params[i], m[i], v[i] = G.adamw(ref_params[i], g.reshape(ref_params[i].shape),
                                               m[i], v[i], s, hp["lr"], hp["b1"], hp["b2"],
                                               hp["eps"], hp["wd"])
    assert gpu[-1] < gpu[0]
    assert max_rel(np.array(gpu), np.array(ref)) <= 1e-4


# ---------------------------------------------------- transformer (AdamW)
@pytest.mark.parametrize("cfg", [
    dict(vocab=96, d_model=64, n_layers=2, n_heads=2, d_ff=160, batch=2, seq_len=64),
    dict(vocab=8192, d_model=512, n_layers=1, n_heads=8, d_ff=1376, batch=16, seq_len=256),
    # the benchmark's 12-layer configuration: the replayed step bench.py times
    pytest.param(dict(vocab=32000, d_model=768, n_layers=12, n_heads=12, d_ff=2048, batch=8,
                      seq_len=1024), marks=[pytest.mark.slow, pytest.mark.timeout(300)]),
])
def test_gpt_adamw_graph_replay_matches_eager(P, cfg):
    batches = []
    for s in range(5):
        seq = O.labels(cfg["batch"] * (cfg["seq_len"] + 1), 70 + s, cfg["vocab"])
        seq = seq.reshape(cfg["batch"], cfg["seq_len"] + 1)
        batches.append((seq[:, :-1].ravel(), seq[:, 1:].ravel()))
    results = []
    for use_graph in (False, True):
        model = P.gpt_init(cfg, 5)
        opt = P.optim_adamw_init(3e-4, 0.9, 0.95, 1e-8, 0.1)
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
            loss = step()  # eager warm-up step
            losses.append(float(P.data(loss)[0]))
            P.reset(ar)
            graph = None
            if use_graph:
                assert P.lib.pico_graph_begin() == 0
                loss = step()
                graph = P.lib.pico_graph_end()
                assert graph, P.lib.pico_gpu_last_error()
            for s in range(1, len(batches)):
                _update_ids(P, tok, batches[s][0])
                _update_ids(P, tgt, batches[s][1])
                if use_graph:
                    assert P.lib.pico_graph_launch(graph) == 0
                    losses.append(float(P.data(loss)[0]))
                    _eager_noise(P)
                else:
                    loss = step()
                    losses.append(float(P.data(loss)[0]))
                    P.reset(ar)
            final = [P.data(p) for p in params]
            if graph:
                P.lib.pico_graph_free(graph)
        P.optim_adamw_free(opt)
        P.gpt_free(model)
        P.lib.arena_destroy(ids_arena)
        results.append((np.array(losses), final))
    (l0, p0), (l1, p1) = results
    assert np.all(np.isfinite(l0)) and len(l0) == 5
    assert np.array_equal(l0, l1)
    for a, b in zip(p0, p1):
        assert np.array_equal(a, b)


# ------------------------------------------------------------ refusals
def test_capture_refuses_allocation_and_copies(P):
    fresh = P.lib.arena_init(1 << 16)
    P.lib.arena_ctx_push(fresh)
    try:
        P.lib.pico_gpu_clear_error()
        assert P.lib.pico_graph_begin() == 0
        # the fresh arena has no device block yet: creating a tensor must allocate
        with pytest.raises(PicoError):
            P.tensor([4, 4])
        assert not P.lib.pico_graph_end()
        assert b"during graph capture" in P.lib.pico_gpu_last_error()
    finally:
        P.lib.arena_ctx_pop()
        P.lib.arena_destroy(fresh)
    with P.arena(1 << 20):
        logits = P.tensor([2, 3], np.zeros(6))
        P.lib.pico_gpu_clear_error()
        assert P.lib.pico_graph_begin() == 0
        # host labels need a synchronous upload: refused
        with pytest.raises(PicoError):
            P.xent(logits, np.array([0, 1], np.int32))
        assert not P.lib.pico_graph_end()
        assert b"during graph capture" in P.lib.pico_gpu_last_error()
        P.lib.pico_gpu_clear_error()
        # the library is usable afterwards
        loss = P.xent(logits, np.array([0, 1], np.int32))
        assert abs(float(P.data(loss)[0]) - np.log(3.0)) < 1e-6
    assert P.lib.pico_graph_launch(None) != 0
    assert not P.lib.pico_graph_end()  # no capture in progress
