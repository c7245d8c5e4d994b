"""Checkpoints (pico_checkpoint_save / _load): a run saved after some AdamW
steps and resumed into a fresh model and optimizer continues bit for bit as
the uninterrupted run; the file is a safetensors file any reader opens (the
values, names, shapes, step count and hyper-parameters are checked with the
safetensors package); a mismatched model is refused before anything is
written."""
import ctypes

import numpy as np
import pytest
from safetensors import safe_open
from safetensors.numpy import load_file

from oracle import oracle as O
from pico_amd.pico import TP, Pico

pytestmark = pytest.mark.gpu

CFG = dict(vocab=96, d_model=64, n_layers=2, n_heads=2, d_ff=160, batch=2, seq_len=64)
HP = (3e-4, 0.9, 0.95, 1e-8, 0.1)


@pytest.fixture(scope="module")
def P():
    return Pico()


def _batches(cfg, count, seed):
    out = []
    for s in range(count):
        seq = O.labels(cfg["batch"] * (cfg["seq_len"] + 1), seed + s, cfg["vocab"])
        seq = seq.reshape(cfg["batch"], cfg["seq_len"] + 1)
        out.append((seq[:, :-1].ravel(), seq[:, 1:].ravel()))
    return out


class Run:
    def __init__(self, P, cfg, seed):
        self.P, self.cfg = P, cfg
        self.model = P.gpt_init(cfg, seed)
        self.opt = P.optim_adamw_init(*HP)
        self.params = P.gpt_params(self.model)
        for p in self.params:
            P.optim_adamw_add(self.opt, p)
        self.names = [P.lib.pico_gpt_param_name(self.model, i) for i in range(len(self.params))]

    def steps(self, batches):
        P, losses = self.P, []
        with P.arena(1 << 26) as ar:
            for tok, tgt in batches:
                P.optim_adamw_zero_grad(self.opt)
                loss = P.gpt_loss(self.model, tok, tgt)
                P.backward(loss)
                P.optim_adamw_step(self.opt)
                losses.append(float(P.data(loss)[0]))
                P.reset(ar)
        return losses

    def _args(self, path):
        n = len(self.params)
        arr = (TP * n)(*self.params)
        names = (ctypes.c_char_p * n)(*self.names)
        return str(path).encode(), n, arr, names, self.opt

    def save(self, path):
        return self.P.lib.pico_checkpoint_save(*self._args(path))

    def load(self, path):
        return self.P.lib.pico_checkpoint_load(*self._args(path))

    def values(self):
        return [self.P.data(p) for p in self.params]

    def free(self):
        self.P.optim_adamw_free(self.opt)
        self.P.gpt_free(self.model)


def test_resume_continues_exactly(P, tmp_path):
    batches = _batches(CFG, 5, 300)
    path = tmp_path / "run.safetensors"
    a = Run(P, CFG, 5)
    a.steps(batches[:3])
    assert a.save(path) == 0, P.lib.pico_gpu_last_error()
    la = a.steps(batches[3:])
    pa = a.values()
    a.free()
    b = Run(P, CFG, 99)  # different initial weights, fresh optimizer
    assert b.load(path) == 0, P.lib.pico_gpu_last_error()
    lb = b.steps(batches[3:])
    pb = b.values()
    b.free()
    assert la == lb
    for x, y in zip(pa, pb):
        assert np.array_equal(x, y)


def test_file_is_safetensors(P, tmp_path):
    path = tmp_path / "ck.safetensors"
    r = Run(P, CFG, 7)
    r.steps(_batches(CFG, 2, 400))
    assert r.save(path) == 0
    data = load_file(str(path))
    with safe_open(str(path), framework="np") as f:
        meta = f.metadata()
    names = [n.decode() for n in r.names]
    assert names[0] == "emb" and names[1] == "layers.0.attn_norm" and names[-1] == "lm_head"
    for name, t, v in zip(names, r.params, r.values()):
        assert data[name].dtype == np.float32
        assert list(data[name].shape) == list(P.shape(t))
        assert np.array_equal(data[name].ravel(), v)
        assert data[name + ".adam_m"].shape == data[name].shape
        assert np.any(data[name + ".adam_v"] != 0)
    assert int(data["adamw.step"]) == 2
    assert float(meta["adamw.lr"]) == pytest.approx(HP[0]) and meta["writer"] == "pico_amd"
    assert len(data) == 3 * len(names) + 1
    r.free()


def test_graph_replays_count_in_the_saved_step(P, tmp_path):
    # replays advance the step count on the device only; the checkpoint reads it there
    r = Run(P, CFG, 8)
    (tok, tgt), = _batches(CFG, 1, 500)
    ids = P.lib.arena_init(1 << 16)
    P.lib.arena_ctx_push(ids)
    tok, tgt = np.ascontiguousarray(tok, np.int32), np.ascontiguousarray(tgt, np.int32)
    dt = P.lib.pico_ids_to_device(tok.ctypes.data_as(ctypes.c_void_p), tok.size)
    dg = P.lib.pico_ids_to_device(tgt.ctypes.data_as(ctypes.c_void_p), tgt.size)
    P.lib.arena_ctx_pop()
    with P.arena(1 << 26) as ar:
        def step():
            P.optim_adamw_zero_grad(r.opt)
            loss = P.gpt_loss(r.model, dt, dg)
            P.backward(loss)
            P.optim_adamw_step(r.opt)
        step()
        P.reset(ar)
        assert P.lib.pico_graph_begin() == 0
        step()
        g = P.lib.pico_graph_end()
        assert g
        for _ in range(3):
            assert P.lib.pico_graph_launch(g) == 0
        P.lib.pico_graph_free(g)
    path = tmp_path / "g.safetensors"
    assert r.save(path) == 0
    assert int(load_file(str(path))["adamw.step"]) == 4
    P.lib.arena_destroy(ids)
    r.free()


def test_load_refuses_a_mismatched_model(P, tmp_path):
    path = tmp_path / "small.safetensors"
    r = Run(P, CFG, 9)
    assert r.save(path) == 0
    r.free()
    other = Run(P, dict(CFG, d_ff=192), 10)
    before = other.values()
    P.lib.pico_gpu_clear_error()
    assert other.load(path) != 0
    assert b"layers.0.w13" in P.lib.pico_gpu_last_error()
    for x, y in zip(before, other.values()):  # nothing was written
        assert np.array_equal(x, y)
    P.lib.pico_gpu_clear_error()
    assert other.load(tmp_path / "missing.safetensors") != 0
    assert b"cannot open" in P.lib.pico_gpu_last_error()
    P.lib.pico_gpu_clear_error()
    other.free()
