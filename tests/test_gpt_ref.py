"""Pins the float64 transformer reference (oracle/gpt_ref.py) -- CPU only.

Its hand-written backward is checked against torch's float64 autograd of an
independently written forward (torch is a library here, not the reference),
and its forward against closed forms: with all weights zero every position
predicts uniformly, so the loss is exactly ln V and only the LM head receives
a gradient.
"""
import numpy as np
import pytest
import torch

from oracle import gpt_ref as G

CFG = dict(vocab=11, d_model=8, n_layers=2, n_heads=2, d_ff=12, batch=2, seq_len=5)


def _params(cfg, seed, std=0.3):
    rng = np.random.default_rng(seed)
    V, d, F = cfg["vocab"], cfg["d_model"], cfg["d_ff"]
    ps = [rng.normal(0, std, (V, d))]
    for _ in range(cfg["n_layers"]):
        ps += [1 + rng.normal(0, 0.1, d)] + [rng.normal(0, std, (d, d)) for _ in range(4)]
        ps += [1 + rng.normal(0, 0.1, d), rng.normal(0, std, (d, F)), rng.normal(0, std, (d, F)),
               rng.normal(0, std, (F, d))]
    ps += [1 + rng.normal(0, 0.1, d), rng.normal(0, std, (d, V))]
    return ps


def _torch_loss(params, cfg, tokens, targets, eps=1e-6):
    B, T, H = cfg["batch"], cfg["seq_len"], cfg["n_heads"]
    P = [torch.tensor(p, dtype=torch.float64, requires_grad=True) for p in params]

    def rms(x, g):
        return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * g

    x = P[0][torch.tensor(tokens)]
    for l in range(cfg["n_layers"]):
        g1, Wq, Wk, Wv, Wo, g2, W1, W3, W2 = P[1 + 9 * l: 10 + 9 * l]
        h = rms(x, g1)
        q, k, v = (t.reshape(B, T, H, -1).transpose(1, 2) for t in (h @ Wq, h @ Wk, h @ Wv))
        att = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
        x = x + att.transpose(1, 2).reshape(B * T, -1) @ Wo
        h = rms(x, g2)
        x = x + torch.nn.functional.silu(h @ W1) * (h @ W3) @ W2
    logits = rms(x, P[-2]) @ P[-1]
    loss = torch.nn.functional.cross_entropy(logits, torch.tensor(targets))
    loss.backward()
    return float(loss), [p.grad.detach().numpy() for p in P]


def test_backward_matches_torch_autograd():
    rng = np.random.default_rng(0)
    n = CFG["batch"] * CFG["seq_len"]
    tokens = rng.integers(0, CFG["vocab"], n)
    targets = rng.integers(0, CFG["vocab"], n)
    params = _params(CFG, 1)
    loss, grads = G.loss_and_grads(params, CFG, tokens, targets)
    tl, tg = _torch_loss(params, CFG, tokens, targets)
    assert abs(loss - tl) <= 1e-12 * abs(tl)
    assert len(grads) == len(tg) == 3 + 9 * CFG["n_layers"]
    for i, (g, t) in enumerate(zip(grads, tg)):
        assert g.shape == t.shape, i
        assert np.max(np.abs(g - t)) <= 1e-10 * max(np.max(np.abs(t)), 1e-30), i


def test_zero_weights_give_uniform_prediction():
    params = [np.zeros_like(p) for p in _params(CFG, 2)]
    for i in range(1, len(params), 9):  # gains stay 1 (only matters for shapes here)
        params[i] = np.ones_like(params[i])
    n = CFG["batch"] * CFG["seq_len"]
    targets = np.arange(n) % CFG["vocab"]
    loss, grads = G.loss_and_grads(params, CFG, np.zeros(n, int), targets)
    assert loss == pytest.approx(np.log(CFG["vocab"]), rel=1e-15)
    assert all(not np.any(g) for g in grads[:-1])


def test_fused_parameter_mapping_round_trips():
    # gpt.c's fused wqkv = [Wq|Wk|Wv], w13 = [W1|W3] against separate weights
    cfg = dict(vocab=7, d_model=4, n_layers=2, n_heads=2, d_ff=6)
    sep = _params(cfg, 5)
    fused = G.join_fused(sep, cfg)
    assert len(fused) == 3 + G.FUSED_PER_LAYER * cfg["n_layers"]
    assert fused[2].shape == (4, 12) and fused[5].shape == (4, 12)
    assert np.array_equal(fused[2][:, 4:8], sep[3]) and np.array_equal(fused[5][:, 6:], sep[8])
    back = G.split_fused([f.ravel() for f in fused], cfg)
    assert all(np.array_equal(a.reshape(b.shape), b) for a, b in zip(back, sep))


def test_by_sequence_split_equals_the_whole_batch():
    """loss_and_grads_by_sequence (one sequence per thread, shares summed) is
    the same function as loss_and_grads over the whole batch"""
    cfg = dict(CFG, batch=3, seq_len=6)
    params = _params(cfg, 5)
    rng = np.random.default_rng(6)
    tokens = rng.integers(0, cfg["vocab"], cfg["batch"] * cfg["seq_len"])
    targets = rng.integers(0, cfg["vocab"], cfg["batch"] * cfg["seq_len"])
    l0, g0 = G.loss_and_grads(params, cfg, tokens, targets)
    l1, g1 = G.loss_and_grads_by_sequence(params, cfg, tokens, targets, workers=3)
    assert abs(l0 - l1) <= 1e-12 * abs(l0)
    for a, b in zip(g0, g1):
        assert np.max(np.abs(a - b)) <= 1e-12 * max(1.0, float(np.max(np.abs(a))))
