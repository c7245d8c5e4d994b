"""float64 numpy reference of the benchmark transformer -- TEST INFRASTRUCTURE.

Only tests/ (as the checker) use this module.  It restates, from the
mathematics, the model that pico_amd/host/gpt.c builds from pico ops: a
pre-norm decoder-only transformer without biases (RMSNorm, causal multi-head
attention, SwiGLU FFN, untied embedding and LM head, mean next-token
cross-entropy), with its backward pass written out by hand so that it shares
nothing with pico's autograd walk.  There is no reference implementation to
follow (pico has no sequence model); the hand-written backward is pinned
against torch's float64 autograd in tests/test_gpt_ref.py ("parity pinned by
an independent autodiff", not by the reference).

Parameters are passed as separate weights: E [V,d]; per layer g_attn [d],
Wq, Wk, Wv, Wo [d,d], g_ffn [d], W1 [d,F], W3 [d,F], W2 [F,d]; g_final [d];
Wlm [d,V].  gpt.c stores the projections that read one input side by side --
wqkv = [Wq | Wk | Wv] [d,3d] and w13 = [W1 | W3] [d,2F], six params per layer
-- and split_fused / join_fused map between the two lists.
"""
from __future__ import annotations

import os

import numpy as np

PER_LAYER = 9
FUSED_PER_LAYER = 6


def split_fused(params, cfg):
    """gpt.c's parameter list (per layer g_attn, wqkv, wo, g_ffn, w13, w2; flat
    or shaped arrays) as this module's list of separate, shaped weights"""
    d, F, V, L = cfg["d_model"], cfg["d_ff"], cfg["vocab"], cfg["n_layers"]
    p = [np.asarray(x) for x in params]
    assert len(p) == 3 + FUSED_PER_LAYER * L
    out = [p[0].reshape(V, d)]
    for l in range(L):
        g1, wqkv, wo, g2, w13, w2 = p[1 + FUSED_PER_LAYER * l: 1 + FUSED_PER_LAYER * (l + 1)]
        wqkv, w13 = wqkv.reshape(d, 3 * d), w13.reshape(d, 2 * F)
        out += [g1.reshape(d), wqkv[:, :d], wqkv[:, d:2 * d], wqkv[:, 2 * d:], wo.reshape(d, d),
                g2.reshape(d), w13[:, :F], w13[:, F:], w2.reshape(F, d)]
    return out + [p[-2].reshape(d), p[-1].reshape(d, V)]


def join_fused(params, cfg):
    """the inverse of split_fused: separate weights into gpt.c's shaped list"""
    d, F, L = cfg["d_model"], cfg["d_ff"], cfg["n_layers"]
    p = [np.asarray(x) for x in params]
    out = [p[0]]
    for l in range(L):
        g1, Wq, Wk, Wv, Wo, g2, W1, W3, W2 = p[1 + PER_LAYER * l: 1 + PER_LAYER * (l + 1)]
        out += [g1, np.concatenate([Wq.reshape(d, d), Wk.reshape(d, d), Wv.reshape(d, d)], 1),
                Wo, g2, np.concatenate([W1.reshape(d, F), W3.reshape(d, F)], 1), W2]
    return out + p[-2:]


def _rms_fwd(x, g, eps):
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * r * g, r


def _rms_bwd(x, g, r, dy):
    C = x.shape[-1]
    dot = np.sum(g * dy * x, axis=-1, keepdims=True)
    dx = r * (g * dy) - x * (r ** 3) * dot / C
    dg = np.sum(dy * x * r, axis=0)
    return dx, dg


def _heads(t, B, T, H):
    return t.reshape(B, T, H, -1).transpose(0, 2, 1, 3)  # [B,H,T,hd]


def _merge(t):
    B, H, T, hd = t.shape
    return t.transpose(0, 2, 1, 3).reshape(B * T, H * hd)


def _attn_fwd(q, k, v, B, T, H):
    Q, K, Vv = _heads(q, B, T, H), _heads(k, B, T, H), _heads(v, B, T, H)
    scale = 1.0 / np.sqrt(Q.shape[-1])
    S = (Q @ K.transpose(0, 1, 3, 2)) * scale
    mask = np.triu(np.ones((T, T), bool), 1)
    S = np.where(mask, -np.inf, S)
    S = S - S.max(-1, keepdims=True)
    P = np.exp(S)
    P /= P.sum(-1, keepdims=True)
    return _merge(P @ Vv), (Q, K, Vv, P, scale)


def _attn_bwd(cache, dout, B, T, H):
    Q, K, Vv, P, scale = cache
    dO = _heads(dout, B, T, H)
    dV = P.transpose(0, 1, 3, 2) @ dO
    dP = dO @ Vv.transpose(0, 1, 3, 2)
    dS = P * (dP - np.sum(dP * P, -1, keepdims=True))
    dQ = (dS @ K) * scale
    dK = (dS.transpose(0, 1, 3, 2) @ Q) * scale
    return _merge(dQ), _merge(dK), _merge(dV)


def loss_and_grads(params, cfg, tokens, targets, eps=1e-6, need_grads=True, n_norm=None):
    """mean cross-entropy (float) and, if asked, one float64 gradient per param.
    n_norm (default: the number of positions) is the denominator of the mean,
    so a share of a batch can be run alone and the shares summed."""
    P = [np.asarray(p, np.float64) for p in params]
    B, T, H, L = cfg["batch"], cfg["seq_len"], cfg["n_heads"], cfg["n_layers"]
    tokens = np.asarray(tokens, np.int64).ravel()
    targets = np.asarray(targets, np.int64).ravel()
    n = tokens.size
    n_norm = n if n_norm is None else n_norm
    E = P[0]
    x = E[tokens]
    caches = []
    for l in range(L):
        g1, Wq, Wk, Wv, Wo, g2, W1, W3, W2 = P[1 + PER_LAYER * l: 1 + PER_LAYER * (l + 1)]
        h, r1 = _rms_fwd(x, g1, eps)
        q, k, v = h @ Wq, h @ Wk, h @ Wv
        a, ac = _attn_fwd(q, k, v, B, T, H)
        x1 = x + a @ Wo
        h2, r2 = _rms_fwd(x1, g2, eps)
        gate, up = h2 @ W1, h2 @ W3
        s = 1.0 / (1.0 + np.exp(-gate))
        act = gate * s * up
        caches.append((x, h, r1, a, ac, x1, h2, r2, gate, up, s, act))
        x = x1 + act @ W2
    gf, Wlm = P[-2], P[-1]
    hf, rf = _rms_fwd(x, gf, eps)
    logits = hf @ Wlm
    m = logits.max(-1, keepdims=True)
    lse = m[:, 0] + np.log(np.exp(logits - m).sum(-1))
    loss = float(np.sum(lse - logits[np.arange(n), targets]) / n_norm)
    if not need_grads:
        return loss, None
    grads = [None] * len(P)
    dlogits = np.exp(logits - lse[:, None])
    dlogits[np.arange(n), targets] -= 1.0
    dlogits /= n_norm
    grads[-1] = hf.T @ dlogits
    dx, grads[-2] = _rms_bwd(x, gf, rf, dlogits @ Wlm.T)
    for l in reversed(range(L)):
        base = 1 + PER_LAYER * l
        g1, Wq, Wk, Wv, Wo, g2, W1, W3, W2 = P[base: base + PER_LAYER]
        x0, h, r1, a, ac, x1, h2, r2, gate, up, s, act = caches[l]
        grads[base + 8] = act.T @ dx
        dact = dx @ W2.T
        dgate = dact * up * s * (1.0 + gate * (1.0 - s))
        dup = dact * gate * s
        grads[base + 6] = h2.T @ dgate
        grads[base + 7] = h2.T @ dup
        dh2 = dgate @ W1.T + dup @ W3.T
        dxr, grads[base + 5] = _rms_bwd(x1, g2, r2, dh2)
        dx1 = dx + dxr
        grads[base + 4] = a.T @ dx1
        dq, dk, dv = _attn_bwd(ac, dx1 @ Wo.T, B, T, H)
        grads[base + 1] = h.T @ dq
        grads[base + 2] = h.T @ dk
        grads[base + 3] = h.T @ dv
        dh = dq @ Wq.T + dk @ Wk.T + dv @ Wv.T
        dxr, grads[base] = _rms_bwd(x0, g1, r1, dh)
        dx = dx1 + dxr
    dE = np.zeros_like(E)
    np.add.at(dE, tokens, dx)
    grads[0] = dE
    return loss, grads


def loss_and_grads_by_sequence(params, cfg, tokens, targets, eps=1e-6, workers=8):
    """loss_and_grads over the batch, one sequence at a time in a thread pool.

    Sequences are independent up to the mean over positions and the sums that
    form the parameter gradients, so each sequence runs alone with the whole
    batch's denominator and the results are added (float64: the changed
    summation order is far below the tests' tolerance).  numpy's BLAS calls
    and large ufuncs release the GIL, so the threads run in parallel; this is
    what makes the 12-layer, 8 x 1024-token configuration's reference
    affordable."""
    from concurrent.futures import ThreadPoolExecutor

    B, T = cfg["batch"], cfg["seq_len"]
    tokens = np.asarray(tokens, np.int64).reshape(B, T)
    targets = np.asarray(targets, np.int64).reshape(B, T)
    one = dict(cfg, batch=1)
    P = [np.asarray(p, np.float64) for p in params]

    def run(b):
        return loss_and_grads(P, one, tokens[b], targets[b], eps=eps, n_norm=B * T)

    try:
        from threadpoolctl import threadpool_limits
    except ImportError:  # pragma: no cover
        threadpool_limits = None
    inner = max(1, (os.cpu_count() or 8) // max(1, min(workers, B)))
    ctx = threadpool_limits(limits=inner) if threadpool_limits else _nullctx()
    with ctx, ThreadPoolExecutor(max_workers=min(workers, B)) as ex:
        parts = list(ex.map(run, range(B)))
    loss = float(sum(p[0] for p in parts))
    grads = [sum(p[1][i] for p in parts) for i in range(len(P))]
    return loss, grads


class _nullctx:
    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False


def adamw(p, g, m, v, step, lr, b1, b2, eps, wd):
    """decoupled-decay AdamW, the update pk_adamw_f32 applies (float64 here)"""
    p = p * (1.0 - lr * wd)
    m = b1 * m + (1.0 - b1) * g
    v = b2 * v + (1.0 - b2) * g * g
    bc1 = 1.0 - b1 ** step
    bc2 = 1.0 - b2 ** step
    p = p - (lr / bc1) * m / (np.sqrt(v) / np.sqrt(bc2) + eps)
    return p, m, v
