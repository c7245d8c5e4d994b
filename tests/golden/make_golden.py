"""Writes tests/golden/golden_ops.npz: input/output vectors for the hot-path ops
the reference does not implement (softmax cross-entropy, RMSNorm, SwiGLU,
causal attention, embedding, AdamW, argmax).

The expected outputs come from torch on the CPU in float64 (torch is an
independent library here, not the reference), using its autograd for the
backward passes and torch.optim.AdamW for the optimizer.  Inputs come from a
fixed numpy generator.  Run from the repo root:

    python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_ops.npz")


def main():
    rng = np.random.default_rng(20261201)
    g = {}

    # ---- softmax cross-entropy (mean over rows) and its gradient
    R, V = 7, 37
    z = (rng.standard_normal((R, V)) * 2.0).astype(np.float32)
    y = rng.integers(0, V, R).astype(np.int32)
    zt = torch.tensor(z, dtype=torch.float64, requires_grad=True)
    loss = torch.nn.functional.cross_entropy(zt, torch.tensor(y, dtype=torch.long))
    loss.backward()
    rows = torch.nn.functional.cross_entropy(
        torch.tensor(z, dtype=torch.float64), torch.tensor(y, dtype=torch.long), reduction="none")
    g.update(xent_z=z, xent_y=y, xent_loss=np.float64(loss.item()), xent_rows=rows.numpy(),
             xent_dz=zt.grad.numpy())

    # ---- RMSNorm y = x * rsqrt(mean(x^2) + eps) * w
    R, C, eps = 5, 24, 1e-6
    x = rng.standard_normal((R, C)).astype(np.float32)
    w = (1.0 + 0.02 * rng.standard_normal(C)).astype(np.float32)
    dy = rng.standard_normal((R, C)).astype(np.float32)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    wt = torch.tensor(w, dtype=torch.float64, requires_grad=True)
    yt = xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + eps) * wt
    yt.backward(torch.tensor(dy, dtype=torch.float64))
    g.update(rms_x=x, rms_w=w, rms_dy=dy, rms_eps=np.float64(eps), rms_y=yt.detach().numpy(),
             rms_dx=xt.grad.numpy(), rms_dw=wt.grad.numpy())

    # ---- SwiGLU h = silu(a) * u
    a = rng.standard_normal((4, 33)).astype(np.float32)
    u = rng.standard_normal((4, 33)).astype(np.float32)
    dh = rng.standard_normal((4, 33)).astype(np.float32)
    at = torch.tensor(a, dtype=torch.float64, requires_grad=True)
    ut = torch.tensor(u, dtype=torch.float64, requires_grad=True)
    ht = torch.nn.functional.silu(at) * ut
    ht.backward(torch.tensor(dh, dtype=torch.float64))
    g.update(swi_a=a, swi_u=u, swi_dh=dh, swi_h=ht.detach().numpy(), swi_da=at.grad.numpy(),
             swi_du=ut.grad.numpy())

    # ---- causal attention, token-major [B*T, H*hd]
    B, H, T, hd = 2, 3, 9, 8
    q = rng.standard_normal((B * T, H * hd)).astype(np.float32)
    k = rng.standard_normal((B * T, H * hd)).astype(np.float32)
    v = rng.standard_normal((B * T, H * hd)).astype(np.float32)
    do = rng.standard_normal((B * T, H * hd)).astype(np.float32)

    def heads(t):
        return t.reshape(B, T, H, hd).permute(0, 2, 1, 3)

    qt, kt, vt = (torch.tensor(t, dtype=torch.float64, requires_grad=True) for t in (q, k, v))
    s = heads(qt) @ heads(kt).transpose(-1, -2) / np.sqrt(hd)
    mask = torch.triu(torch.ones(T, T, dtype=torch.bool), 1)
    s = s.masked_fill(mask, float("-inf"))
    lse = torch.logsumexp(s, -1)
    o = (torch.softmax(s, -1) @ heads(vt)).permute(0, 2, 1, 3).reshape(B * T, H * hd)
    o.backward(torch.tensor(do, dtype=torch.float64))
    g.update(att_B=np.int64(B), att_H=np.int64(H), att_q=q, att_k=k, att_v=v, att_do=do,
             att_o=o.detach().numpy(), att_lse=lse.detach().numpy().reshape(-1),
             att_dq=qt.grad.numpy(), att_dk=kt.grad.numpy(), att_dv=vt.grad.numpy())

    # ---- embedding gather / scatter-add (repeated ids)
    Vv, d = 11, 6
    table = rng.standard_normal((Vv, d)).astype(np.float32)
    ids = np.array([3, 0, 3, 10, 7, 3, 0], np.int32)
    dout = rng.standard_normal((ids.size, d)).astype(np.float32)
    tt = torch.tensor(table, dtype=torch.float64, requires_grad=True)
    et = torch.nn.functional.embedding(torch.tensor(ids, dtype=torch.long), tt)
    et.backward(torch.tensor(dout, dtype=torch.float64))
    g.update(emb_table=table, emb_ids=ids, emb_dout=dout, emb_out=et.detach().numpy(),
             emb_dtable=tt.grad.numpy())

    # ---- AdamW, three steps with different gradients
    n = 19
    p0 = rng.standard_normal(n).astype(np.float32)
    grads = rng.standard_normal((3, n)).astype(np.float32)
    lr, b1, b2, eps, wd = 3e-3, 0.9, 0.95, 1e-8, 0.1
    pt = torch.tensor(p0, dtype=torch.float64, requires_grad=True)
    opt = torch.optim.AdamW([pt], lr=lr, betas=(b1, b2), eps=eps, weight_decay=wd)
    steps = []
    for s_ in range(3):
        pt.grad = torch.tensor(grads[s_], dtype=torch.float64)
        opt.step()
        steps.append(pt.detach().numpy().copy())
    g.update(adamw_p0=p0, adamw_g=grads, adamw_hparams=np.array([lr, b1, b2, eps, wd]),
             adamw_p=np.stack(steps))

    # ---- argmax: ties (first wins), NaN (first NaN wins), -0/+0, all equal
    x = rng.standard_normal((6, 13)).astype(np.float32)
    x[1, 4] = x[1, 9] = x[1].max() + 1.0
    x[2, 7] = np.nan
    x[2, 11] = np.nan
    x[3, :] = 0.0
    x[3, 5] = -0.0
    x[4, :] = 2.5
    x[5, 0] = np.inf
    g.update(argmax_x=x, argmax_idx=torch.argmax(torch.tensor(x), dim=1).numpy().astype(np.int32))

    np.savez_compressed(OUT, **g)
    print("wrote", OUT, sorted(g))


if __name__ == "__main__":
    main()
