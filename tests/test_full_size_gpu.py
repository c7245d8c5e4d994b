"""The row kernels and the fused attention at the benchmark's full sizes.

Every output row of RMSNorm, SwiGLU and softmax-CE depends only on its own
input row, and every attention head only on its own columns, so the kernels
run over the whole config-3 / config-5 tensors (the launch shapes, grids and
loops the benchmark times) and a seeded sample of rows or heads is compared
with the CPU oracle.  Quantities that cover every row are checked whole:
RMSNorm's gain gradient (a sum over all 8192 rows, against a float64 sum)
and softmax-CE's loss rows.
Bar: max relative error <= 1e-4, as everywhere else.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import kernels as K
from tests._util import max_rel

pytestmark = pytest.mark.gpu
TOL = 1e-4


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _rows(R, n, seed):
    """n distinct rows, always including the first and the last"""
    rng = np.random.default_rng(seed)
    pick = rng.choice(np.arange(1, R - 1), size=n - 2, replace=False)
    return np.sort(np.concatenate([[0, R - 1], pick]))


def test_rmsnorm_config3_full(dev):
    R, C = 8192, 4096
    x = O.normal(R * C, 101).reshape(R, C)
    g = O.normal(C, 102, 1.0, 0.02)
    dy = O.normal(R * C, 103).reshape(R, C)
    y, rstd = torch.empty(R, C, device=dev), torch.empty(R, device=dev)
    K.rmsnorm_fwd(cu(x), cu(g), y, rstd, 1e-6)
    dx, dg = torch.empty(R, C, device=dev), torch.empty(C, device=dev)
    K.rmsnorm_bwd(cu(x), cu(g), rstd, cu(dy), dx, dg)
    rows = _rows(R, 64, 104)
    y_ref, rstd_ref = O.rmsnorm_fwd(x[rows], g, 1e-6)
    assert max_rel(host(y)[rows], y_ref) <= TOL
    assert max_rel(host(rstd)[rows], rstd_ref) <= TOL
    dx_ref, _ = O.rmsnorm_bwd(x[rows], g, rstd_ref, dy[rows])
    assert max_rel(host(dx)[rows], dx_ref) <= TOL
    # the gain gradient sums every row: against a float64 sum over all of them
    r64 = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=1) + 1e-6)
    dg_ref = np.einsum("rc,rc,r->c", dy.astype(np.float64), x.astype(np.float64), r64)
    assert max_rel(host(dg), dg_ref) <= TOL


def test_swiglu_config3_full(dev):
    R, F = 8192, 11008
    a = O.normal(R * F, 111).reshape(R, F)
    u = O.normal(R * F, 112).reshape(R, F)
    dh = O.normal(R * F, 113).reshape(R, F)
    h = torch.empty(R, F, device=dev)
    K.swiglu_fwd(cu(a), cu(u), h)
    da, du = torch.empty(R, F, device=dev), torch.empty(R, F, device=dev)
    K.swiglu_bwd(cu(a), cu(u), cu(dh), da, du)
    rows = _rows(R, 48, 114)
    assert max_rel(host(h)[rows], O.swiglu_fwd(a[rows], u[rows])) <= TOL
    da_ref, du_ref = O.swiglu_bwd(a[rows], u[rows], dh[rows])
    assert max_rel(host(da)[rows], da_ref) <= TOL
    assert max_rel(host(du)[rows], du_ref) <= TOL


def test_xent_config3_full(dev):
    R, V = 8192, 32000
    z = O.normal(R * V, 121, 0.0, 2.0).reshape(R, V)
    y = O.labels(R, 122, V)
    loss = torch.empty(R, device=dev)
    dz = torch.empty(R, V, device=dev)
    K.xent_fwd_bwd(cu(z), cu(y), loss, dz, scale=1.0 / R)
    # every row's loss, and the gradient of a sample of rows
    loss_ref, _ = O.xent(z, y, scale=1.0 / R, want_grad=False)
    got = host(loss)
    assert max_rel(got, loss_ref) <= TOL
    mean_ref = float(np.mean(loss_ref.astype(np.float64)))
    assert abs(float(np.mean(got.astype(np.float64))) - mean_ref) <= TOL * abs(mean_ref)
    rows = _rows(R, 48, 123)
    _, dz_ref = O.xent(z[rows], y[rows], scale=1.0 / R)
    assert max_rel(host(dz)[rows], dz_ref) <= TOL


def test_flash_attention_config5_full(dev):
    # B 8, T 1024, 12 heads of 64: all 96 heads run; 6 are compared
    B, H, T, hd = 8, 12, 1024, 64
    D = H * hd
    q, k, v, do = (O.normal(B * T * D, 131 + i).reshape(B * T, D) for i in range(4))
    o, lse = torch.empty(B * T, D, device=dev), torch.empty(B * H * T, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o, lse)
    dq, dk, dv = (torch.empty(B * T, D, device=dev) for _ in range(3))
    K.flash_bwd(B, H, cu(q), cu(k), cu(v), o, lse, cu(do), dq, dk, dv)
    o, lse, dq, dk, dv = (host(t) for t in (o, lse, dq, dk, dv))
    for b, h in ((0, 0), (7, 11), (3, 5), (5, 0), (0, 11), (6, 7)):
        rows, cols = slice(b * T, (b + 1) * T), slice(h * hd, (h + 1) * hd)
        qh, kh, vh, doh = (np.ascontiguousarray(t[rows, cols]) for t in (q, k, v, do))
        o_ref, lse_ref = O.attn_fwd(1, 1, qh, kh, vh)
        assert max_rel(o[rows, cols], o_ref) <= TOL, (b, h)
        head_lse = lse[(b * H + h) * T:(b * H + h + 1) * T]
        assert max_rel(head_lse, lse_ref) <= TOL, (b, h)
        refs = O.attn_bwd(1, 1, qh, kh, vh, o_ref, lse_ref, doh)
        for got, ref in zip((dq, dk, dv), refs):
            assert max_rel(got[rows, cols], ref) <= TOL, (b, h)
