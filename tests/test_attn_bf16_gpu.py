"""bf16 fused attention (pk_flash_attn_{fwd,bwd}_bf16_f32): outside the fp32
parity contract, so pinned against what the arithmetic fixes.

* Forward: a host restatement of the kernel's arithmetic -- Q*scale*log2(e),
  K and V rounded to bf16 (nearest even), scores in float64, a running max per
  64-key block, the block's probabilities rounded to bf16 for the product with
  V and summed unrounded for the normaliser.  What is left between the two is
  fp32 summation order and the last bit of exp2, so the tolerance is 1e-3 of
  max |O| (a permuted key/value pairing inside the products would be off by
  the size of O itself).
* Forward and backward against the fp32 oracle: within bf16 rounding
  (3e-2 of the largest value), and clearly further from it than the fp32
  kernels are -- the products really are bf16.
* Causality holds bit for bit; accumulate bits behave as in fp32.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import kernels as K
from tests._util import max_rel

pytestmark = pytest.mark.gpu
LOG2E = 1.4426950408889634
BF16_TOL = 3e-2


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bf16_round(x):
    """fp32 -> bf16 -> fp32, round to nearest even (finite inputs)"""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def fwd_bf16_restated(B, H, q, k, v):
    """The bf16 forward's arithmetic, 64-query block by 64-key block."""
    BT, D = q.shape
    T, hd = BT // B, 64
    mul = np.float32(hd ** -0.5 * LOG2E)
    out = np.empty((BT, D), np.float64)
    lse = np.empty(B * H * T, np.float64)
    for b in range(B):
        for h in range(H):
            rows, cols = slice(b * T, (b + 1) * T), slice(h * hd, (h + 1) * hd)
            Q = bf16_round(q[rows, cols] * mul).astype(np.float64)
            Kh = bf16_round(k[rows, cols]).astype(np.float64)
            Vh = bf16_round(v[rows, cols]).astype(np.float64)
            for qb in range(T // 64):
                qs = slice(64 * qb, 64 * qb + 64)
                qi = np.arange(64 * qb, 64 * qb + 64)
                m = np.full(64, -np.inf)
                lsum = np.zeros(64)
                acc = np.zeros((64, hd))
                for kb in range(qb + 1):
                    ks = slice(64 * kb, 64 * kb + 64)
                    s = Q[qs] @ Kh[ks].T
                    s[np.arange(64 * kb, 64 * kb + 64)[None, :] > qi[:, None]] = -np.inf
                    mn = np.maximum(m, s.max(axis=1))
                    alpha = np.exp2(m - mn)
                    pr = np.exp2(s - mn[:, None]).astype(np.float32)
                    lsum = lsum * alpha + pr.sum(axis=1, dtype=np.float64)
                    acc = acc * alpha[:, None] + bf16_round(pr).astype(np.float64) @ Vh[ks]
                    m = mn
                out[b * T + qi, cols] = acc / lsum[:, None]
                lse[(b * H + h) * T + qi] = (m + np.log2(lsum)) / LOG2E
    return out, lse


def _inputs(B, H, T, seed):
    D = H * 64
    return [O.normal(B * T * D, seed + i).reshape(B * T, D) for i in range(4)]


@pytest.mark.parametrize("B,H,T", [(1, 2, 128), (2, 1, 256), (1, 2, 384)])
def test_bf16_attention_forward_matches_restatement(dev, B, H, T):
    q, k, v, _ = _inputs(B, H, T, 40)
    o = torch.empty(B * T, H * 64, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o, lse, bf16=True)
    o_ref, lse_ref = fwd_bf16_restated(B, H, q, k, v)
    assert max_rel(host(o), o_ref) <= 1e-3
    assert np.max(np.abs(host(lse) - lse_ref)) <= 1e-4 * np.max(np.abs(lse_ref))


@pytest.mark.parametrize("B,H,T", [(2, 2, 128), (1, 3, 256), (1, 2, 1024), (2, 2, 100),
                                   (1, 2, 999)])
def test_bf16_attention_vs_fp32_oracle(dev, B, H, T):
    D = H * 64
    q, k, v, do = _inputs(B, H, T, 50)
    o = torch.empty(B * T, D, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o, lse, bf16=True)
    o_ref, lse_ref = O.attn_fwd(B, H, q, k, v)
    err_o = max_rel(host(o), o_ref)
    assert 1e-4 < err_o <= BF16_TOL
    assert max_rel(host(lse), lse_ref) <= BF16_TOL
    dq, dk, dv = (torch.full((B * T, D), float("nan"), device=dev) for _ in range(3))
    K.flash_bwd(B, H, cu(q), cu(k), cu(v), cu(o_ref), cu(lse_ref), cu(do), dq, dk, dv,
                bf16=True)
    refs = O.attn_bwd(B, H, q, k, v, o_ref, lse_ref, do)
    for got, ref in zip((dq, dk, dv), refs):
        err = max_rel(host(got), ref)
        assert 1e-4 < err <= BF16_TOL, err
    # accumulate bits: each output adds onto what it holds, bit for bit
    base = [O.normal(B * T * D, 60 + i).reshape(B * T, D) for i in range(3)]
    acc = [cu(x.copy()) for x in base]
    K.flash_bwd(B, H, cu(q), cu(k), cu(v), cu(o_ref), cu(lse_ref), cu(do), *acc, flags=7,
                bf16=True)
    for got, plain, b0 in zip(acc, (dq, dk, dv), base):
        assert np.array_equal(host(got), (b0 + host(plain)).astype(np.float32))


def test_bf16_attention_causality(dev):
    B, H, T, D = 2, 2, 256, 128
    q, k, v, _ = _inputs(B, H, T, 70)
    o1, o2 = torch.empty(B * T, D, device=dev), torch.empty(B * T, D, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o1, lse, bf16=True)
    k2, v2 = k.copy(), v.copy()
    for b in range(B):
        k2[b * T + T - 1] += 1.0
        v2[b * T + T - 1] -= 1.0
    K.flash_fwd(B, H, cu(q), cu(k2), cu(v2), o2, lse, bf16=True)
    a, c = host(o1).reshape(B, T, D), host(o2).reshape(B, T, D)
    assert np.array_equal(a[:, :-1], c[:, :-1]) and not np.array_equal(a[:, -1], c[:, -1])
