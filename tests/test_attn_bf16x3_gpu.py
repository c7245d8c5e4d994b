"""Fused attention with fp32 products from three bf16 ones
(pk_flash_attn_{fwd,bwd}_bf16x3_f32): every product operand split into hi =
bf16(x) and lo = bf16(x - hi), each product taken as hi.hi + hi.lo + lo.hi.
That keeps the fp32 parity bound, so it is held to the fp32 kernels' test:

* forward and backward within 1e-4 (relative to the largest value) of the
  fp32 oracle at padded and unpadded T, and far closer to it than the plain
  bf16 products (which sit near 1e-2);
* the accumulate bits add onto the outputs bit for bit;
* causality holds bit for bit.
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


@pytest.mark.parametrize("B,H,T", [(2, 2, 128), (1, 3, 256), (1, 2, 1024), (2, 2, 100),
                                   (1, 2, 999), (2, 2, 1)])
def test_bf16x3_attention_vs_fp32_oracle(dev, B, H, T):
    D = H * 64
    q, k, v, do = (O.normal(B * T * D, s).reshape(B * T, D) for s in (81, 82, 83, 84))
    o = torch.empty(B * T, D, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o, lse, bf16x3=True)
    o_ref, lse_ref = O.attn_fwd(B, H, q, k, v)
    assert max_rel(host(o), o_ref) <= TOL and max_rel(host(lse), lse_ref) <= TOL
    if T > 1:  # the plain bf16 products are visibly further away
        ob = torch.empty(B * T, D, device=dev)
        K.flash_fwd(B, H, cu(q), cu(k), cu(v), ob, lse, bf16=True)
        assert max_rel(host(ob), o_ref) > 10 * max_rel(host(o), o_ref)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o, lse, bf16x3=True)
    dq, dk, dv = (torch.full((B * T, D), float("nan"), device=dev) for _ in range(3))
    K.flash_bwd(B, H, cu(q), cu(k), cu(v), cu(o_ref), cu(lse_ref), cu(do), dq, dk, dv,
                bf16x3=True)
    refs = O.attn_bwd(B, H, q, k, v, o_ref, lse_ref, do)

    def close(got, ref):
        if not np.any(ref):  # T = 1: dq and dk are 0 up to rounding of dO's scale
            return np.max(np.abs(got)) <= TOL * np.max(np.abs(do))
        return max_rel(got, ref) <= TOL
    for got, ref in zip((dq, dk, dv), refs):
        assert close(host(got), ref)
    base = [O.normal(B * T * D, 90 + i).reshape(B * T, D) for i in range(3)]
    acc = [cu(x.copy()) for x in base]
    K.flash_bwd(B, H, cu(q), cu(k), cu(v), cu(o_ref), cu(lse_ref), cu(do), *acc, flags=7,
                bf16x3=True)
    for got, plain, b0 in zip(acc, (dq, dk, dv), base):
        assert np.array_equal(host(got), (b0 + host(plain)).astype(np.float32))


def test_bf16x3_attention_causality(dev):
    B, H, T, D = 2, 2, 256, 128
    q, k, v = (O.normal(B * T * D, s).reshape(B * T, D) for s in (91, 92, 93))
    o1, o2 = torch.empty(B * T, D, device=dev), torch.empty(B * T, D, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o1, lse, bf16x3=True)
    k2, v2 = k.copy(), v.copy()
    for b in range(B):
        k2[b * T + T - 1] += 1.0
        v2[b * T + T - 1] -= 1.0
    K.flash_fwd(B, H, cu(q), cu(k2), cu(v2), o2, lse, bf16x3=True)
    a, c = host(o1).reshape(B, T, D), host(o2).reshape(B, T, D)
    assert np.array_equal(a[:, :-1], c[:, :-1]) and not np.array_equal(a[:, -1], c[:, -1])
