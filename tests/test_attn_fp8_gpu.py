"""fp8 fused attention (pk_flash_attn_{fwd,bwd}_fp8_f32): outside the fp32
parity contract, pinned against what the arithmetic fixes, as the bf16
attention is (tests/test_attn_bf16_gpu.py).

* Scales: amax[] holds max|q|, max|k|, max|v| after the forward and max|dO|
  after the backward -- checked against numpy.
* Forward: a host restatement of the kernel's arithmetic -- per-tensor powers
  of two e (the smallest putting the tensor's largest value, times
  scale*log2(e) for Q, within e4m3's 448; pinned here by that defining
  property, not by the kernel's formula), Q*scale*log2(e), K, V rounded to
  e4m3 after dividing by 2^e, scores in float64, a running max per 64-key
  block, the block's probabilities rounded as e4m3(256 P) / 256 for the
  product with V and summed unrounded for the normaliser.  What is left is
  fp32 summation order and the last bit of exp2, which can move an e4m3
  rounding of P by one step: the median error must stay at fp32 level, fewer
  than 1 % of the values may be off by more than 1e-4 of max |O|, and none
  by more than 2e-2 of it.  A permuted key/value pairing would be off by the
  size of O itself nearly everywhere.
* Forward and backward against the fp32 oracle: within fp8 rounding (e4m3
  keeps 4 significant bits to bf16's 8: rms errors of 4-8 %, about 16 times
  the bf16 kernels', cosine above 0.995, largest error within a quarter of
  the largest value), and not flushed: the gradients stay that close with
  gradient-sized dO (1e-4), whose dS lies far below e4m3's smallest
  subnormal unless scaled.
* Causality holds bit for bit; accumulate bits behave as in fp32.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import kernels as K
from tests._util import max_rel
from tests.test_attn_bf16_gpu import BF16_TOL
from tests.test_fp8_gpu import e4m3_round

pytestmark = pytest.mark.gpu
LOG2E = 1.4426950408889634
FP8_TOL = 0.25  # max |error| / max |reference|
FP8_RMS = 0.10  # rms error / rms reference (e4m3 operands: measured 0.04-0.08)


def rms_rel(x, ref):
    x, ref = np.asarray(x, np.float64), np.asarray(ref, np.float64)
    return float(np.sqrt(np.mean((x - ref) ** 2) / np.mean(ref ** 2)))


def cosine(x, ref):
    x, ref = np.asarray(x, np.float64).ravel(), np.asarray(ref, np.float64).ravel()
    return float(x @ ref / (np.linalg.norm(x) * np.linalg.norm(ref)))


def cu(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def pow2_exp(amax):
    """the smallest integer e with amax * 2^-e <= 448 (0 for amax 0)"""
    if amax == 0:
        return 0
    e = int(np.floor(np.log2(amax))) - 10
    while amax * 2.0 ** -e > 448.0:
        e += 1
    assert amax * 2.0 ** -(e - 1) > 448.0
    return e


def fp8_in(x, e):
    """x as the kernels' e4m3 operand: e4m3(x * 2^-e) * 2^e, float64"""
    return e4m3_round(np.asarray(x, np.float32) * np.float32(2.0 ** -e)).astype(np.float64) * 2.0 ** e


def fwd_fp8_restated(B, H, q, k, v):
    BT, D = q.shape
    T, hd = BT // B, 64
    mul = np.float32(hd ** -0.5 * LOG2E)
    eq = pow2_exp(float(np.max(np.abs(q))) * float(mul))
    ek = pow2_exp(float(np.max(np.abs(k))))
    ev = pow2_exp(float(np.max(np.abs(v))))
    out = np.empty((BT, D), np.float64)
    for b in range(B):
        for h in range(H):
            rows, cols = slice(b * T, (b + 1) * T), slice(h * hd, (h + 1) * hd)
            Q = fp8_in(q[rows, cols] * mul, eq)
            Kh = fp8_in(k[rows, cols], ek)
            Vh = fp8_in(v[rows, cols], ev)
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
                    p8 = e4m3_round(pr * np.float32(256.0)).astype(np.float64) / 256.0
                    acc = acc * alpha[:, None] + p8 @ Vh[ks]
                    m = mn
                out[b * T + qi, cols] = acc / lsum[:, None]
    return out


def _inputs(B, H, T, seed):
    D = H * 64
    return [O.normal(B * T * D, seed + i).reshape(B * T, D) for i in range(4)]


@pytest.mark.parametrize("B,H,T", [(1, 2, 128), (2, 1, 256), (1, 2, 384)])
def test_fp8_attention_forward_matches_restatement(dev, B, H, T):
    q, k, v, _ = _inputs(B, H, T, 140)
    k = k * 3.0  # the three tensors take different powers of two
    v = v * 0.01
    o = torch.empty(B * T, H * 64, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    amax = torch.full((4,), -1.0, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o, lse, fp8_amax=amax)
    got_amax = host(amax)
    want = [np.max(np.abs(x)) for x in (q, k, v)]
    assert np.array_equal(got_amax[:3], np.array(want, np.float32))
    o_ref = fwd_fp8_restated(B, H, q, k, v)
    got = host(o)
    scale = np.max(np.abs(o_ref))
    # nearly every value to fp32 precision; a few rows where a score's last
    # bit moved one e4m3 rounding of P (rows with few keys feel it most)
    assert np.median(np.abs(got - o_ref)) <= 1e-5 * scale
    assert np.mean(np.abs(got - o_ref) > 1e-4 * scale) < 0.01
    assert max_rel(got, o_ref) <= 2e-2


@pytest.mark.parametrize("B,H,T", [(2, 2, 128), (1, 3, 256), (1, 2, 1024), (2, 2, 100),
                                   (1, 2, 999)])
def test_fp8_attention_vs_fp32_oracle(dev, B, H, T):
    D = H * 64
    q, k, v, do = _inputs(B, H, T, 150)
    do = do * 1e-4  # gradient-sized: dS far below e4m3's smallest subnormal unscaled
    o = torch.empty(B * T, D, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    amax = torch.zeros(4, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o, lse, fp8_amax=amax)
    o_ref, lse_ref = O.attn_fwd(B, H, q, k, v)
    lse16 = torch.empty(B * H * T, device=dev)
    o16 = torch.empty(B * T, D, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o16, lse16, bf16=True)
    assert max_rel(host(o), o_ref) <= FP8_TOL
    assert max_rel(host(lse), lse_ref) <= 3e-2
    # e4m3 keeps 4 significant bits to bf16's 8: the error is about 16 times
    # bf16's (so the products really are fp8), the direction is kept
    err_o = rms_rel(host(o), o_ref)
    assert 5 * rms_rel(host(o16), o_ref) < err_o <= FP8_RMS
    assert cosine(host(o), o_ref) > 0.995
    dq, dk, dv = (torch.full((B * T, D), float("nan"), device=dev) for _ in range(3))
    K.flash_bwd(B, H, cu(q), cu(k), cu(v), cu(o_ref), cu(lse_ref), cu(do), dq, dk, dv,
                fp8_amax=amax)
    assert host(amax)[3] == np.float32(np.max(np.abs(do)))
    refs = O.attn_bwd(B, H, q, k, v, o_ref, lse_ref, do)
    for got, ref in zip((dq, dk, dv), refs):
        g = host(got)
        assert max_rel(g, ref) <= FP8_TOL
        # gradient-sized dO (1e-4): dS is scaled per block, not flushed
        assert BF16_TOL / 10 < rms_rel(g, ref) <= FP8_RMS
        assert cosine(g, ref) > 0.995
    # accumulate bits: each output adds onto what it holds, bit for bit
    base = [O.normal(B * T * D, 160 + i).reshape(B * T, D) * 1e-4 for i in range(3)]
    acc = [cu(x.copy()) for x in base]
    K.flash_bwd(B, H, cu(q), cu(k), cu(v), cu(o_ref), cu(lse_ref), cu(do), *acc, flags=7,
                fp8_amax=amax)
    for got, plain, b0 in zip(acc, (dq, dk, dv), base):
        assert np.array_equal(host(got), (b0 + host(plain)).astype(np.float32))


def test_fp8_attention_causality(dev):
    B, H, T, D = 2, 2, 256, 128
    q, k, v, _ = _inputs(B, H, T, 170)
    o1, o2 = torch.empty(B * T, D, device=dev), torch.empty(B * T, D, device=dev)
    lse = torch.empty(B * H * T, device=dev)
    amax = torch.zeros(4, device=dev)
    K.flash_fwd(B, H, cu(q), cu(k), cu(v), o1, lse, fp8_amax=amax)
    # a change to the last key and value that leaves the tensors' largest
    # magnitudes (and so their powers of two) where they were
    k2, v2 = k.copy(), v.copy()
    for b in range(B):
        k2[b * T + T - 1] *= 0.5
        v2[b * T + T - 1] *= -0.5
    K.flash_fwd(B, H, cu(q), cu(k2), cu(v2), o2, lse, fp8_amax=amax)
    a, c = host(o1).reshape(B, T, D), host(o2).reshape(B, T, D)
    assert np.array_equal(a[:, :-1], c[:, :-1]) and not np.array_equal(a[:, -1], c[:, -1])


def test_fp8_attention_refusals(dev):
    from pico_amd import _lib

    L = _lib.hip_lib()
    x = torch.zeros(128, 64, device=dev)
    lse = torch.zeros(128, device=dev)
    assert L.pk_flash_attn_fwd_fp8_f32(1, 1, 128, 64, 64, 0.125, x.data_ptr(), x.data_ptr(),
                                       x.data_ptr(), x.data_ptr(), lse.data_ptr(), None,
                                       None) != 0
    assert b"amax" in L.pk_last_error()
