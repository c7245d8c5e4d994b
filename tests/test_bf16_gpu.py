"""bf16 matrix products (pk_gemm_bf16_f32, pico_set_matmul_precision): outside
the fp32 parity contract, so pinned against what the arithmetic fixes.

* Operands rounded to bf16 (nearest even, done on the host) multiply exactly
  in fp32, so the GPU result must equal the float64 product of the rounded
  operands up to fp32 summation error: the same normalised error bound (1e-4)
  as the fp32 GEMM, against that reference.
* Against the unrounded operands the error is of the order of bf16 rounding
  (2^-8), and clearly larger than fp32 -- the products really are bf16.
* Integers of magnitude <= 8 are exact in bf16: bit-exact, every tile shape,
  layout and edge path.
* A transformer step in bf16 mode stays close to the fp32 step."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd import kernels as K
from pico_amd.pico import Pico
from tests._util import gemm_err, max_rel

pytestmark = pytest.mark.gpu
TOL = 1e-4


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


def _ops(ta, tb, M, N, Kd, seed, integer=False):
    if integer:
        rng = np.random.default_rng(seed)
        A = rng.integers(-8, 9, (M, Kd)).astype(np.float32)
        B = rng.integers(-8, 9, (Kd, N)).astype(np.float32)
    else:
        A = O.uniform(M * Kd, seed).reshape(M, Kd)
        B = O.uniform(Kd * N, seed + 1).reshape(Kd, N)
    return A, B, (np.ascontiguousarray(A.T) if ta == "T" else A), \
        (np.ascontiguousarray(B.T) if tb == "T" else B)


def test_bf16_rounding_helper_known_values():
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: to even (1); just above rounds up
    x = np.array([1.0, 1 + 2 ** -8, 1 + 2 ** -8 + 2 ** -20, 1 + 3 * 2 ** -8, -2.5], np.float32)
    assert bf16_round(x).tolist() == [1.0, 1.0, 1 + 2 ** -7, 1 + 2 ** -6, -2.5]


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,Kd", [(4096, 4096, 512), (1000, 1376, 516), (8192, 768, 768),
                                    (200, 136, 70), (64, 128, 784)])
def test_bf16_gemm_equals_product_of_rounded_operands(dev, ta, tb, M, N, Kd):
    A, B, As, Bs = _ops(ta, tb, M, N, Kd, seed=M + N + Kd)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm_bf16(ta, tb, cu(As), cu(Bs), C)
    Cn = host(C)
    Ar, Br = bf16_round(A), bf16_round(B)
    assert gemm_err(Cn, Ar, Br) <= TOL
    e = gemm_err(Cn, A, B)
    assert 1e-5 < e < 2 ** -7  # bf16-sized, not fp32-sized


@pytest.mark.parametrize("ta,tb", [("N", "N"), ("N", "T"), ("T", "N"), ("T", "T")])
@pytest.mark.parametrize("M,N,Kd", [(4096, 4096, 256), (4000, 4000, 200), (8192, 768, 768),
                                    (1024, 1024, 1024), (130, 257, 70), (64, 10, 784)])
def test_bf16_gemm_integers_bitexact(dev, ta, tb, M, N, Kd):
    A, B, As, Bs = _ops(ta, tb, M, N, Kd, seed=3 * M + N + Kd, integer=True)
    C = torch.full((M, N), float("nan"), device=dev)
    K.gemm_bf16(ta, tb, cu(As), cu(Bs), C)
    ref = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.float32)
    assert np.array_equal(host(C), ref)
    C = cu(ref.copy())
    K.gemm_bf16(ta, tb, cu(As), cu(Bs), C, alpha=-1.0, beta=1.0)
    assert not np.any(host(C))


def test_bf16_gemm_split_k_workspace(dev):
    # a weight-gradient shape splits over K through the workspace, deterministically
    M, N, Kd = 768, 768, 8192
    A, B, As, Bs = _ops("T", "N", M, N, Kd, seed=11)
    ws = torch.empty(K.gemm_workspace(M, N, Kd) // 4 + 1, device=dev)
    C1 = torch.empty(M, N, device=dev)
    C2 = torch.empty(M, N, device=dev)
    K.gemm_bf16("T", "N", cu(As), cu(Bs), C1, ws=ws)
    K.gemm_bf16("T", "N", cu(As), cu(Bs), C2, ws=ws)
    assert np.array_equal(host(C1), host(C2))
    assert gemm_err(host(C1), bf16_round(A), bf16_round(B)) <= TOL


def test_pico_matmul_precision_switch(dev):
    P = Pico()
    cfg = dict(vocab=96, d_model=64, n_layers=2, n_heads=2, d_ff=160, batch=2, seq_len=64)
    seq = O.labels(cfg["batch"] * (cfg["seq_len"] + 1), 77, cfg["vocab"]).reshape(2, -1)
    tok, tgt = seq[:, :-1].ravel(), seq[:, 1:].ravel()
    assert P.lib.pico_get_matmul_precision() == 0
    out = {}
    for prec in (0, 1):
        assert P.lib.pico_set_matmul_precision(prec) == 0
        model = P.gpt_init(cfg, 3)
        with P.arena(1 << 26):
            loss = P.gpt_loss(model, tok, tgt)
            P.backward(loss)
            out[prec] = (float(P.data(loss)[0]), [P.grad(t) for t in P.gpt_params(model)])
        P.gpt_free(model)
    assert P.lib.pico_set_matmul_precision(0) == 0
    assert P.lib.pico_set_matmul_precision(7) != 0 and P.lib.pico_get_matmul_precision() == 0
    (l32, g32), (l16, g16) = out[0], out[1]
    assert l16 != l32 and abs(l16 - l32) <= 1e-2 * abs(l32)
    for a, b in zip(g32, g16):
        assert max_rel(b, a) <= 5e-2
