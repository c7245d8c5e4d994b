"""Way 2 end to end: pico's OWN op layer on GPU tensors.

oracle/_ref/libpico_way2.so is the reference's src/ compiled with the Way 2
binding applied by oracle/way2_patch.py (pico_add / pico_sub / pico_mul /
pico_matmul call the twins of libpico_amd.so for GPU tensors, _backward is the
GPU hook, pico_backward seeds on the device, SGD steps with pk_sgd_f32, arena
reset / destroy also rewind / free the device blocks).  Here a graph is built
and trained with pico's own functions -- its arena, ops, pico_backward and
SGD -- on tensors pico allocated itself (pico_param with device data and grad,
op outputs placed in pico's own 16-byte arena's device blocks), and compared
with the same calls on the reference compiled for the CPU (oracle/_ref/
libpicoref.so): bit for bit on integer-valued inputs (every product and sum
exact), within 1e-4 on uniform ones.  Both libraries are built here, from the
reference's sources, by oracle/Makefile; absent, the test is skipped.
"""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
WAY2 = os.path.join(ROOT, "oracle", "_ref", "libpico_way2.so")

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not (os.path.exists(WAY2) and O.ref_available()),
                                 reason="oracle/_ref Way 2 / reference builds absent")]

PT, c_p, c_i64 = O.PT, ctypes.c_void_p, ctypes.c_int64


@pytest.fixture(scope="module")
def W():
    from pico_amd.pico import Pico

    Pico()  # libpico_amd.so loaded and initialised; libpico_way2.so binds to it
    L = ctypes.CDLL(WAY2)
    O._declare_api(L)
    for name in ("arena_init", "arena_destroy", "arena_reset", "arena_ctx_push", "arena_ctx_pop"):
        setattr(L, name, getattr(L, "picoref_" + name))
    L.arena_init.argtypes = [ctypes.c_size_t]
    L.arena_init.restype = c_p
    L.arena_destroy.argtypes = [c_p]
    L.arena_reset.argtypes = [c_p]
    L.arena_ctx_push.argtypes = [c_p]
    L.way2_param_device.argtypes = [ctypes.POINTER(c_i64), ctypes.c_uint8]
    L.way2_param_device.restype = PT
    L.way2_free_device.argtypes = [PT]
    L.way2_copy.argtypes = [PT, ctypes.c_int, c_p, ctypes.c_int]
    return L


class Side:
    """one library's tensors: GPU (Way 2) or CPU (the reference)"""

    def __init__(self, L, gpu):
        self.L, self.gpu = L, gpu

    def param(self, shape, values):
        arr = (c_i64 * len(shape))(*shape)
        if self.gpu:
            t = self.L.way2_param_device(arr, len(shape))
            v = np.ascontiguousarray(values, np.float32).ravel()
            assert t and self.L.way2_copy(t, 0, v.ctypes.data_as(c_p), 1) == 0
        else:
            t = self.L.pico_param(arr, len(shape))
            O.set_data(t, values)
        return t

    def read(self, t, which):
        if not self.gpu:
            return O.grad(t) if which else O.data(t)
        out = np.empty(t.contents.numel, np.float32)
        assert self.L.way2_copy(t, which, out.ctypes.data_as(c_p), 0) == 0
        return out

    def free(self, t):
        (self.L.way2_free_device if self.gpu else self.L.pico_free)(t)


def _train(S, vals, steps=2, lr=0.5):
    """h = x.W, z = h + b (bias broadcast), d = z - c, y = d * w, then
    pico_backward(y) and an SGD step on W and b, `steps` times with zero_grad"""
    L = S.L
    ar = L.arena_init(1 << 22)
    L.arena_ctx_push(ar)
    x, Wt, b, c, w = (S.param(s, v) for s, v in vals)
    opt = L.pico_optim_sgd_init(ctypes.c_float(lr))
    for t in (Wt, b):
        L.pico_optim_sgd_add(opt, t)
    seen = []
    for _ in range(steps):
        L.pico_optim_sgd_zero_grad(opt)
        h = L.pico_matmul(x, Wt)
        z = L.pico_add(h, b)
        d = L.pico_sub(z, c)
        y = L.pico_mul(d, w)
        assert h and z and d and y
        L.pico_backward(ar, y)
        seen += [S.read(t, 0) for t in (h, z, d, y)]
        seen += [S.read(t, 1) for t in (x, Wt, b, c, w, h, z, d)]
        L.pico_optim_sgd_step(opt)
        seen += [S.read(t, 0) for t in (Wt, b)]
        L.arena_reset(ar)  # the Way 2 build also rewinds the device blocks
    L.pico_optim_sgd_free(opt)
    for t in (x, Wt, b, c, w):
        S.free(t)
    L.arena_ctx_pop()
    L.arena_destroy(ar)
    return seen


SHAPES = [(6, 5), (5, 4), (4,), (6, 4), (6, 4)]


def test_way2_pico_ops_on_gpu_tensors_integer_bitexact(W):
    rng = np.random.default_rng(3)
    vals = [(s, rng.integers(-4, 5, int(np.prod(s))).astype(np.float32)) for s in SHAPES]
    R = O.ref_api()
    gpu = _train(Side(W, True), vals)
    cpu = _train(Side(R, False), vals)
    assert len(gpu) == len(cpu)
    for i, (g, c) in enumerate(zip(gpu, cpu)):
        assert np.array_equal(g, c), i


def test_way2_pico_ops_on_gpu_tensors_uniform(W):
    vals = [(s, O.uniform(int(np.prod(s)), 90 + i)) for i, s in enumerate(SHAPES)]
    R = O.ref_api()
    gpu = _train(Side(W, True), vals, steps=3, lr=0.1)
    cpu = _train(Side(R, False), vals, steps=3, lr=0.1)
    for i, (g, c) in enumerate(zip(gpu, cpu)):
        scale = max(float(np.max(np.abs(c))), 1e-6)
        assert float(np.max(np.abs(g - c))) / scale <= 1e-4, i


def test_way2_gpu_backend_is_routed_to_the_device(W):
    """a GPU tensor's op output is device memory, read back through
    libpico_amd.so's pico_tensor_copy_to_host; a CPU tensor still runs pico's
    CPU kernel in the same library"""
    from pico_amd.pico import Pico

    P = Pico()
    ar = W.arena_init(1 << 20)
    W.arena_ctx_push(ar)
    a = W.way2_param_device((c_i64 * 2)(2, 3), 2)
    W.way2_copy(a, 0, np.arange(6, dtype=np.float32).ctypes.data_as(c_p), 1)
    s = W.pico_add(a, a)
    out = np.empty(6, np.float32)
    assert P.lib.pico_tensor_copy_to_host(ctypes.cast(s, P.lib.pico_tensor_copy_to_host.argtypes[0]),
                                          out.ctypes.data_as(c_p)) == 0
    assert out.tolist() == [0, 2, 4, 6, 8, 10]
    hc = W.pico_param((c_i64 * 2)(2, 3), 2)
    O.set_data(hc, np.arange(6, dtype=np.float32))
    assert O.data(W.pico_add(hc, hc)).tolist() == [0, 2, 4, 6, 8, 10]
    W.pico_free(hc)
    W.way2_free_device(a)
    W.arena_ctx_pop()
    W.arena_destroy(ar)
