"""pico's own tensors through the GPU twins of its op seam ("Way 2").

pico's ops.c leaves `pico_<op>_gpu(a, b, out)` stubs at src/ops.c:42-44, 86-88,
130-132 (and none yet for matmul at :178), and its backward hooks run on
`self->parents` (src/autograd.h:53-130).  A maintainer who fills those stubs in
calls this library's twins with tensors that pico allocated itself: a struct of
exactly sizeof(struct PicoTensor) = 64 bytes, calloc'd (src/tensor.c:44-84) or
packed back to back in pico's arena blocks, whose data and grad pico took from
device memory.  Those tensors are not this library's nodes: their grads are
always live and every backward contribution accumulates (+=), exactly the
reference's semantics.

Here such tensors are built in host memory with libc's calloc / malloc (never
by this library), with device data and grads from torch or from
arena_alloc_device on a 16-byte pico-layout arena, and the twins' results are
compared with the CPU oracle, which restates pico's loops: bit-exact for
add/sub/mul (pico's order, no contraction) and for matmul on integer-valued
operands (every partial sum exact), within 1e-4 (normalised) for matmul on
uniform operands.  Starting grads are nonzero, so `+=` is what is checked.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from pico_amd.pico import PicoTensor, TP, amd_lib
from tests._util import gemm_err

pytestmark = pytest.mark.gpu

c_p = ctypes.c_void_p
c_i64 = ctypes.c_int64
HOOK = ctypes.CFUNCTYPE(None, TP)
GPU = 1

libc = ctypes.CDLL(None)
libc.calloc.restype = c_p
libc.calloc.argtypes = [ctypes.c_size_t, ctypes.c_size_t]
libc.malloc.restype = c_p
libc.malloc.argtypes = [ctypes.c_size_t]
libc.free.argtypes = [c_p]


@pytest.fixture(scope="module")
def lib(dev):
    L = amd_lib()
    L.pico_init()
    for n in ("pico_add_gpu", "pico_sub_gpu", "pico_mul_gpu", "pico_matmul_gpu"):
        getattr(L, n).argtypes = [TP, TP, TP]
        getattr(L, n).restype = ctypes.c_int
    for n in ("pico_add_backward_gpu", "pico_sub_backward_gpu", "pico_mul_backward_gpu",
              "pico_matmul_backward_gpu", "pico_relu_backward_gpu"):
        getattr(L, n).argtypes = [TP]
        getattr(L, n).restype = None
    L.arena_alloc_device.argtypes = [c_p, ctypes.c_size_t]
    L.arena_alloc_device.restype = c_p
    L.arena_device_reset.argtypes = [c_p]
    L.arena_device_release.argtypes = [c_p]
    L.pico_gpu_synchronize.restype = ctypes.c_int
    L.pico_gpu_last_error.restype = ctypes.c_char_p
    return L


class Foreign:
    """Tensors laid out as pico lays them out: host structs from libc, device
    data and grad.  `packed` puts every struct back to back in one malloc'd
    block, as pico's arena does; otherwise each is its own 64-byte calloc."""

    def __init__(self, packed=False, capacity=16):
        assert ctypes.sizeof(PicoTensor) == 64
        self.keep = []  # torch buffers the structs point at
        self.frees = []
        self.packed = packed
        if packed:
            self.block = libc.malloc(capacity * 64)
            ctypes.memset(self.block, 0xAB, capacity * 64)  # pico's arena memory is not zeroed
            self.frees.append(self.block)
            self.used = 0
            self.capacity = capacity

    def _struct(self):
        if self.packed:
            assert self.used < self.capacity
            addr = self.block + 64 * self.used
            self.used += 1
            ctypes.memset(addr, 0, 64)
        else:
            addr = libc.calloc(1, 64)
            self.frees.append(addr)
        return ctypes.cast(addr, TP)

    def tensor(self, values, grad=None, data_ptr=None, grad_ptr=None):
        """a GPU-backed pico tensor holding `values` (grad = `grad` or zeros)"""
        values = np.ascontiguousarray(values, np.float32)
        shape = values.shape
        t = self._struct()
        nd = len(shape)
        sh = libc.calloc(nd, 8)
        st = libc.calloc(nd, 8)
        self.frees += [sh, st]
        sha = ctypes.cast(sh, ctypes.POINTER(c_i64))
        sta = ctypes.cast(st, ctypes.POINTER(c_i64))
        s = 1
        for i in range(nd - 1, -1, -1):
            sha[i] = shape[i]
            sta[i] = s
            s *= shape[i]
        t.contents.shape = sha
        t.contents.strides = sta
        t.contents.numel = values.size
        t.contents.ndim = nd
        t.contents.backend = GPU
        g = np.zeros(shape, np.float32) if grad is None else np.asarray(grad, np.float32)
        if data_ptr is None:
            d = torch.from_numpy(values.copy()).cuda()
            gd = torch.from_numpy(np.ascontiguousarray(g)).cuda()
            self.keep += [d, gd]
            t.contents.data = d.data_ptr()
            t.contents.grad = gd.data_ptr()
        else:
            t.contents.data = data_ptr
            t.contents.grad = grad_ptr
            _h2d(data_ptr, values)
            _h2d(grad_ptr, g)
        torch.cuda.synchronize()
        return t

    def wire(self, out, parents, backward):
        """out->parents / num_parents / _backward, as pico's ops.c sets them"""
        arr = libc.calloc(len(parents), 8)
        self.frees.append(arr)
        pa = ctypes.cast(arr, ctypes.POINTER(TP))
        for i, p in enumerate(parents):
            pa[i] = p
        out.contents.parents = pa
        out.contents.num_parents = len(parents)
        out.contents._backward = ctypes.cast(backward, c_p).value

    def close(self):
        for a in self.frees:
            libc.free(a)
        self.frees = []


_hip = None


def _hip_lib():
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [c_p, c_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipMemcpy.restype = ctypes.c_int
    return _hip


def _h2d(dst, arr):
    arr = np.ascontiguousarray(arr, np.float32)
    assert _hip_lib().hipMemcpy(dst, arr.ctypes.data, arr.nbytes, 1) == 0


def _d2h(src, shape):
    out = np.empty(shape, np.float32)
    assert _hip_lib().hipMemcpy(out.ctypes.data, src, out.nbytes, 2) == 0
    return out


def data(t):
    return _d2h(t.contents.data, tuple(t.contents.shape[i] for i in range(t.contents.ndim)))


def grad(t):
    return _d2h(t.contents.grad, tuple(t.contents.shape[i] for i in range(t.contents.ndim)))


def ints(shape, seed, lo=-4, hi=5):
    return np.random.default_rng(seed).integers(lo, hi, size=shape).astype(np.float32)


OPS = [("add", 0), ("sub", 1), ("mul", 2)]
SHAPES = [((6, 7), (6, 7)), ((4, 5, 6), (5, 1)), ((3, 1, 8), (1, 5, 8)), ((1,), (9, 4))]


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("op,code", OPS)
@pytest.mark.parametrize("sa,sb", SHAPES)
def test_binary_twins_on_pico_tensors(lib, packed, op, code, sa, sb):
    F = Foreign(packed)
    try:
        a_v = O.uniform(int(np.prod(sa)), 11).reshape(sa)
        b_v = O.uniform(int(np.prod(sb)), 12).reshape(sb)
        ga0 = O.uniform(a_v.size, 13).reshape(sa)
        gb0 = O.uniform(b_v.size, 14).reshape(sb)
        oshape = np.broadcast_shapes(sa, sb)
        g_up = O.uniform(int(np.prod(oshape)), 15).reshape(oshape)
        a = F.tensor(a_v, ga0)
        b = F.tensor(b_v, gb0)
        out = F.tensor(np.zeros(oshape, np.float32), g_up)  # pico zeroes out
        assert getattr(lib, f"pico_{op}_gpu")(a, b, out) == 0
        assert lib.pico_gpu_synchronize() == 0
        assert np.array_equal(data(out), O.binary(code, a_v, b_v))
        F.wire(out, [a, b], getattr(lib, f"pico_{op}_backward_gpu"))
        HOOK(out.contents._backward)(out)  # pico_backward calls the hook this way
        assert lib.pico_gpu_synchronize() == 0
        ea, eb = O.binary_bwd(code, a_v, b_v, g_up, ga0.copy(), gb0.copy())
        assert np.array_equal(grad(a), ea)
        assert np.array_equal(grad(b), eb)
        # the upstream grad and the operands' data are untouched
        assert np.array_equal(grad(out), g_up)
        assert np.array_equal(data(a), a_v) and np.array_equal(data(b), b_v)
    finally:
        F.close()


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("M,K,N", [(2, 3, 2), (37, 29, 41), (128, 256, 96), (300, 64, 520)])
def test_matmul_twins_integer_exact(lib, packed, M, K, N):
    F = Foreign(packed)
    try:
        A, B = ints((M, K), 1), ints((K, N), 2)
        dA0, dB0 = ints((M, K), 3), ints((K, N), 4)
        dC = ints((M, N), 5, -2, 3)
        a, b = F.tensor(A, dA0), F.tensor(B, dB0)
        out = F.tensor(np.zeros((M, N), np.float32), dC)
        assert lib.pico_matmul_gpu(a, b, out) == 0
        assert lib.pico_gpu_synchronize() == 0
        assert np.array_equal(data(out), O.matmul_scalar(A, B))
        F.wire(out, [a, b], lib.pico_matmul_backward_gpu)
        HOOK(out.contents._backward)(out)
        assert lib.pico_gpu_synchronize() == 0
        eA, eB = O.matmul_backward(A, B, dC, dA0.copy(), dB0.copy())
        assert np.array_equal(grad(a), eA)
        assert np.array_equal(grad(b), eB)
    finally:
        F.close()


def test_matmul_twins_uniform_within_tolerance(lib):
    F = Foreign()
    try:
        M, K, N = 257, 513, 130
        A = O.uniform(M * K, 21).reshape(M, K)
        B = O.uniform(K * N, 22).reshape(K, N)
        dA0 = O.uniform(M * K, 23).reshape(M, K)
        dB0 = O.uniform(K * N, 24).reshape(K, N)
        dC = O.uniform(M * N, 25).reshape(M, N)
        a, b = F.tensor(A, dA0), F.tensor(B, dB0)
        out = F.tensor(np.zeros((M, N), np.float32), dC)
        assert lib.pico_matmul_gpu(a, b, out) == 0
        F.wire(out, [a, b], lib.pico_matmul_backward_gpu)
        HOOK(out.contents._backward)(out)
        assert lib.pico_gpu_synchronize() == 0
        assert gemm_err(data(out), A, B) <= 1e-4
        # dA - dA0 = dC . B^T, dB - dB0 = A^T . dC, each against fp64
        ref_dA = dA0.astype(np.float64) + dC.astype(np.float64) @ B.T.astype(np.float64)
        ref_dB = dB0.astype(np.float64) + A.T.astype(np.float64) @ dC.astype(np.float64)
        den_a = np.abs(dC) @ np.abs(B.T) + np.abs(dA0)
        den_b = np.abs(A.T) @ np.abs(dC) + np.abs(dB0)
        assert np.max(np.abs(grad(a) - ref_dA) / den_a) <= 1e-4
        assert np.max(np.abs(grad(b) - ref_dB) / den_b) <= 1e-4
    finally:
        F.close()


def test_relu_backward_twin(lib):
    F = Foreign(packed=True)
    try:
        x = O.uniform(400, 31).reshape(20, 20)
        x[0, :5] = [0.0, -0.0, 1.0, -1.0, 0.5]
        y = O.relu(x)
        g0 = O.uniform(400, 32).reshape(20, 20)
        gy = O.uniform(400, 33).reshape(20, 20)
        xt = F.tensor(x, g0)
        yt = F.tensor(y, gy)
        F.wire(yt, [xt], lib.pico_relu_backward_gpu)
        HOOK(yt.contents._backward)(yt)
        assert lib.pico_gpu_synchronize() == 0
        assert np.array_equal(grad(xt), O.relu_bwd(y, gy, g0.copy()))
    finally:
        F.close()


def test_pico_arena_device_blocks_and_a_small_graph(lib):
    """Data and grads from arena_alloc_device on a 16-byte arena laid out as
    pico's (src/arena.h:27-29, 38-64); a graph z = (x.W + b) * s run through the
    twins and its backward hooks called in pico_backward's reverse post-order
    with the seed written on the device, against the oracle."""
    # pico's arena_init: malloc'd Arena {begin, end} and its first ArenaBlock
    arena = libc.malloc(16)
    block = libc.malloc(32)
    bottom = libc.malloc(1 << 16)
    blk = (ctypes.c_void_p * 4).from_address(block)
    blk[0], blk[1], blk[2], blk[3] = None, 1 << 16, bottom, bottom
    ar = (ctypes.c_void_p * 2).from_address(arena)
    ar[0] = ar[1] = block
    F = Foreign()

    def dev(n):
        p = lib.arena_alloc_device(arena, 4 * n)
        assert p and p % 256 == 0
        return p

    try:
        M, K, N = 8, 12, 5
        X, W = ints((M, K), 41), ints((K, N), 42)
        bias, s = ints((N,), 43), ints((M, N), 44)
        gx0, gw0, gb0, gs0 = ints((M, K), 45), ints((K, N), 46), ints((N,), 47), ints((M, N), 48)

        def mk(v, g):
            return F.tensor(v, g, data_ptr=dev(v.size), grad_ptr=dev(v.size))

        x, w, b, st = mk(X, gx0), mk(W, gw0), mk(bias, gb0), mk(s, gs0)
        zeros = np.zeros((M, N), np.float32)
        h = mk(zeros, zeros)
        assert lib.pico_matmul_gpu(x, w, h) == 0
        F.wire(h, [x, w], lib.pico_matmul_backward_gpu)
        hb = mk(zeros, zeros)
        assert lib.pico_add_gpu(h, b, hb) == 0
        F.wire(hb, [h, b], lib.pico_add_backward_gpu)
        z = mk(zeros, np.ones((M, N), np.float32))  # pico_backward's seed of 1
        assert lib.pico_mul_gpu(hb, st, z) == 0
        F.wire(z, [hb, st], lib.pico_mul_backward_gpu)
        for t in (z, hb, h):  # reverse post-order of the graph
            HOOK(t.contents._backward)(t)
        assert lib.pico_gpu_synchronize() == 0

        Hm = O.matmul_scalar(X, W)
        HB = O.binary(0, Hm, bias)
        Z = O.binary(2, HB, s)
        assert np.array_equal(data(z), Z)
        ghb, gs = O.binary_bwd(2, HB, s, np.ones((M, N), np.float32), zeros.copy(), gs0.copy())
        gh, gb = O.binary_bwd(0, Hm, bias, ghb, zeros.copy(), gb0.copy())
        gx, gw = O.matmul_backward(X, W, gh, gx0.copy(), gw0.copy())
        assert np.array_equal(grad(st), gs)
        assert np.array_equal(grad(b), gb)
        assert np.array_equal(grad(x), gx)
        assert np.array_equal(grad(w), gw)
        # pico's arena_reset adds arena_device_reset: the same addresses again
        first = x.contents.data
        lib.arena_device_reset(arena)
        assert lib.arena_alloc_device(arena, 4 * X.size) == first
    finally:
        lib.arena_device_release(arena)
        F.close()
        untouched = ar[0] == block and ar[1] == block  # pico's own fields
        for p in (bottom, block, arena):
            libc.free(p)
    assert untouched


def test_twins_refuse_cpu_tensors(lib):
    F = Foreign()
    try:
        a = F.tensor(np.ones((2, 2), np.float32))
        b = F.tensor(np.ones((2, 2), np.float32))
        out = F.tensor(np.zeros((2, 2), np.float32))
        b.contents.backend = 0  # CPU
        assert lib.pico_add_gpu(a, b, out) != 0
        assert b"backend is GPU" in lib.pico_gpu_last_error()
        assert lib.pico_matmul_gpu(a, b, out) != 0
        lib.pico_gpu_clear_error()
    finally:
        F.close()
