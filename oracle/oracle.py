"""ctypes bindings of the CPU oracle (oracle/liboracle.so) -- TEST INFRASTRUCTURE.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg use
this module, as the checker; the product (pico_amd/) never imports it.

Also exposes the reference itself (oracle/_ref/libpicoref.so, built from the
reference's own sources where they are present) for cross-checks.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libpicoref.so")

_F = np.float32
c_i64, c_f, c_p, c_int, c_u32 = ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_int, ctypes.c_uint32

_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run make -C oracle)")
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.pico_init()
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    global _ref
    if _ref is None:
        _ref = ctypes.CDLL(REF_PATH)
        _ref.picoref_init_pool()
    return _ref


def p(a):
    return None if a is None else a.ctypes.data_as(c_p)


def f32(a):
    return np.ascontiguousarray(a, dtype=_F)


# ------------------------------------------------------------------ inputs
def uniform(n, seed, lo=-1.0, hi=1.0):
    out = np.empty(n, _F)
    lib().ora_fill_uniform(p(out), c_i64(n), c_u32(seed), c_f(lo), c_f(hi))
    return out


def normal(n, seed, mean=0.0, std=1.0):
    out = np.empty(n, _F)
    lib().ora_fill_normal(p(out), c_i64(n), c_u32(seed), c_f(mean), c_f(std))
    return out


def labels(n, seed, vocab):
    out = np.empty(n, np.int32)
    lib().ora_fill_labels(p(out), c_i64(n), c_u32(seed), c_int(vocab))
    return out


def pico_rand(n, seed):
    out = np.empty(n, _F)
    lib().ora_fill_pico_rand(p(out), c_i64(n), c_u32(seed))
    return out


# ------------------------------------------------------------------ matmul
def set_threads(n):
    lib().ora_set_threads(c_int(n))


def matmul_scalar(A, B, C=None):
    A, B = f32(A), f32(B)
    M, K = A.shape
    N = B.shape[1]
    C = np.zeros((M, N), _F) if C is None else C
    lib().ora_matmul_scalar(c_int(M), c_int(N), c_int(K), p(A), c_i64(K), c_i64(1), p(B),
                            c_i64(N), c_i64(1), p(C), c_i64(N), c_i64(1))
    return C


def matmul_avx(A, B, C=None):
    A, B = f32(A), f32(B)
    M, K = A.shape
    N = B.shape[1]
    C = np.zeros((M, N), _F) if C is None else C
    lib().ora_matmul_avx(c_int(M), c_int(N), c_int(K), p(A), c_i64(K), c_i64(1), p(B), c_i64(N),
                         c_i64(1), p(C), c_i64(N), c_i64(1))
    return C


def matmul_backward(A, B, dC, dA=None, dB=None):
    A, B, dC = f32(A), f32(B), f32(dC)
    M, K = A.shape
    N = B.shape[1]
    dA = np.zeros((M, K), _F) if dA is None else dA
    dB = np.zeros((K, N), _F) if dB is None else dB
    lib().ora_matmul_backward(c_int(M), c_int(K), c_int(N), p(A), p(B), p(dC), p(dA), p(dB))
    return dA, dB


def gemm_pico_order(ta, tb, A, B, C):
    """C += op(A) @ op(B) with float accumulation in k order (pico's backward loops)."""
    A, B = f32(A), f32(B)
    M = A.shape[1] if ta == "T" else A.shape[0]
    K = A.shape[0] if ta == "T" else A.shape[1]
    N = B.shape[0] if tb == "T" else B.shape[1]
    lib().ora_gemm_pico_order(ctypes.c_char(ta.encode()), ctypes.c_char(tb.encode()), c_int(M),
                              c_int(N), c_int(K), p(A), c_i64(A.shape[1]), p(B), c_i64(B.shape[1]),
                              p(C), c_i64(C.shape[1]))
    return C


def gemm_ref_f64(ta, tb, A, B, alpha=1.0, beta=0.0, C=None):
    A, B = f32(A), f32(B)
    M = A.shape[1] if ta == "T" else A.shape[0]
    K = A.shape[0] if ta == "T" else A.shape[1]
    N = B.shape[0] if tb == "T" else B.shape[1]
    C = np.zeros((M, N), _F) if C is None else C
    lib().ora_gemm_ref_f64(ctypes.c_char(ta.encode()), ctypes.c_char(tb.encode()), c_int(M),
                           c_int(N), c_int(K), c_f(alpha), p(A), c_i64(A.shape[1]), p(B),
                           c_i64(B.shape[1]), c_f(beta), p(C), c_i64(C.shape[1]))
    return C


# -------------------------------------------------------------- elementwise
def _shape_arr(s):
    s = list(s) or [1]
    return (c_i64 * len(s))(*s), len(s)


def binary(op, a, b):
    a, b = f32(a), f32(b)
    out_shape = np.broadcast_shapes(a.shape, b.shape)
    out = np.empty(out_shape, _F)
    os_, nd = _shape_arr(out_shape)
    as_, na = _shape_arr(a.shape)
    bs_, nb = _shape_arr(b.shape)
    lib().ora_binary(c_int(op), c_int(nd), os_, p(a), c_int(na), as_, p(b), c_int(nb), bs_, p(out))
    return out


def binary_bwd(op, a, b, gout, ga, gb):
    a, b, gout = f32(a), f32(b), f32(gout)
    os_, nd = _shape_arr(gout.shape)
    as_, na = _shape_arr(a.shape)
    bs_, nb = _shape_arr(b.shape)
    lib().ora_binary_bwd(c_int(op), c_int(nd), os_, p(a), c_int(na), as_, p(b), c_int(nb), bs_,
                         p(gout), p(ga), p(gb))
    return ga, gb


def unary(op, x):
    x = f32(x)
    y = np.empty_like(x)
    lib().ora_unary(c_int(op), c_i64(x.size), p(x), p(y))
    return y


def unary_bwd(op, x, y, gy, gx):
    lib().ora_unary_bwd(c_int(op), c_i64(x.size), p(f32(x)), p(f32(y)), p(f32(gy)), p(gx))
    return gx


def relu(x):
    x = f32(x)
    y = np.empty_like(x)
    lib().ora_relu(c_i64(x.size), p(x), p(y))
    return y


def relu_bwd(y, gy, gx):
    lib().ora_relu_bwd(c_i64(y.size), p(f32(y)), p(f32(gy)), p(gx))
    return gx


def sgd(pv, g, lr):
    lib().ora_sgd(c_i64(pv.size), c_f(lr), p(pv), p(f32(g)))
    return pv


def adamw(pv, g, m, v, lr, b1, b2, eps, wd, step):
    lib().ora_adamw(c_i64(pv.size), c_f(lr), c_f(b1), c_f(b2), c_f(eps), c_f(wd), c_int(step),
                    p(pv), p(None if g is None else f32(g)), p(m), p(v))
    return pv


# ------------------------------------------------------------ row kernels
def xent(logits, labels_, scale=1.0, want_grad=True):
    z = f32(logits)
    R, V = z.shape
    loss = np.empty(R, _F)
    dz = np.empty_like(z) if want_grad else None
    lib().ora_xent_fwd_bwd(c_i64(R), c_i64(V), p(z), p(np.ascontiguousarray(labels_, np.int32)),
                           p(loss), p(dz), c_f(scale))
    return loss, dz


def argmax(x):
    x = f32(x)
    R, V = x.shape
    idx = np.empty(R, np.int32)
    lib().ora_argmax(c_i64(R), c_i64(V), p(x), p(idx))
    return idx


def rmsnorm_fwd(x, g, eps):
    x, g = f32(x), f32(g)
    R, C = x.shape
    y = np.empty_like(x)
    rstd = np.empty(R, _F)
    lib().ora_rmsnorm_fwd(c_i64(R), c_i64(C), c_f(eps), p(x), p(g), p(y), p(rstd))
    return y, rstd


def rmsnorm_bwd(x, g, rstd, dy, dx=None, dg=None):
    x, g, rstd, dy = f32(x), f32(g), f32(rstd), f32(dy)
    R, C = x.shape
    dx = np.zeros_like(x) if dx is None else dx
    dg = np.zeros(C, _F) if dg is None else dg
    lib().ora_rmsnorm_bwd(c_i64(R), c_i64(C), p(x), p(g), p(rstd), p(dy), p(dx), p(dg))
    return dx, dg


def swiglu_fwd(a, u):
    a, u = f32(a), f32(u)
    h = np.empty_like(a)
    lib().ora_swiglu_fwd(c_i64(a.size), p(a), p(u), p(h))
    return h


def swiglu_bwd(a, u, dh, da=None, du=None):
    a, u, dh = f32(a), f32(u), f32(dh)
    da = np.zeros_like(a) if da is None else da
    du = np.zeros_like(a) if du is None else du
    lib().ora_swiglu_bwd(c_i64(a.size), p(a), p(u), p(dh), p(da), p(du))
    return da, du


def attn_fwd(B, H, q, k, v, scale=None):
    q, k, v = f32(q), f32(k), f32(v)
    BT, D = q.shape
    T, hd = BT // B, D // H
    scale = hd ** -0.5 if scale is None else scale
    o = np.empty_like(q)
    lse = np.empty(B * H * T, _F)
    lib().ora_attn_causal_fwd(c_int(B), c_int(H), c_int(T), c_int(hd), c_f(scale), p(q), p(k),
                              p(v), p(o), p(lse))
    return o, lse


def attn_bwd(B, H, q, k, v, o, lse, dout, scale=None):
    q, k, v, o, lse, dout = (f32(t) for t in (q, k, v, o, lse, dout))
    BT, D = q.shape
    T, hd = BT // B, D // H
    scale = hd ** -0.5 if scale is None else scale
    dq, dk, dv = np.zeros_like(q), np.zeros_like(q), np.zeros_like(q)
    lib().ora_attn_causal_bwd(c_int(B), c_int(H), c_int(T), c_int(hd), c_f(scale), p(q), p(k),
                              p(v), p(o), p(lse), p(dout), p(dq), p(dk), p(dv))
    return dq, dk, dv


def embed_fwd(ids, table):
    ids = np.ascontiguousarray(ids, np.int32)
    table = f32(table)
    out = np.empty((ids.size, table.shape[1]), _F)
    lib().ora_embed_fwd(c_i64(ids.size), c_i64(table.shape[1]), p(ids), p(table), p(out))
    return out


def embed_bwd(ids, dout, dtable):
    ids = np.ascontiguousarray(ids, np.int32)
    lib().ora_embed_bwd(c_i64(ids.size), c_i64(dtable.shape[1]), p(ids), p(f32(dout)), p(dtable))
    return dtable


# ------------------------------------------------- pico API (struct level)
class PicoTensor(ctypes.Structure):
    """struct PicoTensor, field for field (src/tensor.h:11-23)."""
    _fields_ = [
        ("shape", ctypes.POINTER(c_i64)),
        ("strides", ctypes.POINTER(c_i64)),
        ("data", ctypes.POINTER(ctypes.c_float)),
        ("grad", ctypes.POINTER(ctypes.c_float)),
        ("_backward", c_p),
        ("parents", c_p),
        ("numel", c_i64),
        ("backend", c_int),
        ("ndim", ctypes.c_uint8),
        ("num_parents", ctypes.c_uint8),
        ("is_persistent", ctypes.c_uint8),
    ]


PT = ctypes.POINTER(PicoTensor)


def api():
    """The oracle's pico_* functions with their C types declared."""
    L = lib()
    if getattr(L, "_api_ready", False):
        return L
    for name in ("pico_add", "pico_sub", "pico_mul", "pico_matmul"):
        getattr(L, name).argtypes = [PT, PT]
        getattr(L, name).restype = PT
    for name in ("pico_tensor_sqrt", "pico_tensor_sin", "pico_tensor_cos", "pico_tensor_tan",
                 "pico_tensor_tanh", "pico_tensor_log", "pico_relu"):
        getattr(L, name).argtypes = [PT]
        getattr(L, name).restype = PT
    _declare_api(L)
    L.arena_init.argtypes = [ctypes.c_size_t]
    L.arena_init.restype = c_p
    L.arena_ctx_push.argtypes = [c_p]
    L.arena_reset.argtypes = [c_p]
    L.arena_destroy.argtypes = [c_p]
    L.pico_softmax_xent.argtypes = [PT, c_p]
    L.pico_softmax_xent.restype = PT
    L.pico_rmsnorm.argtypes = [PT, PT, c_f]
    L.pico_rmsnorm.restype = PT
    L.pico_swiglu.argtypes = [PT, PT]
    L.pico_swiglu.restype = PT
    L.pico_attention_causal.argtypes = [PT, PT, PT, c_int, c_int]
    L.pico_attention_causal.restype = PT
    L.pico_embedding.argtypes = [PT, c_p, c_i64]
    L.pico_embedding.restype = PT
    L.pico_optim_adamw_init.argtypes = [c_f, c_f, c_f, c_f, c_f]
    L.pico_optim_adamw_init.restype = c_p
    L.pico_optim_adamw_add.argtypes = [c_p, PT]
    L.pico_optim_adamw_step.argtypes = [c_p]
    L.pico_optim_adamw_zero_grad.argtypes = [c_p]
    L.pico_optim_adamw_free.argtypes = [c_p]
    L._api_ready = True
    return L


class PicoLinear(ctypes.Structure):
    """struct PicoLinear (src/nn/linear.h:6-11)."""
    _fields_ = [("in_features", c_int), ("out_features", c_int), ("weights", PT), ("bias", PT)]


def _declare_api(L):
    for name in ("pico_add", "pico_sub", "pico_mul", "pico_matmul"):
        getattr(L, name).argtypes = [PT, PT]
        getattr(L, name).restype = PT
    L.pico_relu.argtypes = [PT]
    L.pico_relu.restype = PT
    L.pico_param.argtypes = [ctypes.POINTER(c_i64), ctypes.c_uint8]
    L.pico_param.restype = PT
    L.pico_create_tensor.argtypes = [c_p, ctypes.POINTER(c_i64), ctypes.c_uint8]
    L.pico_create_tensor.restype = PT
    L.pico_free.argtypes = [PT]
    L.pico_backward.argtypes = [c_p, PT]
    L.pico_transpose_2d.argtypes = [PT]
    L.pico_optim_sgd_init.argtypes = [c_f]
    L.pico_optim_sgd_init.restype = c_p
    for name in ("pico_optim_sgd_step", "pico_optim_sgd_zero_grad", "pico_optim_sgd_free"):
        getattr(L, name).argtypes = [c_p]
    L.pico_optim_sgd_add.argtypes = [c_p, PT]
    L.pico_nn_linear_init.argtypes = [c_int, c_int, ctypes.c_bool]
    L.pico_nn_linear_init.restype = ctypes.POINTER(PicoLinear)
    L.pico_nn_linear_forward.argtypes = [ctypes.POINTER(PicoLinear), PT]
    L.pico_nn_linear_forward.restype = PT
    L.pico_nn_linear_free.argtypes = [ctypes.POINTER(PicoLinear)]


def ref_api():
    """The compiled reference's own pico API (src/ops.h, tensor.h, act/,
    optim/, nn/) with its C types declared, plus its static-inline arena
    helpers under their pico names (ref_shim.c's wrappers), so one call
    sequence runs on both ``api()`` and ``ref_api()``.  ``simd`` picks the
    reference's kernel level (pico_init's AVX2 by default, as the oracle's
    pico_init does)."""
    R = ref()
    if not getattr(R, "_api_ready", False):
        _declare_api(R)
        for name in ("arena_init", "arena_destroy", "arena_reset", "arena_ctx_push",
                     "arena_ctx_pop"):
            setattr(R, name, getattr(R, "picoref_" + name))
        R.arena_init.argtypes = [ctypes.c_size_t]
        R.arena_init.restype = c_p
        R.arena_destroy.argtypes = [c_p]
        R.arena_reset.argtypes = [c_p]
        R.arena_ctx_push.argtypes = [c_p]
        R._api_ready = True
    return R


def set_simd(L, level):
    """g_simd_level of a library that exports it (src/global.h:7: 0 none .. 3 AVX2)"""
    c_int.in_dll(L, "g_simd_level").value = level


def param(shape, values=None):
    L = api()
    arr = (c_i64 * len(shape))(*shape)
    t = L.pico_param(arr, len(shape))
    if values is not None:
        set_data(t, values)
    return t


def set_data(t, values):
    v = np.ascontiguousarray(values, _F).reshape(-1)
    ctypes.memmove(t.contents.data, v.ctypes.data, v.nbytes)


def data(t):
    n = t.contents.numel
    return np.ctypeslib.as_array(t.contents.data, shape=(n,)).copy()


def grad(t):
    n = t.contents.numel
    return np.ctypeslib.as_array(t.contents.grad, shape=(n,)).copy()


def set_grad(t, values):
    v = np.ascontiguousarray(values, _F).reshape(-1)
    ctypes.memmove(t.contents.grad, v.ctypes.data, v.nbytes)
