"""ctypes binding of pico's C API (include/pico_amd.h).

``Pico(lib, device=True)`` wraps ``libpico_amd.so`` (GPU tensors: data is
moved with the library's copy helpers).  The same class can drive any
library that exports pico's API with host-memory tensors (``device=False``:
data is read and written through the ``float*`` in place), which is how the
tests run one script against the GPU library and against a CPU build of the
same API.  Nothing here computes; every op is one call into the library.
"""
from __future__ import annotations

import ctypes
import os
from contextlib import contextmanager

import numpy as np

from ._lib import AMD_LIB_PATH

c_p = ctypes.c_void_p
c_i64 = ctypes.c_int64
c_f = ctypes.c_float


class PicoTensor(ctypes.Structure):
    """struct PicoTensor (src/tensor.h:11-23)"""


PicoTensor._fields_ = [
    ("shape", ctypes.POINTER(c_i64)),
    ("strides", ctypes.POINTER(c_i64)),
    ("data", c_p),
    ("grad", c_p),
    ("_backward", c_p),
    ("parents", ctypes.POINTER(ctypes.POINTER(PicoTensor))),
    ("numel", c_i64),
    ("backend", ctypes.c_int),
    ("ndim", ctypes.c_uint8),
    ("num_parents", ctypes.c_uint8),
    ("is_persistent", ctypes.c_uint8),
]
TP = ctypes.POINTER(PicoTensor)


class PicoGPTConfig(ctypes.Structure):
    """struct PicoGPTConfig (include/pico_amd.h)"""
    _fields_ = [(n, ctypes.c_int) for n in
                ("vocab", "d_model", "n_layers", "n_heads", "d_ff", "batch", "seq_len")] + \
               [("norm_eps", ctypes.c_float), ("init_std", ctypes.c_float)]


GPT_KEYS = ("vocab", "d_model", "n_layers", "n_heads", "d_ff", "batch", "seq_len")

_SIGS = {
    "pico_init": (None, []),
    "arena_init": (c_p, [ctypes.c_size_t]),
    "arena_reset": (None, [c_p]),
    "arena_destroy": (None, [c_p]),
    "arena_ctx_push": (None, [c_p]),
    "arena_ctx_pop": (None, []),
    "arena_ctx_current": (c_p, []),
    "pico_param": (TP, [ctypes.POINTER(c_i64), ctypes.c_uint8]),
    "pico_create_tensor": (TP, [c_p, ctypes.POINTER(c_i64), ctypes.c_uint8]),
    "pico_tensor_from_scalar": (TP, [c_f]),
    "pico_free": (None, [TP]),
    "pico_transpose_2d": (None, [TP]),
    "pico_rand": (TP, [c_p, ctypes.POINTER(c_i64), ctypes.c_uint8]),
    "pico_backward": (None, [c_p, TP]),
    "pico_add": (TP, [TP, TP]),
    "pico_sub": (TP, [TP, TP]),
    "pico_mul": (TP, [TP, TP]),
    "pico_matmul": (TP, [TP, TP]),
    "pico_tensor_sqrt": (TP, [TP]),
    "pico_tensor_sin": (TP, [TP]),
    "pico_tensor_cos": (TP, [TP]),
    "pico_tensor_tan": (TP, [TP]),
    "pico_tensor_tanh": (TP, [TP]),
    "pico_tensor_log": (TP, [TP]),
    "pico_relu": (TP, [TP]),
    "pico_softmax_xent": (TP, [TP, c_p]),
    "pico_rmsnorm": (TP, [TP, TP, c_f]),
    "pico_swiglu": (TP, [TP, TP]),
    "pico_attention_causal": (TP, [TP, TP, TP, ctypes.c_int, ctypes.c_int]),
    "pico_embedding": (TP, [TP, c_p, c_i64]),
    "pico_nn_linear_init": (c_p, [ctypes.c_int, ctypes.c_int, ctypes.c_bool]),
    "pico_nn_linear_forward": (TP, [c_p, TP]),
    "pico_nn_linear_free": (None, [c_p]),
    "pico_optim_sgd_init": (c_p, [c_f]),
    "pico_optim_sgd_add": (None, [c_p, TP]),
    "pico_optim_sgd_step": (None, [c_p]),
    "pico_optim_sgd_zero_grad": (None, [c_p]),
    "pico_optim_sgd_free": (None, [c_p]),
    "pico_optim_adamw_init": (c_p, [c_f, c_f, c_f, c_f, c_f]),
    "pico_optim_adamw_add": (None, [c_p, TP]),
    "pico_optim_adamw_step": (None, [c_p]),
    "pico_optim_adamw_zero_grad": (None, [c_p]),
    "pico_optim_adamw_free": (None, [c_p]),
}
_GPU_SIGS = {
    "pico_tensor_copy_from_host": (ctypes.c_int, [TP, c_p]),
    "pico_tensor_copy_to_host": (ctypes.c_int, [TP, c_p]),
    "pico_tensor_grad_to_host": (ctypes.c_int, [TP, c_p]),
    "pico_tensor_grad_from_host": (ctypes.c_int, [TP, c_p]),
    "pico_ids_to_device": (c_p, [c_p, c_i64]),
    "pico_ids_update": (ctypes.c_int, [c_p, c_p, c_i64]),
    "pico_graph_begin": (ctypes.c_int, []),
    "pico_graph_end": (c_p, []),
    "pico_graph_launch": (ctypes.c_int, [c_p]),
    "pico_graph_free": (None, [c_p]),
    "pico_argmax": (ctypes.c_int, [TP, c_p]),
    "pico_gpu_synchronize": (ctypes.c_int, []),
    "pico_gpu_last_error": (ctypes.c_char_p, []),
    "pico_gpu_clear_error": (None, []),
    "pico_gpu_fail_next_workspaces": (None, [ctypes.c_int]),
    "pico_gpu_memory": (None, [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]),
    "pico_randn": (TP, [c_p, ctypes.POINTER(c_i64), ctypes.c_uint8]),
    "pico_gpt_init": (c_p, [ctypes.POINTER(PicoGPTConfig), ctypes.c_uint64]),
    "pico_gpt_loss": (TP, [c_p, c_p, c_p]),
    "pico_gpt_num_params": (ctypes.c_int, [c_p]),
    "pico_gpt_param": (TP, [c_p, ctypes.c_int]),
    "pico_gpt_free": (None, [c_p]),
    "pico_gpt_param_name": (ctypes.c_char_p, [c_p, ctypes.c_int]),
    "pico_split_cols": (ctypes.c_int, [TP, ctypes.c_int, ctypes.POINTER(TP)]),
    "pico_matmul_add": (TP, [TP, TP, TP]),
    "pico_swiglu_matmul_add": (TP, [TP, TP, TP, TP]),
    "pico_matmul_gate_up": (TP, [TP, TP]),
    "pico_set_matmul_precision": (ctypes.c_int, [ctypes.c_int]),
    "pico_get_matmul_precision": (ctypes.c_int, []),
    "pico_checkpoint_save": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(TP),
                                            ctypes.POINTER(ctypes.c_char_p), c_p]),
    "pico_checkpoint_load": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, ctypes.POINTER(TP),
                                            ctypes.POINTER(ctypes.c_char_p), c_p]),
}

_amd = None


def amd_lib() -> ctypes.CDLL:
    """libpico_amd.so, loaded once (raises if it has not been built)."""
    global _amd
    if _amd is None:
        from . import _lib

        _lib.hip_lib()  # the launcher library it links against, same runtime as torch
        if not os.path.exists(AMD_LIB_PATH):
            raise RuntimeError(f"pico_amd: {AMD_LIB_PATH} is missing; build it first "
                               "(there is no CPU fallback)")
        _amd = ctypes.CDLL(AMD_LIB_PATH)
    return _amd


def _i64s(xs):
    return (c_i64 * len(xs))(*[int(x) for x in xs])


class PicoError(RuntimeError):
    pass


class Pico:
    """pico's API over one library.  ``device`` says whether tensor data is
    device memory (moved with the copy helpers) or host memory."""

    def __init__(self, lib=None, device=True):
        self.lib = lib if lib is not None else amd_lib()
        self.device = device
        for name, (res, args) in _SIGS.items():
            f = getattr(self.lib, name)
            f.restype, f.argtypes = res, args
        if device:
            for name, (res, args) in _GPU_SIGS.items():
                f = getattr(self.lib, name)
                f.restype, f.argtypes = res, args
        self.lib.pico_init()
        self._keep = []  # host arrays whose addresses the library may still hold

    # ---------------------------------------------------------------- arena
    @contextmanager
    def arena(self, nbytes=1 << 26):
        a = self.lib.arena_init(nbytes)
        if not a:
            raise PicoError("arena_init failed")
        self.lib.arena_ctx_push(a)
        try:
            yield a
        finally:
            self.lib.arena_ctx_pop()
            self.lib.arena_destroy(a)
            self._keep.clear()

    def reset(self, arena):
        self.lib.arena_reset(arena)
        self._keep.clear()

    # -------------------------------------------------------------- tensors
    def _check(self, t, what):
        if not t:
            msg = ""
            if self.device:
                msg = self.lib.pico_gpu_last_error().decode(errors="replace")
            raise PicoError(f"{what} returned NULL {msg}".strip())
        return t

    def param(self, shape, values=None):
        t = self._check(self.lib.pico_param(_i64s(shape), len(shape)), "pico_param")
        if values is not None:
            self.set(t, values)
        return t

    def tensor(self, shape, values=None):
        a = self.lib.arena_ctx_current()
        t = self._check(self.lib.pico_create_tensor(a, _i64s(shape), len(shape)),
                        "pico_create_tensor")
        if values is not None:
            self.set(t, values)
        return t

    def scalar(self, v):
        return self._check(self.lib.pico_tensor_from_scalar(v), "pico_tensor_from_scalar")

    def free(self, t):
        self.lib.pico_free(t)

    def shape(self, t):
        return tuple(t.contents.shape[i] for i in range(t.contents.ndim))

    def strides(self, t):
        return tuple(t.contents.strides[i] for i in range(t.contents.ndim))

    def set(self, t, values):
        v = np.ascontiguousarray(values, dtype=np.float32).ravel()
        n = t.contents.numel
        if v.size != n:
            raise ValueError(f"expected {n} values, got {v.size}")
        if self.device:
            if self.lib.pico_tensor_copy_from_host(t, v.ctypes.data_as(c_p)):
                raise PicoError("copy to device failed")
        else:
            ctypes.memmove(t.contents.data, v.ctypes.data, 4 * n)

    def set_grad(self, t, values):
        v = np.ascontiguousarray(values, dtype=np.float32).ravel()
        if self.device:
            if self.lib.pico_tensor_grad_from_host(t, v.ctypes.data_as(c_p)):
                raise PicoError("grad copy to device failed")
        else:
            ctypes.memmove(t.contents.grad, v.ctypes.data, 4 * t.contents.numel)

    def _read(self, t, grad):
        n = t.contents.numel
        out = np.empty(n, np.float32)
        if self.device:
            fn = self.lib.pico_tensor_grad_to_host if grad else self.lib.pico_tensor_copy_to_host
            if fn(t, out.ctypes.data_as(c_p)):
                raise PicoError("copy to host failed")
        else:
            ctypes.memmove(out.ctypes.data, t.contents.grad if grad else t.contents.data, 4 * n)
        return out

    def data(self, t):
        """the tensor's storage (numel floats, storage order)"""
        return self._read(t, False)

    def grad(self, t):
        return self._read(t, True)

    def value(self, t):
        """logical contents in row-major order of the tensor's shape"""
        return self._logical(self.data(t), t)

    def grad_value(self, t):
        return self._logical(self.grad(t), t)

    def _logical(self, buf, t):
        shape, strides = self.shape(t), self.strides(t)
        return np.lib.stride_tricks.as_strided(
            buf, shape=shape, strides=tuple(4 * s for s in strides)).copy()

    def ids(self, arr):
        """an int32 array the library may read until the arena is reset"""
        a = np.ascontiguousarray(arr, dtype=np.int32)
        self._keep.append(a)
        return a.ctypes.data_as(c_p)

    def memory(self):
        """(bytes of device memory the library holds, its peak)"""
        a, b = ctypes.c_size_t(0), ctypes.c_size_t(0)
        self.lib.pico_gpu_memory(ctypes.byref(a), ctypes.byref(b))
        return a.value, b.value

    def sync(self):
        if self.device:
            self.lib.pico_gpu_synchronize()

    # ------------------------------------------------------------------ ops
    def __getattr__(self, name):
        # pico_<op> passthrough with NULL checking: P.add(a, b) -> pico_add(a, b)
        for cand in ("pico_" + name, "pico_tensor_" + name):
            if cand in _SIGS or cand in _GPU_SIGS:
                fn = getattr(self.lib, cand)

                def call(*args, _fn=fn, _n=cand):
                    r = _fn(*args)
                    if _fn.restype is TP:
                        self._check(r, _n)
                    return r

                return call
        raise AttributeError(name)

    def split_cols(self, t, n):
        """pico_split_cols: n column-block views of t [M, n*C]"""
        outs = (TP * n)()
        if self.lib.pico_split_cols(t, n, outs):
            raise PicoError("pico_split_cols failed")
        return list(outs)

    def xent(self, logits, labels):
        return self._check(self.lib.pico_softmax_xent(logits, self.ids(labels)),
                           "pico_softmax_xent")

    def embedding(self, table, ids):
        a = np.ascontiguousarray(ids, dtype=np.int32)
        return self._check(self.lib.pico_embedding(table, self.ids(a), a.size), "pico_embedding")

    # ------------------------------------------------------------ the model
    def gpt_init(self, cfg, seed, norm_eps=1e-6, init_std=0.02):
        c = PicoGPTConfig(*[int(cfg[k]) for k in GPT_KEYS], norm_eps, init_std)
        m = self.lib.pico_gpt_init(ctypes.byref(c), seed)
        if not m:
            raise PicoError("pico_gpt_init failed " +
                            self.lib.pico_gpu_last_error().decode(errors="replace"))
        return m

    def gpt_params(self, model):
        return [self.lib.pico_gpt_param(model, i)
                for i in range(self.lib.pico_gpt_num_params(model))]

    def gpt_loss(self, model, tokens, targets):
        """tokens / targets: int32 numpy arrays (staged per call) or device pointers"""
        tp = tokens if isinstance(tokens, int) else self.ids(tokens)
        gp = targets if isinstance(targets, int) else self.ids(targets)
        return self._check(self.lib.pico_gpt_loss(model, tp, gp), "pico_gpt_loss")

    def backward(self, loss):
        if self.device:
            self.lib.pico_gpu_clear_error()
        self.lib.pico_backward(self.lib.arena_ctx_current(), loss)
        if self.device:
            err = self.lib.pico_gpu_last_error().decode(errors="replace")
            if err:
                self.lib.pico_gpu_clear_error()
                raise PicoError(err)
