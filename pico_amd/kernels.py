"""Thin Python bindings of the pk_* C-ABI over torch device tensors.

torch supplies device memory and the current stream; every computation runs
in the hand-written HIP kernels of ``libpico_hip.so``.  Each function checks
shapes on the host before launching (so a kernel never sees a shape its grid
does not cover) and raises ``PkError`` on a non-zero status.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import check, hip_lib

ACCUM = 1
ACCUM2 = 2
BINARY_OPS = {"add": 0, "sub": 1, "mul": 2}
UNARY_OPS = {"sqrt": 0, "sin": 1, "cos": 2, "tan": 3, "tanh": 4, "log": 5}


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _f32(*ts):
    for t in ts:
        if t is not None:
            if t.dtype != torch.float32 or not t.is_cuda:
                raise TypeError("expected a float32 CUDA tensor")


def _rowmajor(t, name):
    if t.dim() == 2 and t.numel() == 0:
        return max(1, t.shape[1])
    if t.dim() != 2 or (t.shape[1] > 1 and t.stride(1) != 1):
        raise ValueError(f"{name} must be a 2-D tensor with unit column stride")
    return max(t.stride(0), t.shape[1])


def gemm(ta, tb, A, B, C, alpha=1.0, beta=0.0):
    """C = alpha * op(A) @ op(B) + beta * C  (op = transpose for 'T')."""
    _f32(A, B, C)
    lda, ldb, ldc = _rowmajor(A, "A"), _rowmajor(B, "B"), _rowmajor(C, "C")
    M = A.shape[1] if ta == "T" else A.shape[0]
    K = A.shape[0] if ta == "T" else A.shape[1]
    Kb = B.shape[1] if tb == "T" else B.shape[0]
    N = B.shape[0] if tb == "T" else B.shape[1]
    if K != Kb or tuple(C.shape) != (M, N):
        raise ValueError(f"gemm shape mismatch: op(A) {M}x{K}, op(B) {Kb}x{N}, C {tuple(C.shape)}")
    check("pk_gemm_f32", hip_lib().pk_gemm_f32(
        ta.encode(), tb.encode(), M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C), ldc,
        _stream()))
    return C


def gemm_bf16x3(ta, tb, A, B, C, alpha=1.0, beta=0.0, ws=None):
    """gemm as three bf16 products per fp32 one (pk_gemm_bf16x3_f32)"""
    return gemm_bf16(ta, tb, A, B, C, alpha, beta, ws, split=True)


def gemm_fp8(ta, tb, A, B, C, alpha=1.0, beta=0.0, ws=None):
    """gemm with e4m3 multiplies and fp32 accumulation (pk_gemm_fp8_f32)"""
    return gemm_bf16(ta, tb, A, B, C, alpha, beta, ws, _name="pk_gemm_fp8_f32")


def fp8_scales(A, B, scales):
    """scales[0], scales[1] = largest powers of two keeping A, B within e4m3
    (pk_fp8_scales_f32); A, B 2-D float32 tensors as stored"""
    _f32(A, B, scales)
    lda, ldb = _rowmajor(A, "A"), _rowmajor(B, "B")
    check("pk_fp8_scales_f32", hip_lib().pk_fp8_scales_f32(
        A.shape[0], A.shape[1], _ptr(A), lda, B.shape[0], B.shape[1], _ptr(B), ldb, _ptr(scales),
        _stream()))
    return scales


def fp8_quantized_shape(R, K):
    """(rows, row stride in bytes) of the buffer pk_fp8_quantize_f32 fills"""
    ld = ctypes.c_int64(0)
    nbytes = int(hip_lib().pk_fp8_quantized_bytes(R, K, ctypes.byref(ld)))
    return (nbytes // ld.value if ld.value else 0), ld.value


def fp8_quantize(X, trans, scale, out=None):
    """e4m3(scale * op(X)) as a zero-padded uint8 [rows, ld] tensor: op(X) =
    X (trans False) or X^T; scale a one-element float32 device tensor (or a
    view of pk_fp8_scales_f32's output)"""
    _f32(X, scale)
    ldx = _rowmajor(X, "X")
    R, Kd = (X.shape[1], X.shape[0]) if trans else (X.shape[0], X.shape[1])
    rows, ld = fp8_quantized_shape(R, Kd)
    if out is None:
        out = torch.empty((rows, ld), dtype=torch.uint8, device=X.device)
    if out.dtype != torch.uint8 or out.dim() != 2 or out.shape[0] < rows or out.shape[1] < ld \
            or not out.is_contiguous():
        raise ValueError(f"fp8_quantize: out must be contiguous uint8 of at least {rows}x{ld}")
    check("pk_fp8_quantize_f32", hip_lib().pk_fp8_quantize_f32(
        R, Kd, _ptr(X), ldx, int(bool(trans)), _ptr(scale), _ptr(out), out.stride(0), _stream()))
    return out


def gemm_fp8q(M, N, Kd, A8, B8, scales, C, alpha=1.0, beta=0.0):
    """C = alpha / (scales[0] * scales[1]) * A8 . B8^T (+ beta C), A8 [M, K] and
    B8 [N, K] as fp8_quantize writes them (pk_gemm_fp8q_f32)"""
    _f32(C, scales)
    ldc = _rowmajor(C, "C")
    if tuple(C.shape) != (M, N):
        raise ValueError(f"gemm_fp8q: C {tuple(C.shape)} is not {M}x{N}")
    for name, Q, R in (("A8", A8, M), ("B8", B8, N)):
        rows, ld = fp8_quantized_shape(R, Kd)
        if Q.dtype != torch.uint8 or Q.dim() != 2 or Q.shape[0] < rows or Q.shape[1] < ld:
            raise ValueError(f"gemm_fp8q: {name} must be uint8 of at least {rows}x{ld}")
    check("pk_gemm_fp8q_f32", hip_lib().pk_gemm_fp8q_f32(
        M, N, Kd, alpha, _ptr(A8), A8.stride(0), _ptr(B8), B8.stride(0), _ptr(scales), beta,
        _ptr(C), ldc, _stream()))
    return C


def mx8_bytes(R, Kd):
    """bytes of an MX8 matrix of R rows of Kd values (pk_mx8_bytes)"""
    return int(hip_lib().pk_mx8_bytes(R, Kd))


def bf16q_bytes(R, Kd):
    """bytes of a bf16 operand matrix of R rows of Kd values (pk_bf16q_bytes)"""
    return int(hip_lib().pk_bf16q_bytes(R, Kd))


def bf16x3q_bytes(R, Kd):
    """bytes of a split-bf16 operand matrix of R rows of Kd values (pk_bf16x3q_bytes)"""
    return int(hip_lib().pk_bf16x3q_bytes(R, Kd))


# the narrow-operand formats: (bytes, cast, dual cast, product, product with workspace)
_NARROW = {"mx8": (mx8_bytes, "pk_mx8_quantize_f32", "pk_mx8_quantize2_f32", "pk_gemm_mx8_f32",
                   "pk_gemm_mx8_ex_f32"),
           "bf16q": (bf16q_bytes, "pk_bf16q_quantize_f32", "pk_bf16q_quantize2_f32", "pk_gemm_bf16q_f32",
                     "pk_gemm_bf16q_ex_f32"),
           "bf16x3q": (bf16x3q_bytes, "pk_bf16x3q_quantize_f32", None, "pk_gemm_bf16x3q_f32",
                       "pk_gemm_bf16x3q_ex_f32")}


def _narrow_cast(fmt, X, trans, out):
    nbytes_fn, cast = _NARROW[fmt][0], _NARROW[fmt][1]
    _f32(X)
    ldx = _rowmajor(X, "X")
    R, Kd = (X.shape[1], X.shape[0]) if trans else (X.shape[0], X.shape[1])
    nbytes = nbytes_fn(R, Kd)
    if out is None:
        out = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=X.device)
    if out.dtype != torch.uint8 or out.numel() < nbytes or not out.is_contiguous():
        raise ValueError(f"{cast}: out must be contiguous uint8 of at least {nbytes} bytes")
    check(cast, getattr(hip_lib(), cast)(R, Kd, _ptr(X), ldx, int(bool(trans)), _ptr(out), _stream()))
    return out


def _narrow_cast2(fmt, X):
    nbytes_fn, cast2 = _NARROW[fmt][0], _NARROW[fmt][2]
    _f32(X)
    ldx = _rowmajor(X, "X")
    M, N = X.shape
    QR = torch.empty(max(nbytes_fn(M, N), 1), dtype=torch.uint8, device=X.device)
    QT = torch.empty(max(nbytes_fn(N, M), 1), dtype=torch.uint8, device=X.device)
    check(cast2, getattr(hip_lib(), cast2)(M, N, _ptr(X), ldx, _ptr(QR), _ptr(QT), _stream()))
    return QR, QT


def _narrow_gemm(fmt, M, N, Kd, A8, B8, C, alpha, beta, X, ws):
    nbytes_fn, name, name_ex = _NARROW[fmt][0], _NARROW[fmt][3], _NARROW[fmt][4]
    _f32(C, X)
    ldc = _rowmajor(C, "C")
    if tuple(C.shape) != (M, N):
        raise ValueError(f"{name}: C {tuple(C.shape)} is not {M}x{N}")
    for what, Q, R in (("A", A8, M), ("B", B8, N)):
        if Q.dtype != torch.uint8 or Q.numel() < nbytes_fn(R, Kd):
            raise ValueError(f"{name}: {what} must be uint8 of at least {nbytes_fn(R, Kd)} bytes")
    ldx = 0
    if X is None and beta != 0.0:
        X = C
    if X is not None:
        if X.dim() == 1:
            if X.shape[0] != N:
                raise ValueError(f"{name}: a row X must have N values")
        else:
            if tuple(X.shape) != (M, N):
                raise ValueError(f"{name}: X must be [M, N] or [N]")
            ldx = _rowmajor(X, "X")
    if ws is None:
        check(name, getattr(hip_lib(), name)(
            M, N, Kd, alpha, _ptr(A8), _ptr(B8), beta, _ptr(X), ldx, _ptr(C), ldc, _stream()))
    else:
        check(name_ex, getattr(hip_lib(), name_ex)(
            M, N, Kd, alpha, _ptr(A8), _ptr(B8), beta, _ptr(X), ldx, _ptr(C), ldc, _ptr(ws),
            ws.numel() * ws.element_size(), _stream()))
    return C


def mx8_quantize(X, trans, out=None):
    """op(X) (X, or X^T when trans) as an MX8 matrix: e4m3 values with an E8M0
    scale per 32 of a row (pk_mx8_quantize_f32); a uint8 tensor"""
    return _narrow_cast("mx8", X, trans, out)


def mx8_quantize2(X):
    """(X as an MX8 [M, N], X^T as an MX8 [N, M]) from one read of X
    (pk_mx8_quantize2_f32)"""
    return _narrow_cast2("mx8", X)


def bf16q_quantize(X, trans, out=None):
    """op(X) as a bf16 operand matrix (pk_bf16q_quantize_f32); a uint8 tensor"""
    return _narrow_cast("bf16q", X, trans, out)


def bf16q_quantize2(X):
    """(X as a bf16 [M, N], X^T as a bf16 [N, M]) from one read of X
    (pk_bf16q_quantize2_f32)"""
    return _narrow_cast2("bf16q", X)


def bf16x3q_quantize(X, trans, out=None):
    """op(X) as a split-bf16 operand matrix (hi and lo bf16 parts of every
    value, pk_bf16x3q_quantize_f32); a uint8 tensor"""
    return _narrow_cast("bf16x3q", X, trans, out)


def mx8_plan(M, N, Kd):
    """(tile rows, tile columns, K splits) pk_gemm_mx8_f32 picks with a workspace"""
    tm, tn, sp = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    check("pk_gemm_mx8_plan", hip_lib().pk_gemm_mx8_plan(M, N, Kd, ctypes.byref(tm), ctypes.byref(tn),
                                                          ctypes.byref(sp)))
    return tm.value, tn.value, sp.value


def mx8_workspace(M, N, Kd):
    """workspace bytes of the K split pk_gemm_mx8_f32 picks (0: none)"""
    return int(hip_lib().pk_gemm_mx8_workspace(M, N, Kd))


def bf16q_workspace(M, N, Kd):
    """workspace bytes of the K split pk_gemm_bf16q_f32 picks (0: none)"""
    return int(hip_lib().pk_gemm_bf16q_workspace(M, N, Kd))


def gemm_mx8(M, N, Kd, A8, B8, C, alpha=1.0, beta=0.0, X=None, ws=None):
    """C = alpha * A8 . B8^T + beta * X (pk_gemm_mx8_f32): A8 [M, Kd] and B8
    [N, Kd] MX8 matrices as mx8_quantize writes them; X a [M, N] tensor, a
    [N] row added to every row, or C itself; ws: workspace for a K split
    (pk_gemm_mx8_ex_f32)"""
    return _narrow_gemm("mx8", M, N, Kd, A8, B8, C, alpha, beta, X, ws)


def gemm_bf16q(M, N, Kd, A16, B16, C, alpha=1.0, beta=0.0, X=None, ws=None):
    """gemm_mx8 for bf16 operand matrices (pk_gemm_bf16q_f32 / _ex_f32)"""
    return _narrow_gemm("bf16q", M, N, Kd, A16, B16, C, alpha, beta, X, ws)


def bf16x3q_workspace(M, N, Kd):
    """workspace bytes of the K split pk_gemm_bf16x3q_f32 picks (0: none)"""
    return int(hip_lib().pk_gemm_bf16x3q_workspace(M, N, Kd))


def gemm_bf16x3q(M, N, Kd, A, B, C, alpha=1.0, beta=0.0, X=None, ws=None):
    """gemm_mx8 for split-bf16 operand matrices: three bf16 products per fp32
    one (pk_gemm_bf16x3q_f32 / _ex_f32)"""
    return _narrow_gemm("bf16x3q", M, N, Kd, A, B, C, alpha, beta, X, ws)


def gemm_bf16(ta, tb, A, B, C, alpha=1.0, beta=0.0, ws=None, split=False, _name=None):
    """gemm with bf16 multiplies and fp32 accumulation (fp32 tensors in and out);
    ws: optional workspace for a K split (as gemm_ex); split: hi/lo operands,
    three products (pk_gemm_bf16x3_f32)"""
    _f32(A, B, C)
    lda, ldb, ldc = _rowmajor(A, "A"), _rowmajor(B, "B"), _rowmajor(C, "C")
    M = A.shape[1] if ta == "T" else A.shape[0]
    K = A.shape[0] if ta == "T" else A.shape[1]
    Kb = B.shape[1] if tb == "T" else B.shape[0]
    N = B.shape[0] if tb == "T" else B.shape[1]
    if K != Kb or tuple(C.shape) != (M, N):
        raise ValueError(f"gemm shape mismatch: op(A) {M}x{K}, op(B) {Kb}x{N}, C {tuple(C.shape)}")
    name = _name or ("pk_gemm_bf16x3_f32" if split else "pk_gemm_bf16_f32")
    if ws is None:
        check(name, getattr(hip_lib(), name)(
            ta.encode(), tb.encode(), M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C),
            ldc, _stream()))
    else:
        name = name.replace("pk_gemm_", "pk_gemm_ex_")
        check(name, getattr(hip_lib(), name)(
            ta.encode(), tb.encode(), M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C),
            ldc, _ptr(ws), ws.numel() * ws.element_size(), _stream()))
    return C


def gemm_workspace(M, N, K):
    return int(hip_lib().pk_gemm_workspace_f32(M, N, K))


def gemm_ex(ta, tb, A, B, C, alpha=1.0, beta=0.0, ws=None):
    """gemm with a workspace: K is split when C has too few tiles (ws=None
    allocates the size pk_gemm_workspace_f32 asks for)."""
    _f32(A, B, C)
    lda, ldb, ldc = _rowmajor(A, "A"), _rowmajor(B, "B"), _rowmajor(C, "C")
    M = A.shape[1] if ta == "T" else A.shape[0]
    K = A.shape[0] if ta == "T" else A.shape[1]
    N = B.shape[0] if tb == "T" else B.shape[1]
    if ws is None:
        need = gemm_workspace(M, N, K)
        ws = torch.empty(max(1, need // 4), device=C.device, dtype=torch.float32)
    check("pk_gemm_ex_f32", hip_lib().pk_gemm_ex_f32(
        ta.encode(), tb.encode(), M, N, K, alpha, _ptr(A), lda, _ptr(B), ldb, beta, _ptr(C), ldc,
        _ptr(ws), ws.numel() * 4, _stream()))
    return C


def gemm_batched(ta, tb, M, N, K, alpha, A, lda, sAo, sAi, B, ldb, sBo, sBi, beta, C, ldc, sCo,
                 sCi, batch, inner, causal=0):
    """Raw batched GEMM on flat tensors (strides in elements)."""
    _f32(A, B, C)
    check("pk_gemm_batched_f32", hip_lib().pk_gemm_batched_f32(
        ta.encode(), tb.encode(), M, N, K, alpha, _ptr(A), lda, sAo, sAi, _ptr(B), ldb, sBo, sBi,
        beta, _ptr(C), ldc, sCo, sCi, batch, inner, causal, _stream()))
    return C


def _bcast_strides(shape, out_shape):
    """Strides of a contiguous `shape` mapped onto `out_shape` (0 on broadcast dims)."""
    nd = len(out_shape)
    st = [0] * nd
    s = 1
    for d in range(len(shape) - 1, -1, -1):
        od = d + nd - len(shape)
        st[od] = 0 if shape[d] == 1 else s
        s *= shape[d]
    return st


def _i64s(xs):
    return (ctypes.c_int64 * len(xs))(*xs)


def binary(op, a, b, out=None):
    _f32(a, b)
    out_shape = list(torch.broadcast_shapes(a.shape, b.shape))
    if out is None:
        out = torch.empty(out_shape, device=a.device, dtype=torch.float32)
    nd = max(1, len(out_shape))
    osh = out_shape or [1]
    sa = _bcast_strides(list(a.shape) or [1], osh)
    sb = _bcast_strides(list(b.shape) or [1], osh)
    check("pk_binary_f32", hip_lib().pk_binary_f32(
        BINARY_OPS[op], nd, _i64s(osh), _i64s(sa), _i64s(sb), _ptr(a.contiguous()),
        _ptr(b.contiguous()), _ptr(out), _stream()))
    return out


def binary_bwd(op, which, out_shape, x_shape, other_shape, gout, other, gx, accumulate=False):
    osh = list(out_shape) or [1]
    sx = _bcast_strides(list(x_shape) or [1], osh)
    so = _bcast_strides(list(other_shape) or [1], osh)
    xn = 1
    for s in x_shape:
        xn *= s
    check("pk_binary_bwd_f32", hip_lib().pk_binary_bwd_f32(
        BINARY_OPS[op], which, len(osh), _i64s(osh), _i64s(sx), _i64s(so), xn, _ptr(gout),
        _ptr(other), _ptr(gx), ACCUM if accumulate else 0, _stream()))
    return gx


def unary(op, x, y):
    check("pk_unary_f32", hip_lib().pk_unary_f32(UNARY_OPS[op], x.numel(), _ptr(x), _ptr(y),
                                                  _stream()))
    return y


def unary_bwd(op, x, y, gy, gx, accumulate=True):
    check("pk_unary_bwd_f32", hip_lib().pk_unary_bwd_f32(
        UNARY_OPS[op], x.numel(), _ptr(x), _ptr(y), _ptr(gy), _ptr(gx),
        ACCUM if accumulate else 0, _stream()))
    return gx


def relu(x, y):
    check("pk_relu_f32", hip_lib().pk_relu_f32(x.numel(), _ptr(x), _ptr(y), _stream()))
    return y


def relu_bwd(y, gy, gx, accumulate=True):
    check("pk_relu_bwd_f32", hip_lib().pk_relu_bwd_f32(
        y.numel(), _ptr(y), _ptr(gy), _ptr(gx), ACCUM if accumulate else 0, _stream()))
    return gx


def fill(x, value):
    check("pk_fill_f32", hip_lib().pk_fill_f32(x.numel(), value, _ptr(x), _stream()))
    return x


def axpy(alpha, x, y, alpha_dev=None, accumulate=True):
    check("pk_axpy_f32", hip_lib().pk_axpy_f32(x.numel(), alpha, _ptr(alpha_dev), _ptr(x),
                                                _ptr(y), ACCUM if accumulate else 0, _stream()))
    return y


def reduce_sum(x, out, scale=1.0, accumulate=False):
    check("pk_reduce_sum_f32", hip_lib().pk_reduce_sum_f32(
        x.numel(), _ptr(x), scale, _ptr(out), ACCUM if accumulate else 0, _stream()))
    return out


def sgd(p, g, lr):
    check("pk_sgd_f32", hip_lib().pk_sgd_f32(p.numel(), lr, _ptr(p), _ptr(g), _stream()))
    return p


def adamw(p, g, m, v, lr, beta1, beta2, eps, wd, step):
    check("pk_adamw_f32", hip_lib().pk_adamw_f32(p.numel(), lr, beta1, beta2, eps, wd, step,
                                                  _ptr(p), _ptr(g), _ptr(m), _ptr(v), _stream()))
    return p


class PkAdamwChunk(ctypes.Structure):
    """struct PkAdamwChunk (include/pico_hip.h)"""
    _fields_ = [("p", ctypes.c_void_p), ("g", ctypes.c_void_p), ("m", ctypes.c_void_p),
                ("v", ctypes.c_void_p), ("n", ctypes.c_int64)]


ADAMW_CHUNK = 65536


def adamw_multi(groups, lr, beta1, beta2, eps, wd, state):
    """One multi-tensor AdamW step over groups of (p, g or None, m, v).  state:
    a device int32 tensor of >= 3 elements -- the step count (advanced here)
    and the two bias corrections, as floats, in elements 1 and 2.  Returns the
    device chunk table, which must stay alive until the launch has run."""
    _f32(*[t for grp in groups for t in grp])
    if state.dtype != torch.int32 or state.numel() < 3 or not state.is_cuda:
        raise ValueError("state must be a device int32 tensor of >= 3 elements")
    chunks = []
    for p, g, m, v in groups:
        n = p.numel()
        if any(t is not None and t.numel() != n for t in (g, m, v)):
            raise ValueError("p, g, m, v must have the same size")
        for off in range(0, n, ADAMW_CHUNK):
            chunks.append(PkAdamwChunk(p.data_ptr() + 4 * off,
                                       None if g is None else g.data_ptr() + 4 * off,
                                       m.data_ptr() + 4 * off, v.data_ptr() + 4 * off,
                                       min(ADAMW_CHUNK, n - off)))
    arr = (PkAdamwChunk * max(1, len(chunks)))(*chunks)
    table = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8).to(state.device)
    coef = ctypes.c_void_p(state.data_ptr() + 4)
    check("pk_adamw_prep_f32", hip_lib().pk_adamw_prep_f32(_ptr(state), lr, beta1, beta2, coef,
                                                            _stream()))
    check("pk_adamw_multi_f32", hip_lib().pk_adamw_multi_f32(
        len(chunks), _ptr(table), lr, beta1, beta2, eps, wd, coef, _stream()))
    return table


def xent_fwd_bwd(logits, labels, loss_rows=None, dlogits=None, scale=1.0, accumulate=False,
                 scale_dev=None):
    R, V = logits.shape
    if labels.dtype != torch.int32 or labels.numel() != R:
        raise ValueError("labels must be int32 with one entry per row")
    check("pk_xent_fwd_bwd_f32", hip_lib().pk_xent_fwd_bwd_f32(
        R, V, _ptr(logits), _rowmajor(logits, "logits"), _ptr(labels), _ptr(loss_rows),
        _ptr(dlogits), V if dlogits is None else _rowmajor(dlogits, "dlogits"), scale,
        _ptr(scale_dev), ACCUM if accumulate else 0, _stream()))


def xent_mean(logits, labels, out, loss_rows=None, dlogits=None, scale=1.0, mean_scale=1.0,
              accumulate=False, accumulate_out=False):
    """xent_fwd_bwd plus out[0] (+)= mean_scale * sum(loss rows) (pk_xent_mean_f32)"""
    R, V = logits.shape
    if labels.dtype != torch.int32 or labels.numel() != R:
        raise ValueError("labels must be int32 with one entry per row")
    flags = (ACCUM if accumulate else 0) | (2 if accumulate_out else 0)
    check("pk_xent_mean_f32", hip_lib().pk_xent_mean_f32(
        R, V, _ptr(logits), _rowmajor(logits, "logits"), _ptr(labels), _ptr(loss_rows),
        _ptr(dlogits), V if dlogits is None else _rowmajor(dlogits, "dlogits"), scale, flags,
        mean_scale, _ptr(out), _stream()))
    return out


def argmax(x, idx):
    R, V = x.shape
    check("pk_argmax_f32", hip_lib().pk_argmax_f32(R, V, _ptr(x), _rowmajor(x, "x"), _ptr(idx),
                                                    _stream()))
    return idx


def rmsnorm_fwd(x, g, y, rstd, eps):
    R, C = x.shape
    if g.numel() != C or y.shape != x.shape or (rstd is not None and rstd.numel() != R):
        raise ValueError("rmsnorm_fwd shape mismatch")
    check("pk_rmsnorm_fwd_f32", hip_lib().pk_rmsnorm_fwd_f32(R, C, eps, _ptr(x), _ptr(g), _ptr(y),
                                                              _ptr(rstd), _stream()))


def rmsnorm_bwd_workspace(R, C):
    return int(hip_lib().pk_rmsnorm_bwd_workspace(R, C))


RMS_KEEP_PARTIALS = 8


def rmsnorm_bwd(x, g, rstd, dy, dx, dg, ws=None, accum_dx=False, accum_dg=False, dx_in=None,
                keep_partials=False):
    """dx_in: the accumulated term of dx read from another buffer
    (pk_rmsnorm_bwd_into_f32; accum_dx is then ignored).  keep_partials (with
    dg None): leave dg's partial sums in ws for rmsnorm_dg_reduce."""
    R, C = x.shape
    need = rmsnorm_bwd_workspace(R, C)
    if ws is None and (dg is not None or keep_partials):
        ws = torch.empty(max(1, need // 4), device=x.device, dtype=torch.float32)
    wsb = 0 if ws is None else ws.numel() * 4
    if dx_in is not None or keep_partials:
        flags = (ACCUM2 if accum_dg else 0) | (RMS_KEEP_PARTIALS if keep_partials else 0)
        src = dx_in if dx_in is not None else (dx if accum_dx else None)
        check("pk_rmsnorm_bwd_into_f32", hip_lib().pk_rmsnorm_bwd_into_f32(
            R, C, _ptr(x), _ptr(g), _ptr(rstd), _ptr(dy), _ptr(src), _ptr(dx), _ptr(dg),
            flags, _ptr(ws), wsb, _stream()))
        return ws
    flags = (ACCUM if accum_dx else 0) | (ACCUM2 if accum_dg else 0)
    check("pk_rmsnorm_bwd_f32", hip_lib().pk_rmsnorm_bwd_f32(
        R, C, _ptr(x), _ptr(g), _ptr(rstd), _ptr(dy), _ptr(dx), _ptr(dg), flags, _ptr(ws), wsb,
        _stream()))


def rmsnorm_dg_reduce(R, C, ws, dg, accum=False):
    check("pk_rmsnorm_dg_reduce_f32", hip_lib().pk_rmsnorm_dg_reduce_f32(
        R, C, _ptr(ws), ws.numel() * 4, _ptr(dg), ACCUM if accum else 0, _stream()))


def swiglu_fwd(a, u, h):
    R, F = a.shape
    check("pk_swiglu_fwd_f32", hip_lib().pk_swiglu_fwd_f32(
        R, F, _ptr(a), _rowmajor(a, "a"), _ptr(u), _rowmajor(u, "u"), _ptr(h), _rowmajor(h, "h"),
        _stream()))
    return h


def swiglu_bwd(a, u, dh, da, du, accum_da=False, accum_du=False):
    R, F = a.shape
    ldd = _rowmajor(da if da is not None else du, "da")
    flags = (ACCUM if accum_da else 0) | (ACCUM2 if accum_du else 0)
    check("pk_swiglu_bwd_f32", hip_lib().pk_swiglu_bwd_f32(
        R, F, _ptr(a), _rowmajor(a, "a"), _ptr(u), _rowmajor(u, "u"), _ptr(dh), _rowmajor(dh, "dh"),
        _ptr(da), _ptr(du), ldd, flags, _stream()))


def _attn_layout(B, H, q, k, v, o, *grads):
    """(T, hd, ld): q, k, v and their grads [B*T, H*hd] with unit column stride
    and one shared row stride ld >= H*hd (column blocks of a fused projection
    allowed); o (and dout) contiguous."""
    _f32(q, k, v, o, *grads)
    BT, D = q.shape
    T, hd = BT // B, D // H
    ld = q.stride(0) if BT > 1 else D
    if B * T != BT or H * hd != D or o.shape != q.shape:
        raise ValueError("attention shape mismatch")
    for t in (q, k, v) + tuple(grads):
        if t.shape != q.shape or (BT > 1 and t.stride(0) != ld) or (D > 1 and t.stride(1) != 1):
            raise ValueError("q, k, v and their gradients need one row stride and unit columns")
    if ld < D or not o.is_contiguous():
        raise ValueError("attention: row stride below H*hd, or o not contiguous")
    return T, hd, ld


def attn_fwd(B, H, q, k, v, o, lse, P, scale=None):
    T, hd, ld = _attn_layout(B, H, q, k, v, o)
    if P.numel() < B * H * T * T or lse.numel() < B * H * T:
        raise ValueError("attention shape mismatch")
    scale = hd ** -0.5 if scale is None else scale
    check("pk_attn_causal_fwd_f32", hip_lib().pk_attn_causal_fwd_f32(
        B, H, T, hd, ld, scale, _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), _ptr(P),
        _stream()))


def attn_bwd(B, H, q, k, v, P, dout, dq, dk, dv, dP_ws, accumulate=False, scale=None):
    T, hd, ld = _attn_layout(B, H, q, k, v, dout, dq, dk, dv)
    if dP_ws.numel() < B * H * T * T:
        raise ValueError("attention backward workspace too small")
    scale = hd ** -0.5 if scale is None else scale
    check("pk_attn_causal_bwd_f32", hip_lib().pk_attn_causal_bwd_f32(
        B, H, T, hd, ld, scale, _ptr(q), _ptr(k), _ptr(v), _ptr(P), _ptr(dout), _ptr(dq),
        _ptr(dk), _ptr(dv), _ptr(dP_ws), 7 if accumulate else 0, _stream()))


def flash_supported(T, hd):
    return bool(hip_lib().pk_flash_attn_supported(T, hd))


def flash_fwd(B, H, q, k, v, o, lse, scale=None, bf16=False, fp8_amax=None, bf16x3=False):
    """Fused causal attention; bf16=True rounds the matrix-product operands to
    bf16 (pk_flash_attn_fwd_bf16_f32); bf16x3=True takes each product as three
    bf16 ones of split operands (pk_flash_attn_fwd_bf16x3_f32); fp8_amax (4
    float32 on the device) runs the e4m3 products (pk_flash_attn_fwd_fp8_f32)
    and receives max|q|, max|k|, max|v| for the backward."""
    T, hd, ld = _attn_layout(B, H, q, k, v, o)
    if lse.numel() < B * H * T:
        raise ValueError("attention shape mismatch")
    scale = hd ** -0.5 if scale is None else scale
    if fp8_amax is not None:
        _f32(fp8_amax)
        check("pk_flash_attn_fwd_fp8_f32", hip_lib().pk_flash_attn_fwd_fp8_f32(
            B, H, T, hd, ld, scale, _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse),
            _ptr(fp8_amax), _stream()))
        return
    name = ("pk_flash_attn_fwd_bf16x3_f32" if bf16x3 else
            "pk_flash_attn_fwd_bf16_f32" if bf16 else "pk_flash_attn_fwd_f32")
    check(name, getattr(hip_lib(), name)(
        B, H, T, hd, ld, scale, _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), _stream()))


FLASH_RECOMPUTE = 16


def flash_bwd(B, H, q, k, v, o, lse, dout, dq, dk, dv, flags=0, scale=None, bf16=False,
              recompute=False, fp8_amax=None, bf16x3=False):
    """recompute: PK_FLASH_RECOMPUTE, dQ from recomputed scores (a workspace of
    the row constants only); fp8_amax: the e4m3 products, with the amax the
    forward filled (pk_flash_attn_bwd_fp8_f32)"""
    T, hd, ld = _attn_layout(B, H, q, k, v, o, dq, dk, dv)
    if not dout.is_contiguous() or dout.shape != o.shape:
        raise ValueError("attention: dout must be contiguous like o")
    scale = hd ** -0.5 if scale is None else scale
    if recompute:
        flags |= FLASH_RECOMPUTE
        need = int(hip_lib().pk_flash_attn_bwd_workspace_recompute(B, H, T))
    else:
        need = int(hip_lib().pk_flash_attn_bwd_workspace(B, H, T))
    ws = torch.empty(max(1, need // 4), device=q.device, dtype=torch.float32)
    if fp8_amax is not None:
        _f32(fp8_amax)
        check("pk_flash_attn_bwd_fp8_f32", hip_lib().pk_flash_attn_bwd_fp8_f32(
            B, H, T, hd, ld, scale, _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), _ptr(dout),
            _ptr(dq), _ptr(dk), _ptr(dv), _ptr(fp8_amax), _ptr(ws), ws.numel() * 4, flags,
            _stream()))
        return
    name = ("pk_flash_attn_bwd_bf16x3_f32" if bf16x3 else
            "pk_flash_attn_bwd_bf16_f32" if bf16 else "pk_flash_attn_bwd_f32")
    check(name, getattr(hip_lib(), name)(
        B, H, T, hd, ld, scale, _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), _ptr(dout),
        _ptr(dq), _ptr(dk), _ptr(dv), _ptr(ws), ws.numel() * 4, flags, _stream()))


def causal_softmax_fwd(BH, T, S, P, lse, scale=1.0):
    check("pk_causal_softmax_fwd_f32", hip_lib().pk_causal_softmax_fwd_f32(
        BH, T, scale, _ptr(S), _ptr(P), _ptr(lse), _stream()))


def causal_softmax_bwd(BH, T, P, dP, dS):
    check("pk_causal_softmax_bwd_f32", hip_lib().pk_causal_softmax_bwd_f32(
        BH, T, _ptr(P), _ptr(dP), _ptr(dS), _stream()))


def embed_fwd(ids, table, out):
    n, d = out.shape
    check("pk_embed_fwd_f32", hip_lib().pk_embed_fwd_f32(n, d, table.shape[0], _ptr(ids),
                                                          _ptr(table), _ptr(out), _stream()))
    return out


def embed_bwd(ids, dout, dtable):
    """dtable[ids[i]] += dout[i], each row's adds in increasing i"""
    n, d = dout.shape
    need = hip_lib().pk_embed_bwd_workspace(n)
    ws = torch.empty(max(1, need), dtype=torch.uint8, device=dout.device)
    check("pk_embed_bwd_f32", hip_lib().pk_embed_bwd_f32(n, d, dtable.shape[0], _ptr(ids),
                                                          _ptr(dout), _ptr(dtable), _ptr(ws),
                                                          need, _stream()))
    return dtable


def device_info():
    cu, clk = ctypes.c_int(0), ctypes.c_int(0)
    arch = ctypes.create_string_buffer(64)
    check("pk_device_info", hip_lib().pk_device_info(ctypes.byref(cu), ctypes.byref(clk), arch, 64))
    return {"cu_count": cu.value, "clock_khz": clk.value, "arch": arch.value.decode()}
