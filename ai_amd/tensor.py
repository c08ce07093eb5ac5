"""Host-side mirror of fiber/ai's tensor operators on the EmbeddingGemma path,
computed on the GPU through the C ABI (include/fa_rocm.h).

Names, argument meaning and error behaviour follow the reference's Go API
(tensor/matmul.go, tensor/matmul_fused.go, tensor/attention.go,
tensor/rope.go): arrays are numpy float32, shapes are checked the way the
reference checks them, and a shape error raises TensorError (the reference
panics with *tensor.Error{Op, Msg}, tensor/errors.go:5-31). Computation
happens on the device; there is no CPU fallback.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import _native as N

MASK_NEG = np.float32(-1e9)  # tensor/attention.go:17

NoAct, ReLUAct, GELUAct = N.FA_ACT_NONE, N.FA_ACT_RELU, N.FA_ACT_GELU


class TensorError(ValueError):
    """Shape/argument error: the reference's *tensor.Error{Op, Msg}."""

    def __init__(self, op: str, msg: str):
        super().__init__(f"tensor: {op}: {msg}")
        self.op = op
        self.msg = msg


def _fail(op: str, msg: str):
    raise TensorError(op, msg)


_default_ctx: N.Context | None = None


def default_context() -> N.Context:
    global _default_ctx
    if _default_ctx is None:
        _default_ctx = N.Context(0)
    return _default_ctx


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _call(op: str, ctx: N.Context, rc: int) -> None:
    if rc == N.FA_OK:
        return
    msg = N.lib().fa_last_error(ctx.h).decode()
    if rc == N.FA_ERR_ARG:
        raise TensorError(op, msg)
    raise N.FaError(rc, msg)


@dataclass
class Fused:
    """Epilogue of MatMulFused (tensor/matmul_fused.go:11-23), applied in the
    order Bias, RowScale, Act, Mul, Residual."""
    Bias: np.ndarray | None = None
    Act: int = NoAct
    Mul: np.ndarray | None = None
    RowScale: np.ndarray | None = None
    Residual: np.ndarray | None = None


def MatMulFused(x, w, f: Fused | None = None, *, w_layout: int = N.FA_B_KN, ctx: N.Context | None = None):
    """epilogue(x . w) for 2-D x [m x k] and w [k x n] (tensor/matmul_fused.go:40-96).

    w may be float32 or bfloat16 (a uint16 array of bf16 bits); with
    w_layout=FA_B_NK it is stored [n x k] (a checkpoint's [out, in]).
    """
    ctx = ctx or default_context()
    x = _f32(x)
    w = np.asarray(w)
    if x.ndim != 2 or w.ndim != 2:
        _fail("MatMulFused", f"expected 2-D operands, got {list(x.shape)} and {list(w.shape)}")
    if w.dtype == np.uint16:
        b_dtype = N.FA_DT_BF16
    else:
        w = _f32(w)
        b_dtype = N.FA_DT_F32
    w = np.ascontiguousarray(w)
    m, k = x.shape
    if w_layout == N.FA_B_KN:
        kk, n = w.shape
    else:
        n, kk = w.shape
    if k != kk:
        _fail("MatMulFused", f"shape mismatch {list(x.shape)} · {list(w.shape)}")
    f = f or Fused()
    keep = []
    e = N.Epilogue()
    e.act = f.Act
    if f.Bias is not None:
        b = _f32(f.Bias).ravel()
        if b.size != n:
            _fail("MatMulFused", f"bias has {b.size} elements for {n} columns")
        keep.append(b)
        e.bias = b.ctypes.data
    if f.RowScale is not None:
        rs = _f32(f.RowScale).ravel()
        if rs.size != m:
            _fail("MatMulFused", f"row scale has {rs.size} elements for {m} rows")
        keep.append(rs)
        e.row_scale = rs.ctypes.data
    for name, t in (("mul", f.Mul), ("residual", f.Residual)):
        if t is not None:
            t = _f32(t)
            if t.shape != (m, n):
                _fail("MatMulFused", f"Mul/Residual must be [{m}×{n}], got {list(t.shape)}")
            keep.append(t)
            setattr(e, name, t.ctypes.data)
            setattr(e, "ldm" if name == "mul" else "ldr", n)
    out = np.empty((m, n), np.float32)
    ldb = w.shape[1]
    _call("MatMulFused", ctx, N.lib().fa_matmul_fused(ctx.h, m, n, k, N.ptr(x), k, N.ptr(w), ldb, b_dtype, w_layout,
                                                      N.C.byref(e), N.ptr(out), n))
    return out


def _view(a: np.ndarray) -> np.ndarray:
    """a as float32 whose strides are non-negative multiples of 4 bytes (a
    view unchanged when it already is; a copy otherwise)."""
    if a.dtype != np.float32:
        return a.astype(np.float32)
    if any(s < 0 or s % 4 for s in a.strides):
        return np.ascontiguousarray(a)
    return a


def _broadcast_shapes(a: tuple, b: tuple) -> tuple:
    """broadcastShapes (tensor/shape.go:94-118)."""
    n = max(len(a), len(b))
    out = []
    for i in range(n, 0, -1):
        da = a[len(a) - i] if i <= len(a) else 1
        db = b[len(b) - i] if i <= len(b) else 1
        if da == db or db == 1:
            out.append(da)
        elif da == 1:
            out.append(db)
        else:
            _fail("MatMul", f"shapes {list(a)} and {list(b)} are not broadcastable")
    return tuple(out)


def _matrix(a: np.ndarray, batch: tuple) -> N.Matrix:
    """fa_matrix of a's last two dimensions, with broadcastStrides over batch
    (tensor/shape.go:122-131: stride 0 where a batch dimension is broadcast)."""
    v = N.Matrix()
    v.data = a.ctypes.data
    v.rs, v.cs = a.strides[-2] // 4, a.strides[-1] // 4
    lead = a.shape[:-2]
    off = len(batch) - len(lead)
    for d in range(len(batch)):
        if d >= off and lead[d - off] != 1:
            v.bstride[d] = a.strides[d - off] // 4
    return v


def _matmul_views(x: np.ndarray, w: np.ndarray, batch: tuple, ctx: N.Context) -> np.ndarray:
    m, k, n = x.shape[-2], x.shape[-1], w.shape[-1]
    out = np.empty(batch + (m, n), np.float32)
    if out.size == 0:
        return out
    if len(batch) > N.FA_MAX_BATCH_DIMS:
        _fail("MatMul", f"{len(batch)} batch dimensions, at most {N.FA_MAX_BATCH_DIMS}")
    a, b = _matrix(x, batch), _matrix(w, batch)
    bshape = (N.i64 * max(len(batch), 1))(*batch)
    _call("MatMul", ctx, N.lib().fa_matmul_strided(ctx.h, len(batch), bshape, m, n, k, N.C.byref(a), N.C.byref(b),
                                                   None, N.ptr(out)))
    return out


def MatMul(x, w, *, w_layout: int = N.FA_B_KN, ctx: N.Context | None = None):
    """tensor.MatMul (tensor/matmul.go:10-127): NumPy semantics. 2-D x 2-D is
    the matrix product; a 1-D operand is promoted to a row (left) or a column
    (right) and the added dimension removed; with more dimensions the batch
    dimensions broadcast (stride 0). Strided numpy views (transposes, slices,
    broadcast_to) are read through their strides on the device, not copied.

    A bfloat16 w (uint16 bits) or w_layout=FA_B_NK ([n x k] storage) takes the
    2-D weight path of MatMulFused.
    """
    ctx = ctx or default_context()
    x, w = np.asarray(x), np.asarray(w)
    if w.dtype == np.uint16 or w_layout != N.FA_B_KN:
        return MatMulFused(x, w, None, w_layout=w_layout, ctx=ctx)
    if x.ndim == 0 or w.ndim == 0:
        _fail("MatMul", f"operands must be at least 1-D, got {list(x.shape)} and {list(w.shape)}")
    if x.ndim == 1 and w.ndim == 1:
        if x.shape[0] != w.shape[0]:
            _fail("MatMul", f"shape mismatch {list(x.shape)} · {list(w.shape)}")
        return MatMul(x[None, :], w[:, None], ctx=ctx).reshape(())
    if x.ndim == 1:
        return MatMul(x[None, :], w, ctx=ctx)[..., 0, :]
    if w.ndim == 1:
        return MatMul(x, w[:, None], ctx=ctx)[..., 0]
    x, w = _view(x), _view(w)
    m, k, n = x.shape[-2], x.shape[-1], w.shape[-1]
    if k != w.shape[-2]:
        _fail("MatMul", f"shape mismatch {list(x.shape)} · {list(w.shape)}")
    if x.ndim == 2 and w.ndim == 2:
        return _matmul_views(x, w, (), ctx)
    if w.ndim == 2 and x.flags.c_contiguous:  # [B..., m, k] . [k, n]: the batch folds into M
        rows = int(np.prod(x.shape[:-2], dtype=np.int64)) * m
        return _matmul_views(x.reshape(rows, k), w, (), ctx).reshape(x.shape[:-2] + (m, n))
    return _matmul_views(x, w, _broadcast_shapes(x.shape[:-2], w.shape[:-2]), ctx)


def RowSumSquares(x, *, ctx: N.Context | None = None):
    """Per-row sum of squares of a 2-D tensor (tensor/matmul_fused.go:125-143)."""
    ctx = ctx or default_context()
    x = np.asarray(x)
    if x.ndim != 2:
        _fail("RowSumSquares", f"expected a 2-D tensor, got {list(x.shape)}")
    x = _f32(x)  # a transposed view is made contiguous, as the reference does
    out = np.empty(x.shape[0], np.float32)
    _call("RowSumSquares", ctx, N.lib().fa_row_sum_squares(ctx.h, N.ptr(x), x.shape[0], x.shape[1], N.ptr(out)))
    return out


def RMSNorm(x, g, eps: float, *, ctx: N.Context | None = None):
    """x / sqrt(mean(x^2) + eps) * g over the last dimension (tensor/attention.go:292-337)."""
    ctx = ctx or default_context()
    x = _f32(x)
    if x.ndim == 0:
        _fail("RMSNorm", "expected at least a 1-D input")
    n = x.shape[-1]
    g = _f32(g).ravel()
    if g.size != n:
        _fail("RMSNorm", f"g must have {n} elements, got {g.size}")
    out = np.empty_like(x)
    rows = x.size // n if n else 0
    _call("RMSNorm", ctx, N.lib().fa_rmsnorm(ctx.h, N.ptr(x), N.ptr(g), eps, rows, n, N.ptr(out)))
    return out


def RoPE(x, base: float, positions, *, ctx: N.Context | None = None):
    """Rotary embedding of [..., T, D] at the given positions (tensor/rope.go:20-61)."""
    ctx = ctx or default_context()
    x = _f32(x)
    if x.ndim < 2:
        _fail("RoPE", f"expected at least a 2-D input, got {list(x.shape)}")
    T, D = x.shape[-2], x.shape[-1]
    if D % 2 != 0:
        _fail("RoPE", f"head dimension {D} must be even")
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    if pos.size != T:
        _fail("RoPE", f"got {pos.size} positions for {T} slots")
    out = np.empty_like(x)
    rows = x.size // D if D else 0
    if rows == 0:
        return out
    _call("RoPE", ctx, N.lib().fa_rope(ctx.h, N.ptr(x), float(base), N.ptr(pos), rows, T, D, N.ptr(out)))
    return out


def _strides_el(a: np.ndarray) -> tuple[int, ...]:
    return tuple(s // a.itemsize for s in a.strides)


def AttentionScaled(q, k, v, mask, scale: float, *, ctx: N.Context | None = None):
    """softmax(scale * q.k^T + mask) . v (tensor/attention.go:67-83).

    q [..., T, D], k/v [..., S, D] with the same leading dims (up to two);
    k and v may be broadcast views over the head axis (np.broadcast_to, the
    reference's Expand) for grouped-query attention. mask is None or
    broadcastable to [..., T, S].
    """
    ctx = ctx or default_context()
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    nd = q.ndim
    if nd < 2 or k.ndim != nd or v.ndim != nd:
        _fail("Attention", f"q, k, v must have the same rank ≥ 2, got {list(q.shape)} {list(k.shape)} {list(v.shape)}")
    D = q.shape[-1]
    if k.shape[-1] != D or v.shape[-2] != k.shape[-2]:
        _fail("Attention", f"shapes do not match: q {list(q.shape)}, k {list(k.shape)}, v {list(v.shape)}")
    if k.shape[:-2] != q.shape[:-2] or v.shape[:-2] != q.shape[:-2] or v.shape[-1] != D:
        _fail("Attention", "leading dimensions of q, k, v differ")
    if nd > 4:
        lead = q.shape[:-2]
        q = q.reshape(1, -1, *q.shape[-2:])
        k = np.ascontiguousarray(k).reshape(1, -1, *k.shape[-2:])
        v = np.ascontiguousarray(v).reshape(1, -1, *v.shape[-2:])
        if mask is not None:
            mask = np.broadcast_to(np.asarray(mask, np.float32), (*lead, q.shape[-2], k.shape[-2]))
            mask = np.ascontiguousarray(mask).reshape(1, -1, q.shape[-2], k.shape[-2])
        out = AttentionScaled(q, k, v, mask, scale, ctx=ctx)
        return out.reshape(*lead, *out.shape[-2:])
    orig_shape = q.shape
    # to 4-D [B, H, T, D]
    while q.ndim < 4:
        q, k, v = q[None], k[None], v[None]
    B, H, T, _ = q.shape
    S = k.shape[-2]

    def prep(a):
        # rows of D contiguous; lead strides kept (0 where broadcast)
        if a.strides[-1] != a.itemsize or (a.shape[-2] > 1 and a.strides[-2] != a.shape[-1] * a.itemsize):
            a = np.ascontiguousarray(a)
        return a

    q, k, v = prep(q), prep(k), prep(v)
    qs, ks, vs = _strides_el(q), _strides_el(k), _strides_el(v)
    mp = None
    msb = msh = msr = msc = 0
    if mask is not None:
        m = np.asarray(mask, dtype=np.float32)
        if m.ndim > 4:
            _fail("Attention", f"mask rank {m.ndim} > 4")
        try:
            mb = np.broadcast_to(m, (B, H, T, S))
        except ValueError:
            _fail("Attention", f"mask {list(m.shape)} does not broadcast to {[B, H, T, S]}")
        base = m
        while base.ndim < 4:
            base = base[None]
        base = np.ascontiguousarray(base)
        mb = np.broadcast_to(base, (B, H, T, S))
        msb, msh, msr, msc = _strides_el(mb)
        mp = base
    out = np.empty((B, H, T, D), np.float32)
    # pass the base pointers of the (possibly broadcast) arrays
    _call("Attention", ctx, N.lib().fa_attention(
        ctx.h, q.ctypes.data, k.ctypes.data, v.ctypes.data, B, H, T, S, D, qs[0], qs[1], ks[0], ks[1], vs[0], vs[1],
        None if mp is None else mp.ctypes.data, msb, msh, msr, msc, float(scale), N.ptr(out)))
    return out.reshape(orig_shape)


def Attention(q, k, v, mask, *, ctx: N.Context | None = None):
    """Attention with the default scale 1/sqrt(D) (tensor/attention.go:56-59)."""
    D = np.asarray(q).shape[-1]
    return AttentionScaled(q, k, v, mask, float(np.float32(1.0 / np.sqrt(np.float64(D)))), ctx=ctx)


def PaddingMask(lengths, n: int) -> np.ndarray:
    """[len(lengths), 1, 1, n] additive mask hiding j >= length (tensor/attention.go:33-42)."""
    lengths = list(lengths)
    m = np.zeros((len(lengths), 1, 1, n), np.float32)
    for i, l in enumerate(lengths):
        m[i, 0, 0, max(0, l):] = MASK_NEG
    return m


def WindowMask(n: int, w: int) -> np.ndarray:
    """[n, n] additive mask: 0 where |i-j| < w (tensor/attention.go:97-107)."""
    i = np.arange(n)[:, None]
    j = np.arange(n)[None, :]
    return np.where((j - i >= w) | (i - j >= w), MASK_NEG, np.float32(0)).astype(np.float32)


def CausalMask(n: int) -> np.ndarray:
    """[n, n] additive mask hiding j > i (tensor/attention.go:21-29)."""
    i = np.arange(n)[:, None]
    j = np.arange(n)[None, :]
    return np.where(j > i, MASK_NEG, np.float32(0)).astype(np.float32)
