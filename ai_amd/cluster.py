"""Host-side mirror of fiber/ai's cluster package (cluster/cluster.go),
computed on the GPU through the C ABI (include/fa_rocm.h).

Normalize, KMeans (-> Result with Centres, Assignment, Similarity, Sizes,
Iterations and Inertia()), Nearest, Cosine and Similarities keep the
reference's names, argument meaning and panics (raised here as
ClusterError, or TensorError for the shape checks of the tensor layer).
Rows are numpy float32 arrays; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field

import numpy as np

from . import _native as N
from .tensor import TensorError, _call, _f32, default_context


class ClusterError(ValueError):
    """The reference's panic("cluster: ...")."""


def _rows(x, op: str) -> np.ndarray:
    x = _f32(x)
    if x.ndim != 2:
        raise TensorError(op, f"want a 2-D tensor, got shape {list(x.shape)}")
    return x


def Normalize(x, *, ctx: N.Context | None = None) -> np.ndarray:
    """Every row scaled to unit length; zero rows stay zero (cluster.go:17-28)."""
    ctx = ctx or default_context()
    x = _rows(x, "Normalize")
    out = np.empty_like(x)
    _call("Normalize", ctx, N.lib().fa_cluster_normalize(ctx.h, N.ptr(x), x.shape[0], x.shape[1], N.ptr(out)))
    return out


@dataclass
class Result:
    """cluster.Result (cluster.go:30-37)."""
    Centres: np.ndarray
    Assignment: np.ndarray
    Similarity: np.ndarray
    Sizes: np.ndarray
    Iterations: int = 0

    def Inertia(self) -> float:
        """Mean cosine distance of rows to their centres (cluster.go:148-159)."""
        if len(self.Similarity) == 0:
            return math.nan
        s = 0.0
        for v in self.Similarity.tolist():
            s += 1 - float(np.float32(v))
        return s / len(self.Similarity)


def KMeans(x, k: int, iters: int, seed: int, *, ctx: N.Context | None = None) -> Result:
    """k-means++ seeding and Lloyd rounds on the unit-length rows of x
    (cluster.go:39-131)."""
    ctx = ctx or default_context()
    x = _rows(x, "KMeans")
    n, d = x.shape
    if k <= 0 or k > n:
        raise ClusterError("cluster: k must be between 1 and the number of rows")
    centres = np.empty((k, d), np.float32)
    assign = np.empty(n, np.int32)
    sim = np.empty(n, np.float32)
    sizes = np.empty(k, np.int32)
    it = C.c_int32(0)
    _call("KMeans", ctx, N.lib().fa_cluster_kmeans(ctx.h, N.ptr(x), n, d, k, iters, C.c_uint64(seed & (2**64 - 1)),
                                                    N.ptr(centres), N.ptr(assign), N.ptr(sim), N.ptr(sizes),
                                                    C.byref(it)))
    return Result(centres, assign, sim, sizes, it.value)


def Nearest(x, centres, *, ctx: N.Context | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Index of the most similar centre for every row, and that similarity
    (cluster.go:134-146)."""
    ctx = ctx or default_context()
    x, c = _rows(x, "MatMul"), _rows(centres, "MatMul")
    if x.shape[1] != c.shape[1]:
        raise TensorError("MatMul", f"shapes {list(x.shape)} and {[c.shape[1], c.shape[0]]} do not chain")
    n = x.shape[0]
    idx = np.empty(n, np.int32)
    sim = np.empty(n, np.float32)
    _call("Nearest", ctx, N.lib().fa_cluster_nearest(ctx.h, N.ptr(x), n, N.ptr(c), c.shape[0], x.shape[1],
                                                      N.ptr(idx), N.ptr(sim)))
    return idx, sim


def Similarities(queries, docs, *, ctx: N.Context | None = None) -> np.ndarray:
    """[q x n] dot products of unit-length rows, one product (cluster.go:180-190)."""
    from .tensor import MatMul
    q, dm = _f32(queries), _f32(docs)
    if q.ndim != 2 or dm.ndim != 2 or q.shape[1] != dm.shape[1]:
        raise ClusterError(f"cluster: Similarities: shapes {list(q.shape)} and {list(dm.shape)}")
    return MatMul(q, dm, w_layout=N.FA_B_NK, ctx=ctx)


def Cosine(a, b, *, ctx: N.Context | None = None) -> float:
    """Cosine similarity of two equal-length vectors; 0 when either is all
    zero or both are empty (cluster.go:161-178). The three sums come from
    one product of the stacked pair with itself; the quotient is float64."""
    a, b = _f32(a).ravel(), _f32(b).ravel()
    if len(a) != len(b):
        raise ClusterError(f"cluster: Cosine: lengths {len(a)} and {len(b)} differ")
    if len(a) == 0:
        return 0.0
    from .tensor import MatMul
    pair = np.stack([a, b])
    g = MatMul(pair, pair, w_layout=N.FA_B_NK, ctx=ctx)
    dot, na, nb = g[0, 1], g[0, 0], g[1, 1]
    if na == 0 or nb == 0:
        return 0.0
    return float(np.float32(float(dot) / math.sqrt(float(na) * float(nb))))
