"""tensor.MatMul's operand semantics on the GPU (fa_matmul_strided[_dev]).

The reference's MatMul consumes transposed and offset views without copying,
broadcasts batch dimensions (stride 0) and promotes 1-D operands
(tensor/matmul.go:10-127). These tests hand numpy views of every such kind to
the Python mirror (ai_amd/tensor.py MatMul, which passes the views' strides
to the C ABI) and compare with float64 products at the reference's bar,
|got - want| <= 1e-4 (1 + |want|) (tensor/tensor_test.go:10-26, 370-433).
cluster.Similarities is MatMul(q, docs.T()) (cluster/cluster.go:185-190): at
config 5's size (256 x 768 queries against 100 000 x 768 docs) its scores
through the strided path are checked against float64 and its top-10 against
the CPU oracle's.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from ai_amd import _native as N
from ai_amd import synth as S
from ai_amd import tensor as T

pytestmark = pytest.mark.gpu


def close(got, want, tol=1e-4, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    d = np.abs(got - want)
    worst = float(d.max()) if d.size else 0.0
    print(f"{what}: max|d|={worst:.3g}", flush=True)
    bad = np.argwhere(d > tol * (1 + np.abs(want)))
    assert bad.size == 0, f"{what}: {bad.shape[0]} elements out of tolerance, first at {bad[0]}"
    return worst


def f64mm(a, b):
    return np.matmul(np.asarray(a, np.float64), np.asarray(b, np.float64))


def rn(r, *shape):
    return r.standard_normal(shape).astype(np.float32)


# the reference's TestMatMul shapes (tensor/tensor_test.go:372), m, k, n
SHAPES = [(1, 1, 1), (2, 3, 4), (7, 5, 9), (64, 64, 64), (33, 17, 65), (1, 40, 50), (50, 40, 1), (130, 70, 90),
          (300, 768, 257)]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_transposed_views(ctx, m, k, n):
    r = np.random.default_rng(m * 1000 + k * 10 + n)
    a, b = rn(r, m, k), rn(r, k, n)
    at, bt = rn(r, k, m).T, rn(r, n, k).T  # views with unit row stride
    assert not at.flags.c_contiguous or m == 1 or k == 1
    close(T.MatMul(a, b, ctx=ctx), f64mm(a, b), what=f"AB {m}x{k}x{n}")
    close(T.MatMul(at, b, ctx=ctx), f64mm(at, b), what=f"AtB {m}x{k}x{n}")
    close(T.MatMul(a, bt, ctx=ctx), f64mm(a, bt), what=f"ABt {m}x{k}x{n}")
    close(T.MatMul(at, bt, ctx=ctx), f64mm(at, bt), what=f"AtBt {m}x{k}x{n}")


def test_vector_forms(ctx):
    """1-D promotion (matmul.go:24-30): exact on small integers."""
    v = np.array([1, 2, 3], np.float32)
    m = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    d = T.MatMul(v, v, ctx=ctx)
    assert d.shape == () and float(d) == 14.0
    assert np.array_equal(T.MatMul(m, v, ctx=ctx), [14, 32])
    assert np.array_equal(T.MatMul(v, m.T, ctx=ctx), [14, 32])
    r = np.random.default_rng(3)
    x, y = rn(r, 4, 3, 9), rn(r, 9)
    close(T.MatMul(x, y, ctx=ctx), f64mm(x, y), what="batched . 1-D")
    z = rn(r, 2, 9, 5)
    close(T.MatMul(y, z, ctx=ctx), f64mm(y, z), what="1-D . batched")


def test_batched_broadcast(ctx):
    r = np.random.default_rng(11)
    a, b = rn(r, 3, 2, 4, 5), rn(r, 2, 5, 6)
    got = T.MatMul(a, b, ctx=ctx)
    assert got.shape == (3, 2, 4, 6)
    close(got, f64mm(a, b), what="batched broadcast")
    c = rn(r, 5, 7)  # batched x 2-D: folds into M
    close(T.MatMul(a, c, ctx=ctx), f64mm(a, c), what="batched x 2-D")
    bt = np.swapaxes(rn(r, 2, 6, 5), 1, 2)  # strided batch operand
    close(T.MatMul(a, bt, ctx=ctx), f64mm(a, bt), what="batched transposed")
    x, y = rn(r, 64, 8, 8), rn(r, 64, 8, 8)  # many small products
    close(T.MatMul(x, y, ctx=ctx), f64mm(x, y), what="small batch")
    # a non-contiguous batched left operand against a 2-D right operand
    xt = np.swapaxes(rn(r, 3, 9, 4), 1, 2)
    w = rn(r, 9, 33)
    close(T.MatMul(xt, w, ctx=ctx), f64mm(xt, w), what="strided batch x 2-D")
    # stride-0 batch dimensions on either side, and broadcasting both ways
    e = np.broadcast_to(rn(r, 1, 4, 8), (5, 4, 8))
    f = rn(r, 5, 8, 3)
    close(T.MatMul(e, f, ctx=ctx), f64mm(e, f), what="stride-0 batch left")
    g = np.broadcast_to(rn(r, 8, 3), (6, 8, 3))
    left = rn(r, 6, 4, 8)
    close(T.MatMul(left, g, ctx=ctx), f64mm(left, g), what="stride-0 batch right")
    p, q = rn(r, 2, 1, 3, 40), rn(r, 1, 5, 40, 7)
    close(T.MatMul(p, q, ctx=ctx), f64mm(p, q), what="two-way broadcast [2,1]x[1,5]")
    # attention's composed path shape: [B,H,T,D] . [B,H,D,S] as Transpose(-2,-1) of k
    qh, kh = rn(r, 2, 3, 50, 64), rn(r, 2, 3, 70, 64)
    kt = np.swapaxes(kh, -1, -2)
    close(T.MatMul(qh, kt, ctx=ctx), f64mm(qh, kt), what="q . k^T (batched transposed)")


def test_offset_and_zero_stride_views(ctx):
    r = np.random.default_rng(21)
    big = rn(r, 70, 90)
    an = big[3:43, 5:69]  # offset rows and columns, row stride 90
    bn = rn(r, 100, 50)[17:81]
    close(T.MatMul(an, bn, ctx=ctx), f64mm(an, bn), what="offset views")
    brow = np.broadcast_to(rn(r, 1, 50), (64, 50))  # row stride 0
    close(T.MatMul(an, brow, ctx=ctx), f64mm(an, brow), what="row stride 0")
    cols = rn(r, 64, 200)[:, ::4]  # column stride 4
    close(T.MatMul(an, cols, ctx=ctx), f64mm(an, cols), what="column stride 4")
    # a misaligned start (one float in) of a row-major A with k % 32 == 0: packed, not read in place
    base = rn(r, 33 * 64 + 1)
    am = base[1:].reshape(33, 64)
    bm = rn(r, 64, 40)
    close(T.MatMul(am, bm, ctx=ctx), f64mm(am, bm), what="misaligned A")


def test_empty_and_errors(ctx):
    assert np.array_equal(T.MatMul(np.zeros((3, 0), np.float32), np.zeros((0, 4), np.float32), ctx=ctx), np.zeros((3, 4)))
    assert T.MatMul(np.zeros((0, 5), np.float32), np.ones((5, 4), np.float32), ctx=ctx).shape == (0, 4)
    assert T.MatMul(np.zeros((2, 0, 3, 5), np.float32), np.ones((5, 4), np.float32), ctx=ctx).shape == (2, 0, 3, 4)
    for a, b in [((2, 3), (2, 3)), ((2, 3, 4), (3, 4, 5))]:
        with pytest.raises(T.TensorError):
            T.MatMul(np.zeros(a, np.float32), np.zeros(b, np.float32), ctx=ctx)
    with pytest.raises(T.TensorError):
        T.MatMul(np.float32(1), np.zeros(2, np.float32), ctx=ctx)
    # the C ABI's own checks: negative strides, an epilogue on a batch
    L = N.lib()
    a = N.Matrix(); a.rs, a.cs = -1, 1
    b = N.Matrix(); b.rs, b.cs = 1, 1
    out = np.empty(4, np.float32)
    rc = L.fa_matmul_strided(ctx.h, 0, None, 2, 2, 2, C.byref(a), C.byref(b), None, N.ptr(out))
    assert rc == N.FA_ERR_ARG and b"negative stride" in L.fa_last_error(ctx.h)
    a.rs = 2
    batch = (N.i64 * 1)(2)
    rc = L.fa_matmul_strided(ctx.h, 1, batch, 2, 2, 2, C.byref(a), C.byref(b), C.byref(N.Epilogue()), N.ptr(out))
    assert rc == N.FA_ERR_ARG and b"MatMulFused" in L.fa_last_error(ctx.h)


def test_dev_variant_batched_transposed(ctx):
    """fa_matmul_strided_dev on device buffers: [4, 2] batches of A^T . B with
    B's batch dimension 0 broadcast."""
    r = np.random.default_rng(31)
    xa = rn(r, 4, 2, 96, 37)  # stored [.., k, m]; A = its transpose
    xb = rn(r, 1, 2, 96, 45)  # [1, 2, k, n], broadcast over the first batch dim
    want = f64mm(np.swapaxes(xa, -1, -2), xb)
    L = N.lib()
    bufs = []
    for arr in (xa, xb):
        p = C.c_void_p()
        N.check(ctx.h, L.fa_device_alloc(ctx.h, arr.nbytes, C.byref(p)))
        N.check(ctx.h, L.fa_memcpy_h2d(ctx.h, p, arr.ctypes.data, arr.nbytes))
        bufs.append(p)
    po = C.c_void_p()
    N.check(ctx.h, L.fa_device_alloc(ctx.h, want.size * 4, C.byref(po)))
    try:
        a = N.Matrix(); a.data = bufs[0].value; a.rs, a.cs = 1, 37
        a.bstride[0], a.bstride[1] = 2 * 96 * 37, 96 * 37
        b = N.Matrix(); b.data = bufs[1].value; b.rs, b.cs = 45, 1
        b.bstride[0], b.bstride[1] = 0, 96 * 45
        batch = (N.i64 * 2)(4, 2)
        N.check(ctx.h, L.fa_matmul_strided_dev(ctx.h, 2, batch, 37, 45, 96, C.byref(a), C.byref(b), None, po))
        got = np.empty(want.shape, np.float32)
        N.check(ctx.h, L.fa_memcpy_d2h(ctx.h, got.ctypes.data, po, got.nbytes))
    finally:
        for p in bufs + [po]:
            L.fa_device_free(ctx.h, p)
    close(got, want, what="dev batched A^T B")


def test_similarities_through_matmul_c5(ctx):
    """cluster.Similarities(q, docs) = q.MatMul(docs.T()) (cluster.go:185-190)
    at config 5's size: docs.T is a transposed view (unit row stride), read in
    place. Scores against float64; top-10 against the CPU oracle."""
    q = S.unit_rows(5, "queries", 256, 768)
    docs = S.unit_rows(5, "corpus", 100000, 768)
    scores = T.MatMul(q, docs.T, ctx=ctx)
    assert scores.shape == (256, 100000)
    exact = f64mm(q, docs.T)
    worst = close(scores, exact, what="Similarities via MatMul (C5)")
    assert worst < 2e-6
    oi, ov = O.similarities_topk(q, docs, 10)
    # top-10 by the GPU scores (value descending, lower index first on ties)
    gi = np.argsort(-scores, axis=1, kind="stable")[:, :10]
    ex_sorted = -np.sort(-exact, axis=1)
    gaps = np.minimum(np.abs(np.diff(ex_sorted[:, :11], axis=1)).min(axis=1), 1.0)
    clear = gaps > 4 * worst + 1e-7  # rows whose order no rounding at this size can change
    print(f"rows with clear top-11 gaps: {int(clear.sum())} / 256", flush=True)
    assert clear.sum() >= 200
    assert np.array_equal(gi[clear], oi[clear])
    close(np.take_along_axis(scores, oi.astype(np.int64), 1), ov, what="oracle top-10 values")
