"""GPU parity of the tensor-level operators against the CPU oracle.

Every call goes through the C ABI (libfa_rocm.so) on the device. Tolerances
are the reference's: |gpu - want| <= 1e-4 * (1 + |want|) for products
(internal/blas/gemm_test.go:39-56), 1e-5/1e-6 for RMSNorm and RoPE
(tensor/rope_test.go:83-102), 1e-4 for attention
(tensor/attention_test.go:64-91). Max |delta| is printed for each case.
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from ai_amd import _native as N
from ai_amd import synth as S
from ai_amd import tensor as T

pytestmark = pytest.mark.gpu


def rng(seed):
    return np.random.default_rng(seed)


def close(got, want, tol=1e-4, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    d = np.abs(got - want)
    lim = tol * (1 + np.abs(want))
    worst = float(d.max()) if d.size else 0.0
    # relative to the output's scale (element-wise ratios blow up near zeros)
    rel = worst / max(float(np.abs(want).max()), 1e-30) if d.size else 0.0
    print(f"{what}: max|d|={worst:.3g} max rel={rel:.3g}", flush=True)
    bad = np.argwhere(d > lim)
    assert bad.size == 0, f"{what}: {bad.shape[0]} elements out of tolerance, first {bad[0]}: got {got[tuple(bad[0])]} want {want[tuple(bad[0])]}"
    return worst


# The reference's GEMM test shapes (internal/blas/gemm_test.go:75-79), m, n, k.
REF_SHAPES = [(1, 1, 1), (1, 1, 100), (1, 17, 5), (1, 100, 300), (5, 1, 7), (300, 1, 100), (3, 3, 3), (4, 16, 1),
              (6, 16, 7), (8, 12, 3), (12, 32, 9), (13, 33, 9), (5, 17, 9), (7, 37, 19), (64, 64, 64),
              (129, 65, 33), (133, 257, 300), (100, 20, 513), (257, 33, 1), (31, 4097, 7), (300, 300, 300)]


@pytest.mark.parametrize("m,n,k", REF_SHAPES)
def test_matmul_reference_shapes_f32(ctx, m, n, k):
    r = rng(m * 10007 + n * 101 + k)
    a = r.uniform(-1, 1, (m, k)).astype(np.float32)
    b = r.uniform(-1, 1, (k, n)).astype(np.float32)
    want = a.astype(np.float64) @ b.astype(np.float64)
    close(T.MatMul(a, b, ctx=ctx), want, what=f"f32 KN {m}x{n}x{k}")
    close(T.MatMul(a, np.ascontiguousarray(b.T), w_layout=N.FA_B_NK, ctx=ctx), want, what=f"f32 NK {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (13, 33, 9), (129, 65, 33), (133, 257, 300), (300, 300, 300)])
def test_matmul_bf16_weights(ctx, m, n, k):
    r = rng(7 + m)
    a = r.uniform(-1, 1, (m, k)).astype(np.float32)
    wb = S.normal_bf16(11, f"w{m}", 0.5, (n, k))
    wf = S.bf16_to_f32(wb)
    want = a.astype(np.float64) @ wf.T.astype(np.float64)
    close(T.MatMul(a, wb, w_layout=N.FA_B_NK, ctx=ctx), want, what=f"bf16 NK {m}x{n}x{k}")
    close(T.MatMul(a, np.ascontiguousarray(wb.T), w_layout=N.FA_B_KN, ctx=ctx), want, what=f"bf16 KN {m}x{n}x{k}")


# The encoder's product shapes at the configs (M rows; K, N) with bf16 weights.
@pytest.mark.parametrize("rows", [128, 5120, 8192, 16384, 32768])
@pytest.mark.parametrize("kdim,ncols", [(768, 1280), (768, 768), (768, 256), (768, 2304), (1152, 768)])
def test_matmul_config_shapes_vs_oracle(ctx, rows, kdim, ncols):
    r = rng(rows + kdim + ncols)
    a = r.standard_normal((rows, kdim)).astype(np.float32)
    wb = S.normal_bf16(5, f"cfg{kdim}x{ncols}", 0.02, (ncols, kdim))
    wf = S.bf16_to_f32(wb)
    got = T.MatMul(a, wb, w_layout=N.FA_B_NK, ctx=ctx)
    want = O.gemm(a, np.ascontiguousarray(wf.T))
    close(got, want, what=f"config M={rows} K={kdim} N={ncols}")


@pytest.mark.parametrize("act", [T.NoAct, T.ReLUAct, T.GELUAct])
def test_matmul_fused_epilogue_vs_oracle(ctx, act):
    r = rng(30 + act)
    m, n, k = 133, 257, 300
    a = r.uniform(-1, 1, (m, k)).astype(np.float32)
    b = r.uniform(-1, 1, (k, n)).astype(np.float32)
    bias = r.uniform(-1, 1, n).astype(np.float32)
    rs = r.uniform(0.5, 1.5, m).astype(np.float32)
    mul = r.uniform(-1, 1, (m, n)).astype(np.float32)
    res = r.uniform(-1, 1, (m, n)).astype(np.float32)
    got = T.MatMulFused(a, b, T.Fused(Bias=bias, RowScale=rs, Act=act, Mul=mul, Residual=res), ctx=ctx)
    want = O.gemm(a, b, bias, rs, act, mul, res)
    close(got, want, what=f"epilogue act={act}")
    # each field alone
    for f, args in [(T.Fused(Bias=bias), dict(bias=bias)), (T.Fused(RowScale=rs), dict(rowscale=rs)),
                    (T.Fused(Act=act), dict(act=act)), (T.Fused(Mul=mul), dict(mul=mul)),
                    (T.Fused(Residual=res), dict(residual=res))]:
        close(T.MatMulFused(a, b, f, ctx=ctx), O.gemm(a, b, **args), what=f"epilogue single {list(args)}")


@pytest.mark.parametrize("m,n,k", [(1, 3072, 768), (7, 257, 96), (33, 768, 3072), (128, 1280, 32), (200, 130, 1152)])
def test_matmul_bf16_few_rows_fused_vs_oracle(ctx, m, n, k):
    """bf16 [n x k] weights at few rows (the small-M split-bf16 kernel: eight
    waves share each 32 x 64 tile's K, K = 32 leaving seven idle) with the
    full epilogue, against the oracle's fused product."""
    r = rng(m * 31 + n + k)
    a = r.standard_normal((m, k)).astype(np.float32)
    wb = S.normal_bf16(17, f"few{m}x{n}x{k}", 0.05, (n, k))
    wt = np.ascontiguousarray(S.bf16_to_f32(wb).T)
    bias = r.uniform(-1, 1, n).astype(np.float32)
    rs = r.uniform(0.5, 1.5, m).astype(np.float32)
    mul = r.uniform(-1, 1, (m, n)).astype(np.float32)
    res = r.uniform(-1, 1, (m, n)).astype(np.float32)
    close(T.MatMul(a, wb, w_layout=N.FA_B_NK, ctx=ctx), O.gemm(a, wt), what=f"few rows {m}x{n}x{k}")
    got = T.MatMulFused(a, wb, T.Fused(Bias=bias, RowScale=rs, Act=T.GELUAct, Mul=mul, Residual=res),
                        w_layout=N.FA_B_NK, ctx=ctx)
    close(got, O.gemm(a, wt, bias, rs, T.GELUAct, mul, res), what=f"few rows fused {m}x{n}x{k}")


def test_matmul_padding_untouched(ctx):
    """A C with row gaps keeps the bytes between rows (gemm_test.go:50-55)."""
    r = rng(99)
    m, n, k = 37, 45, 64
    a = r.uniform(-1, 1, (m, k)).astype(np.float32)
    b = r.uniform(-1, 1, (k, n)).astype(np.float32)
    ldc = n + 7
    c = np.full(m * ldc, 123.0, np.float32)
    rc = N.lib().fa_matmul_fused(ctx.h, m, n, k, N.ptr(a), k, N.ptr(b), n, N.FA_DT_F32, N.FA_B_KN, None, N.ptr(c), ldc)
    N.check(ctx.h, rc)
    cm = c.reshape(m, ldc)
    close(cm[:, :n], a.astype(np.float64) @ b, what="ldc>n")
    assert np.all(cm[:, n:] == 123.0)


def test_matmul_errors(ctx):
    with pytest.raises(T.TensorError):
        T.MatMul(np.zeros((2, 3), np.float32), np.zeros((4, 5), np.float32), ctx=ctx)
    with pytest.raises(T.TensorError):
        T.MatMulFused(np.zeros((2, 3), np.float32), np.zeros((3, 5), np.float32),
                      T.Fused(Bias=np.zeros(4, np.float32)), ctx=ctx)


def test_row_sum_squares_kat(ctx):
    """tensor/matmul_fused_test.go:62-71."""
    x = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    assert T.RowSumSquares(x, ctx=ctx).tolist() == [14, 77]
    assert T.RowSumSquares(x.T, ctx=ctx).tolist() == [17, 29, 45]


@pytest.mark.parametrize("rows,n", [(20, 64), (3 * 8, 16), (5, 768), (1000, 256), (7, 1)])
def test_rmsnorm_vs_oracle(ctx, rows, n):
    r = rng(rows * n)
    x = (r.standard_normal((rows, n)) * 2).astype(np.float32)
    g = r.standard_normal(n).astype(np.float32)
    got = T.RMSNorm(x, g, 1e-6, ctx=ctx)
    close(got, O.rmsnorm(x, g, 1e-6), tol=1e-5, what=f"rmsnorm {rows}x{n}")


def test_rope_known(ctx):
    """tensor/rope_test.go:9-25."""
    got = T.RoPE(np.array([[1, 0]], np.float32), 10000, [1], ctx=ctx)
    assert abs(got[0, 0] - np.float32(np.cos(1))) <= 1e-6 and abs(got[0, 1] - np.float32(np.sin(1))) <= 1e-6
    ident = T.RoPE(np.array([[3, -4, 5, 6]], np.float32), 10000, [0], ctx=ctx)
    assert np.abs(ident - np.array([[3, -4, 5, 6]])).max() <= 1e-6


@pytest.mark.parametrize("base", [1e4, 1e6])
def test_rope_vs_oracle(ctx, base):
    r = rng(int(base))
    x = r.standard_normal((2, 3, 8, 256)).astype(np.float32)
    pos = [0, 5, 9, 100, 500, 1000, 2047, 7]
    got = T.RoPE(x, base, pos, ctx=ctx)
    close(got, O.rope(x, base, pos), tol=1e-5, what=f"rope base={base}")
    # norm preservation (rope_test.go:27-38)
    xn = (x.astype(np.float64) ** 2).sum(-1)
    yn = (got.astype(np.float64) ** 2).sum(-1)
    assert np.all(np.abs(xn - yn) <= 1e-3 * (xn + 1))


def test_attention_matches_naive_float64(ctx):
    """tensor/attention_test.go:56-92: B=2, H=3, T=5, S=7, D=4, with/without padding mask."""
    r = rng(41)
    B, H, Tq, Sk, D = 2, 3, 5, 7, 4
    q = r.standard_normal((B, H, Tq, D)).astype(np.float32)
    k = r.standard_normal((B, H, Sk, D)).astype(np.float32)
    v = r.standard_normal((B, H, Sk, D)).astype(np.float32)
    for mask in (None, T.PaddingMask([Sk, 3], Sk)):
        got = T.Attention(q, k, v, mask, ctx=ctx)
        s = np.einsum("bhtd,bhsd->bhts", q.astype(np.float64), k.astype(np.float64)) / np.sqrt(D)
        if mask is not None:
            s = s + mask.astype(np.float64)
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        want = np.einsum("bhts,bhsd->bhtd", p, v.astype(np.float64))
        close(got, want, what=f"attention naive mask={mask is not None}")


@pytest.mark.parametrize("B,H,Tq,Sk,D", [(2, 3, 65, 65, 256), (1, 3, 300, 300, 256), (2, 2, 17, 100, 64)])
def test_attention_vs_oracle_gqa_window_padding(ctx, B, H, Tq, Sk, D):
    r = rng(B * H * Tq)
    q = r.standard_normal((B, H, Tq, D)).astype(np.float32)
    k1 = r.standard_normal((B, 1, Sk, D)).astype(np.float32)
    v1 = r.standard_normal((B, 1, Sk, D)).astype(np.float32)
    k = np.broadcast_to(k1, (B, H, Sk, D))  # the reference's Expand
    v = np.broadcast_to(v1, (B, H, Sk, D))
    lengths = [Sk] + [max(1, Sk // 3)] * (B - 1)
    pad = T.PaddingMask(lengths, Sk)
    masks = [None, pad]
    if Tq == Sk:
        masks.append(pad + T.WindowMask(Tq, 17).reshape(1, 1, Tq, Tq))
    for mask in masks:
        got = T.AttentionScaled(q, k, v, mask, 0.0625, ctx=ctx)
        want = O.attention(q, k, v, mask, 0.0625)
        close(got, want, what=f"attention oracle {B},{H},{Tq},{Sk},{D}")


def test_masked_attention_weights_are_exact_zeros(ctx):
    """tensor/attention_test.go:266-285: causal position 0 reproduces v[0]."""
    r = rng(11)
    n, d = 64, 16
    q, k, v = (r.standard_normal((1, 1, n, d)).astype(np.float32) for _ in range(3))
    out = T.Attention(q, k, v, T.CausalMask(n), ctx=ctx)
    assert np.abs(out[0, 0, 0] - v[0, 0, 0]).max() <= 1e-6


def test_similarities_topk_vs_oracle(ctx):
    r = rng(5)
    q = r.standard_normal((33, 96)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    docs = r.standard_normal((5000, 96)).astype(np.float32)
    docs /= np.linalg.norm(docs, axis=1, keepdims=True)
    idx = np.empty((33, 10), np.int32)
    val = np.empty((33, 10), np.float32)
    N.check(ctx.h, N.lib().fa_similarities_topk(ctx.h, N.ptr(q), 33, N.ptr(docs), 5000, 96, 10, N.ptr(idx),
                                                N.ptr(val)))
    oi, ov = O.similarities_topk(q, docs, 10)
    s64 = q.astype(np.float64) @ docs.T.astype(np.float64)
    for i in range(33):
        if not np.array_equal(idx[i], oi[i]):
            # only a near-tie may reorder: the scores must agree to rounding
            assert np.allclose(s64[i, idx[i]], s64[i, oi[i]], atol=1e-6), (i, idx[i], oi[i])
    assert np.abs(val - ov).max() <= 1e-5


def test_topk_ties_lower_index_first(ctx):
    q = np.ones((1, 4), np.float32) * 0.5
    docs = np.zeros((300, 4), np.float32)
    docs[[7, 3, 250, 100], :] = 0.5  # equal best scores
    idx = np.empty((1, 5), np.int32)
    val = np.empty((1, 5), np.float32)
    N.check(ctx.h, N.lib().fa_similarities_topk(ctx.h, N.ptr(q), 1, N.ptr(docs), 300, 4, 5, N.ptr(idx), N.ptr(val)))
    assert idx[0, :4].tolist() == [3, 7, 100, 250]
    assert idx[0, 4] == 0  # first of the zero scores


@pytest.mark.parametrize("nd", [32, 4097, 300_000, 300_001])
@pytest.mark.parametrize("k", [1, 8, 9, 16, 17, 32])
def test_topk_exact_ties_across_chunks(ctx, nd, k):
    """Scores from 21 exact levels (value/16 times a unit query), so equal
    scores recur throughout the row: the top-k must be the first k of the
    stable order (score descending, index ascending) whatever the split of
    the row into chunks (reduce.go:286-289). nd % 4 == 0 takes the 16-byte
    load path."""
    r = rng(nd + k)
    nq, d = 3, 4
    q = np.zeros((nq, d), np.float32)
    q[:, 0] = 1.0
    docs = np.zeros((nd, d), np.float32)
    docs[:, 0] = r.integers(0, 21, nd) / 16.0
    docs[:, 1] = 1.0  # orthogonal to the query
    idx = np.empty((nq, k), np.int32)
    val = np.empty((nq, k), np.float32)
    N.check(ctx.h, N.lib().fa_similarities_topk(ctx.h, N.ptr(q), nq, N.ptr(docs), nd, d, k, N.ptr(idx), N.ptr(val)))
    s = docs[:, 0]
    want = np.lexsort((np.arange(nd), -s))[:k]
    for i in range(nq):
        assert idx[i].tolist() == want.tolist(), (nd, k, i)
        assert np.array_equal(val[i], s[want])


def test_topk_query_limit(ctx):
    q = np.zeros((1, 4), np.float32)
    docs = np.ones((8, 4), np.float32)
    idx = np.empty((1, 1), np.int32)
    rc = N.lib().fa_similarities_topk_dev(ctx.h, N.ptr(q), 65536, N.ptr(docs), 8, 4, 1, N.ptr(idx), N.ptr(idx))
    assert rc != 0


def test_similarities_topk_dev_fresh_context():
    """The device-pointer entry point as the first call of a fresh context
    (its scoring and candidate buffers are both taken on that call), twice,
    against the oracle's top-10."""
    c = N.Context(0)
    L = N.lib()
    r = rng(21)
    nq, nd, d, k = 64, 20000, 768, 10
    q = r.standard_normal((nq, d)).astype(np.float32)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    docs = r.standard_normal((nd, d)).astype(np.float32)
    docs /= np.linalg.norm(docs, axis=1, keepdims=True)
    ptrs = [C.c_void_p() for _ in range(4)]
    try:
        for p, n in zip(ptrs, (q.nbytes, docs.nbytes, nq * k * 4, nq * k * 4)):
            N.check(c.h, L.fa_device_alloc(c.h, n, C.byref(p)))
        dq, dd, di, dv = ptrs
        N.check(c.h, L.fa_memcpy_h2d(c.h, dq, q.ctypes.data, q.nbytes))
        N.check(c.h, L.fa_memcpy_h2d(c.h, dd, docs.ctypes.data, docs.nbytes))
        oi, ov = O.similarities_topk(q, docs, k)
        for _ in range(2):
            N.check(c.h, L.fa_similarities_topk_dev(c.h, dq, nq, dd, nd, d, k, di, dv))
            idx = np.empty((nq, k), np.int32)
            val = np.empty((nq, k), np.float32)
            N.check(c.h, L.fa_memcpy_d2h(c.h, idx.ctypes.data, di, idx.nbytes))
            N.check(c.h, L.fa_memcpy_d2h(c.h, val.ctypes.data, dv, val.nbytes))
            c.sync()
            s64 = q.astype(np.float64) @ docs.T.astype(np.float64)
            for i in range(nq):
                if not np.array_equal(idx[i], oi[i]):
                    assert np.allclose(s64[i, idx[i]], s64[i, oi[i]], atol=1e-6), (i, idx[i], oi[i])
            assert np.abs(val - ov).max() <= 1e-5
    finally:
        for p in ptrs:
            if p.value:
                L.fa_device_free(c.h, p)
        c.close()


# ---- the MFMA path of fa_attention (head dims 64, 128, 256, 512) -----------------

@pytest.mark.parametrize("D", [64, 128, 256, 512])
@pytest.mark.parametrize("B,H,Hkv,Tq,Sk", [(2, 4, 4, 70, 70), (1, 3, 1, 130, 33), (2, 2, 1, 17, 200)])
def test_attention_mfma_vs_oracle(ctx, D, B, H, Hkv, Tq, Sk):
    """fa_attention's MFMA kernel against the oracle (the reference's
    AttentionBlock algebra) at the reference's 1e-4 bar
    (tensor/attention_test.go:64-91): GQA as stride-0 head views (Expand),
    padding masks [B,1,1,S], window and causal masks [T,S] broadcast over
    batch and head, T != S, lengths that are not whole tiles."""
    r = rng(D * 7 + B * H + Tq + Sk)
    q = r.standard_normal((B, H, Tq, D)).astype(np.float32)
    k1 = r.standard_normal((B, Hkv, Sk, D)).astype(np.float32)
    v1 = r.standard_normal((B, Hkv, Sk, D)).astype(np.float32)
    assert Hkv in (1, H)
    k = np.broadcast_to(k1, (B, H, Sk, D))  # head stride 0 when Hkv == 1 (the reference's Expand)
    v = np.broadcast_to(v1, (B, H, Sk, D))
    lengths = [Sk] + [max(1, Sk // 3)] * (B - 1)
    masks = [None, T.PaddingMask(lengths, Sk)]
    if Tq == Sk:
        masks.append(T.WindowMask(Tq, 9).reshape(1, 1, Tq, Tq))
        masks.append(T.CausalMask(Tq))
    for mask in masks:
        for scale in (1.0 / np.sqrt(D), -0.03):
            got = T.AttentionScaled(q, k, v, mask, scale, ctx=ctx)
            want = O.attention(q, k, v, mask, scale)
            close(got, want, what=f"MFMA attention D={D} B={B} H={H}/{Hkv} T={Tq} S={Sk} "
                                  f"mask={None if mask is None else mask.shape} scale={scale:.3g}")


def test_attention_mfma_masked_weights_are_exact_zeros(ctx):
    """tensor/attention_test.go:266-285 on the MFMA path (D = 64): causal
    position 0 reproduces v[0], and keys behind the mask carry weight exactly
    0 (values of 1e30 there change nothing)."""
    r = rng(12)
    n, d = 64, 64
    q, k, v = (r.standard_normal((1, 1, n, d)).astype(np.float32) for _ in range(3))
    out = T.Attention(q, k, v, T.CausalMask(n), ctx=ctx)
    assert np.abs(out[0, 0, 0] - v[0, 0, 0]).max() <= 1e-6
    lengths = [40]
    pad = T.PaddingMask(lengths, n)
    base = T.Attention(q, k, v, pad, ctx=ctx)
    vv = v.copy()
    vv[:, :, 40:] = 1e30
    got = T.Attention(q, k, vv, pad, ctx=ctx)
    assert np.isfinite(got).all()
    assert np.array_equal(got, base)


def test_attention_mfma_dev_entry_point(ctx):
    """fa_attention_dev on device buffers equals fa_attention (host)."""
    r = rng(13)
    B, H, Tq, D = 2, 3, 96, 128
    q, k, v = (r.standard_normal((B, H, Tq, D)).astype(np.float32) for _ in range(3))
    want = T.AttentionScaled(q, k, v, None, 0.1, ctx=ctx)
    L = N.lib()
    ptrs = []
    for a in (q, k, v, np.empty_like(q)):
        p = C.c_void_p()
        N.check(ctx.h, L.fa_device_alloc(ctx.h, a.nbytes, C.byref(p)))
        N.check(ctx.h, L.fa_memcpy_h2d(ctx.h, p, a.ctypes.data, a.nbytes))
        ptrs.append(p)
    st = Tq * D
    N.check(ctx.h, L.fa_attention_dev(ctx.h, ptrs[0], ptrs[1], ptrs[2], B, H, Tq, Tq, D, H * st, st, H * st, st, H * st,
                                      st, None, 0, 0, 0, 0, 0.1, ptrs[3]))
    got = np.empty_like(q)
    N.check(ctx.h, L.fa_memcpy_d2h(ctx.h, got.ctypes.data, ptrs[3], got.nbytes))
    for p in ptrs:
        L.fa_device_free(ctx.h, p)
    assert np.array_equal(got, want)
