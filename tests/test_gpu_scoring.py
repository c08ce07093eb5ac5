"""The fused similarities + top-k path (score.hip: split-bf16 stage with lane
candidate lists, exact rescoring, exact fallback scan) through the C ABI.

cluster.Similarities (cluster/cluster.go:185-190) followed by a top-k with the
first-max tie rule of (*Tensor).Argmax (tensor/reduce.go:269-297). From 128
queries fa_similarities_topk takes the fused path, whose scores are the exact
dot products rounded to float32: the expected lists are the float64 products
rounded to float32, ordered by (value desc, index asc), with NaN scores below
every number and index -1 past a row's non-NaN scores.
"""
import numpy as np
import pytest

from ai_amd import _native as N

pytestmark = pytest.mark.gpu


def unit(a):
    return (a / np.linalg.norm(a, axis=1, keepdims=True)).astype(np.float32)


def topk_gpu(ctx, q, docs, k):
    nq, d = q.shape
    idx = np.full((nq, k), -7, np.int32)
    val = np.empty((nq, k), np.float32)
    N.check(ctx.h, N.lib().fa_similarities_topk(ctx.h, N.ptr(q), nq, N.ptr(docs), docs.shape[0], d, k, N.ptr(idx),
                                                N.ptr(val)))
    return idx, val


def expected(q, docs, k):
    s64 = q.astype(np.float64) @ docs.astype(np.float64).T
    s32 = s64.astype(np.float32)
    key = np.where(np.isnan(s32), -np.inf, s32)
    nd = docs.shape[0]
    idx = np.empty((q.shape[0], k), np.int64)
    for i in range(q.shape[0]):
        order = np.lexsort((np.arange(nd), -key[i]))[:k]
        order = np.where(np.isnan(s32[i, order]), -1, order)
        idx[i] = order
    return idx, s64, s32


def check(ctx, q, docs, k, what):
    gi, gv = topk_gpu(ctx, q, docs, k)
    wi, s64, s32 = expected(q, docs, k)
    bad = []
    for i in range(q.shape[0]):
        if not np.array_equal(gi[i], wi[i]):
            # a float64 product within rounding of a float32 midpoint may round
            # the other way than the GPU's: only exchanges of (nearly) equal
            # scores are allowed
            ok = (gi[i] >= 0).all() and np.allclose(s64[i, gi[i]], s64[i, wi[i]], rtol=0, atol=1e-12)
            if not ok:
                bad.append(i)
    assert not bad, (what, bad[:5], gi[bad[0]], wi[bad[0]])
    sel = gi >= 0
    rows = np.nonzero(sel)
    np.testing.assert_allclose(gv[rows], s32[rows[0], gi[rows]], rtol=0, atol=1e-7)
    assert np.isnan(gv[~sel]).all()
    print(f"{what}: {q.shape[0]} queries x {docs.shape[0]} docs, top-{k} identical to the rounded exact order",
          flush=True)
    return gi, gv


@pytest.mark.parametrize("k", [1, 10, 16])
def test_fused_exact_order(ctx, k):
    """300 queries (a full and a partial block of 256) against 20 013 docs
    (not a multiple of the 32-doc blocks), unit rows of width 768."""
    r = np.random.default_rng(100 + k)
    q = unit(r.standard_normal((300, 768)))
    docs = unit(r.standard_normal((20013, 768)))
    check(ctx, q, docs, k, f"fused k={k}")


def test_fused_duplicates_take_the_exact_fallback(ctx):
    """Forty copies of one doc at scattered and adjacent indices and a query
    equal to it: more than a lane list's four entries and the merge's sixteen
    tie at the top, so the exact fallback scan must order them by index."""
    r = np.random.default_rng(7)
    docs = unit(r.standard_normal((5000, 256)))
    dup = np.concatenate([np.arange(100, 120), r.choice(np.arange(200, 5000), 20, replace=False)])
    docs[dup] = docs[50]
    q = unit(r.standard_normal((130, 256)))
    q[3] = docs[50]
    q[77] = docs[50] * 0.5 + unit(r.standard_normal((1, 256)))[0] * 0.01
    gi, _ = check(ctx, q, docs, 16, "duplicates")
    assert gi[3].tolist() == sorted([50] + dup.tolist())[:16]


def test_fused_nan_rows_and_unnormalised_rows(ctx):
    """NaN docs are never selected; rows of other lengths (x3, x0.01) keep the
    exact order (the stage-1 error bound scales with |q| |doc|)."""
    r = np.random.default_rng(8)
    docs = unit(r.standard_normal((3000, 128)))
    docs[::7] *= 3.0
    docs[5::11] *= 0.01
    docs[[0, 13, 2999]] = np.nan
    q = unit(r.standard_normal((160, 128)))
    q[::5] *= 2.5
    check(ctx, q, docs, 10, "NaN / non-unit rows")


def test_fused_fewer_docs_than_a_tile(ctx):
    """37 docs: one partial 128-doc tile over two workgroups of one and two
    32-doc blocks; k = 16."""
    r = np.random.default_rng(9)
    docs = unit(r.standard_normal((37, 64)))
    q = unit(r.standard_normal((128, 64)))
    check(ctx, q, docs, 16, "37 docs")


def test_fused_all_nan_row_pads_with_minus_one(ctx):
    r = np.random.default_rng(10)
    docs = unit(r.standard_normal((40, 32)))
    docs[5:] = np.nan
    q = unit(r.standard_normal((128, 32)))
    gi, gv = check(ctx, q, docs, 8, "NaN beyond five docs")
    assert (gi[:, 5:] == -1).all() and np.isnan(gv[:, 5:]).all()


def test_fused_and_per_query_paths_agree(ctx):
    """The same 128 queries through the fused path and one at a time (the
    fp32-MFMA product and two-pass top-k): identical lists wherever the
    float64 scores leave no near-tie."""
    r = np.random.default_rng(11)
    docs = unit(r.standard_normal((30000, 768)))
    q = unit(r.standard_normal((128, 768)))
    fi, _ = topk_gpu(ctx, q, docs, 10)
    s64 = q.astype(np.float64) @ docs.astype(np.float64).T
    for i in range(0, 128, 8):
        oi, _ = topk_gpu(ctx, q[i:i + 1].copy(), docs, 10)
        srt = -np.sort(-s64[i])[:11]
        if np.diff(-srt).min() > 2e-6:
            assert fi[i].tolist() == oi[0].tolist(), i
