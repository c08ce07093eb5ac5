"""End-to-end parity of the GPU encoder (libfa_rocm.so) with the CPU oracle.

Bar: cosine >= 0.9999 per sentence, top-1
nearest-neighbour indices identical; max |delta| printed.
"""
import numpy as np
import pytest

import oracle_lib as O
from ai_amd import gemma as G
from ai_amd import synth as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def models(ctx):
    shape = S.ModelShape()
    gm = G.Model(shape, ctx)
    gm.load_synthetic()
    om = O.OracleModel(shape)
    om.load_synthetic()
    yield gm, om
    gm.close()
    om.close()


def cos_rows(a, b):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return (a * b).sum(1) / (np.linalg.norm(a, axis=1) * np.linalg.norm(b, axis=1) + 1e-12)


def compare(gpu, ref, what):
    c = cos_rows(gpu, ref)
    d = np.abs(gpu.astype(np.float64) - ref).max()
    nn_g = (gpu.astype(np.float64) @ gpu.T.astype(np.float64))
    nn_r = (ref.astype(np.float64) @ ref.T.astype(np.float64))
    np.fill_diagonal(nn_g, -np.inf)
    np.fill_diagonal(nn_r, -np.inf)
    top1_g, top1_r = nn_g.argmax(1), nn_r.argmax(1)
    print(f"{what}: cosine min={c.min():.8f} mean={c.mean():.8f} max|d|={d:.3g} top1 equal={np.array_equal(top1_g, top1_r)}",
          flush=True)
    assert c.min() >= 0.9999
    if gpu.shape[0] > 2:
        assert np.array_equal(top1_g, top1_r)
    return c


def test_c1(models):
    gm, om = models
    b = S.make_batch("C1")
    compare(gm.embed_ids(b.ids, b.lengths), om.embed(b.ids, b.lengths), "C1")


def test_c2_subset(models):
    """C2 (32 x 256, ragged): the first 8 and the last 4 sequences through
    the oracle (each sequence's embedding does not depend on the others,
    gemma_test.go:117-135). At 5 517 tokens the GPU runs the batch as three
    micro-batches on three streams; these rows come from the first and the
    last."""
    gm, om = models
    b = S.make_batch("C2")
    got = gm.embed_ids(b.ids, b.lengths)
    for sub in (slice(0, 8), slice(28, 32)):
        Tm = int(b.lengths[sub].max())
        ref = om.embed(b.ids[sub, :Tm], b.lengths[sub])
        compare(got[sub], ref, f"C2[{sub.start}:{sub.stop}]")


def test_batch_and_padding_invariance(models):
    """A sequence's embedding is the same alone or batched with longer ones."""
    gm, _ = models
    b = S.make_batch("C2")
    full = gm.embed_ids(b.ids, b.lengths)
    for i in (0, 5, 17):
        L = int(b.lengths[i])
        alone = gm.embed_ids(b.ids[i:i + 1, :L], b.lengths[i:i + 1])
        c = cos_rows(alone, full[i:i + 1])
        assert c.min() >= 0.9999


@pytest.mark.parametrize("lengths", [[2000, 7, 300], [1500, 1500], [40] * 60 + [2048]])
def test_microbatch_groups_match_single_sequences(models, lengths):
    """From 2 048 tokens a batch runs as two to four token-balanced groups
    of sequences on their own streams; with one dominant sequence, two sequences
    or many short ones every sequence's embedding still equals its
    single-sequence run, and the shortest one the oracle's."""
    gm, om = models
    rng = np.random.default_rng(len(lengths))
    T = max(lengths)
    lens = np.array(lengths, np.int32)
    ids = rng.integers(3, 262144, (len(lens), T)).astype(np.int32)
    ids[:, 0] = 2
    ids[np.arange(T)[None, :] >= lens[:, None]] = 0
    full = gm.embed_ids(ids, lens)
    for i in sorted(set([0, len(lens) - 1, int(np.argmin(lens))])):
        L = int(lens[i])
        alone = gm.embed_ids(ids[i:i + 1, :L], lens[i:i + 1])
        assert cos_rows(alone, full[i:i + 1]).min() >= 0.99999, (lengths, i)
    i = int(np.argmin(lens))
    L = int(lens[i])
    compare(full[i:i + 1], om.embed(ids[i:i + 1, :L], lens[i:i + 1]), f"groups {lengths[:3]}.. [{i}]")
    # Matryoshka truncation on the micro-batched path (embed.go:421-427)
    d256 = gm.embed_ids(ids, lens, dim=256).astype(np.float64)
    want = full[:, :256].astype(np.float64)
    want /= np.linalg.norm(want, axis=1, keepdims=True)
    np.testing.assert_allclose(d256, want, atol=2e-6)


def test_dim_truncation(models):
    """Matryoshka Dim: truncation before L2 (embed.go:421-427)."""
    gm, om = models
    b = S.make_batch("C1")
    g = gm.embed_ids(b.ids, b.lengths, dim=256)
    r = om.embed(b.ids, b.lengths, dim=256)
    assert g.shape == (1, 256)
    assert abs(np.linalg.norm(g) - 1) < 1e-5
    assert cos_rows(g, r).min() >= 0.9999
    with pytest.raises(G.GemmaError):
        gm.embed_ids(b.ids, b.lengths, dim=769)


def test_bad_inputs(models):
    gm, _ = models
    ids = np.full((1, 4), 5, np.int32)
    with pytest.raises(G.GemmaError):
        gm.embed_ids(ids, np.array([5], np.int32))  # length > T
    with pytest.raises(G.GemmaError):
        gm.embed_ids(np.full((1, 4), 262144, np.int32), np.array([4], np.int32))  # id out of range
    with pytest.raises(G.GemmaError):
        gm.embed_ids(ids, np.array([0], np.int32))


def test_c3_sliding_band(models):
    """C3 (64 x 512, all full length): T = 512 > 257, so the 20 sliding layers
    mask |i-j| >= 257 (embed.go:169-172,183-186) and differ from the global
    ones. All 64 on the GPU, the first 4 through the oracle."""
    gm, om = models
    b = S.make_batch("C3")
    got = gm.embed_ids(b.ids, b.lengths)
    assert np.allclose(np.linalg.norm(got, axis=1), 1, atol=1e-5)
    ref = om.embed(b.ids[:4], b.lengths[:4])
    compare(got[:4], ref, "C3[0:4]")


def test_key_split_attention_with_sliding_band(models):
    """Two full 512-token sequences (1 024 tokens on one stream, 96
    attention items): the attention cuts each item's keys into runs (the
    key-split path) while the 20 sliding layers mask |i-j| >= 257. The
    first sequence against the oracle, both against their rows in C3's
    64-sequence batch (no key split)."""
    gm, om = models
    b = S.make_batch("C3")
    two = gm.embed_ids(b.ids[:2], b.lengths[:2])
    compare(two[:1], om.embed(b.ids[:1], b.lengths[:1]), "C3[0] key-split")
    full = gm.embed_ids(b.ids, b.lengths)
    assert cos_rows(two, full[:2]).min() >= 0.99999


def test_c4_long_sequences(models):
    """C4 (8 x 2048, lengths 1024..2048): the GPU batch against the oracle for
    the shortest sequence (band active, far beyond one attention tile)."""
    gm, om = models
    b = S.make_batch("C4")
    got = gm.embed_ids(b.ids, b.lengths)
    i = int(np.argmin(b.lengths))
    L = int(b.lengths[i])
    ref = om.embed(b.ids[i:i + 1, :L], b.lengths[i:i + 1])
    compare(got[i:i + 1], ref, f"C4[{i}] L={L}")
    # the other sequences: unit norm and batch invariance against a single-sequence run
    j = int(np.argmax(b.lengths))
    alone = gm.embed_ids(b.ids[j:j + 1, :int(b.lengths[j])], b.lengths[j:j + 1])
    assert cos_rows(alone, got[j:j + 1]).min() >= 0.9999


def _topk_agree(q, docs, gi, oi, k, what):
    """Top-k index lists agree wherever the float64 scores leave no near-tie
    (gap > 1e-5 among the k+1 best); elsewhere the GPU's list must still be a
    valid top-k within that tolerance. Ties order by lower index
    (reduce.go:286-289)."""
    s = q.astype(np.float64) @ docs.astype(np.float64).T
    srt = -np.sort(-s, axis=1)[:, :k + 1]
    gaps = np.diff(-srt, axis=1).min(1)
    clear = gaps > 1e-5
    assert np.array_equal(gi[clear], oi[clear]), what
    kth = srt[:, k - 1]
    got_scores = np.take_along_axis(s, gi.astype(np.int64), 1)
    assert (got_scores.min(1) >= kth - 1e-5).all(), what
    print(f"{what}: {int(clear.sum())}/{len(clear)} rows without near-ties, all identical", flush=True)
    return clear


def test_c5_scoring_top10(models, ctx):
    """C5 (256 x 128 ragged) + scoring against 100 000 unit docs: embeddings
    vs the oracle on 8 queries; GPU top-10 (fa_similarities_topk) vs the
    oracle's top-10 on the same queries, and end to end from the oracle's own
    embeddings of those 8."""
    from ai_amd import _native as N
    gm, om = models
    b = S.make_batch("C5")
    q = gm.embed_ids(b.ids, b.lengths)
    sub = slice(0, 8)
    Tm = int(b.lengths[sub].max())
    ref = om.embed(b.ids[sub, :Tm], b.lengths[sub])
    compare(q[sub], ref, "C5[0:8]")
    docs = b.corpus
    k = 10
    idx = np.empty((q.shape[0], k), np.int32)
    val = np.empty((q.shape[0], k), np.float32)
    N.check(ctx.h, N.lib().fa_similarities_topk(ctx.h, N.ptr(q), q.shape[0], N.ptr(docs), docs.shape[0], 768, k,
                                                N.ptr(idx), N.ptr(val)))
    nq = 64
    oi, ov = O.similarities_topk(q[:nq], docs, k)
    clear = _topk_agree(q[:nq], docs, idx[:nq], oi, k, "C5 scoring, same queries")
    assert clear.mean() >= 0.9
    assert np.allclose(val[:nq], ov, atol=1e-5)
    oi2, _ = O.similarities_topk(ref, docs, k)
    _topk_agree(ref, docs, idx[sub], oi2, k, "C5 scoring, oracle embeddings end to end")
