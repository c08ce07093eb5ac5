"""The CPU oracle of the cluster package (cluster/cluster.go) pinned on the CPU.

* Go's math/rand/v2 PCG (the generator cluster.KMeans seeds, cluster.go:47):
  its 128-bit LCG step against numpy's independent PCG64 with Go's
  multiplier/increment state, its DXSM output against numpy's PCG64DXSM,
  and the first eight draws of NewPCG(1, 2) against the known-answer list
  of Go's src/math/rand/v2/pcg_test.go (TestPCG). IntN (Lemire's
  multiply-shift with rejection) and Float64 against big-integer and exact
  closed forms.
* Normalize and Nearest against float64 numpy.
* KMeans: the reference's own test (TestKMeansRecoversPlantedClusters,
  cluster_test.go:28-65) restated; Lloyd fixed-point invariants at
  convergence (centres = normalised sums of their rows, sizes = counts,
  similarity = row . centre, assignment = argmax); k-means++ properties (k = n
  picks every distinct row once; when every weight is zero the pick is row
  0; the second pick's frequencies follow the squared cosine distance); the
  empty-centre restart on rows with one nonzero dyadic coordinate, where
  every step is exact and the result is fixed by hand.
"""
import math

import numpy as np
import pytest

import oracle_lib as O

M64 = (1 << 64) - 1
GO_INC = (6364136223846793005 << 64) | 1442695040888963407


def go_pcg_via_numpy(s1, s2, count):
    """Go's Uint64 stream composed from numpy's PCG64 (the LCG step) and
    PCG64DXSM (whose output is DXSM of its current state)."""
    state = (s1 << 64) | s2
    lcg, dx = np.random.PCG64(), np.random.PCG64DXSM()
    out = []
    for _ in range(count):
        lcg.state = {"bit_generator": "PCG64", "state": {"state": state, "inc": GO_INC}, "has_uint32": 0,
                     "uinteger": 0}
        lcg.random_raw(1)
        state = lcg.state["state"]["state"]
        dx.state = {"bit_generator": "PCG64DXSM", "state": {"state": state, "inc": 1}, "has_uint32": 0,
                    "uinteger": 0}
        out.append(int(dx.random_raw(1)[0]))
    return out


@pytest.mark.parametrize("s1,s2", [(1, 2), (7, 7 ^ 0x9e3779b97f4a7c15), (0, 0), (M64, M64), (12345, 0)])
def test_pcg_matches_numpy_lcg_and_dxsm(s1, s2):
    got = [int(v) for v in O.pcg_uint64s(s1, s2, 64)]
    assert got == go_pcg_via_numpy(s1, s2, 64)


def test_pcg_go_known_answers():
    want = [0xc4f5a58656eef510, 0x9dcec3ad077dec6c, 0xc8d04605312f8088, 0xcbedc0dcb63ac19a,
            0x3bf98798cae97950, 0xa8c6d7f8d485abc, 0x7ffa3780429cd279, 0x730ad2626b1c2f8e]
    assert [int(v) for v in O.pcg_uint64s(1, 2, 8)] == want


def intn_ref(stream, n):
    """Rand.uint64n over an iterator of Uint64 draws, in big integers."""
    if n & (n - 1) == 0:
        return next(stream) & (n - 1)
    m = next(stream) * n
    if (m & M64) < n:
        thresh = ((1 << 64) - n) % n
        while (m & M64) < thresh:
            m = next(stream) * n
    return m >> 64


@pytest.mark.parametrize("n", [1, 2, 3, 7, 600, 1024, 50000, (1 << 40) + 3, (1 << 63) + 12345, M64])
def test_intn_closed_form(n):
    count = 300
    got = [int(v) for v in O.pcg_intns(5, 9, n, count)]
    stream = iter(int(v) for v in O.pcg_uint64s(5, 9, 10 * count))
    want = [intn_ref(stream, n) for _ in range(count)]
    assert got == want
    assert all(0 <= v < n for v in got)


def test_intn_uniform():
    v = O.pcg_intns(3, 4, 600, 60000).astype(np.int64)
    counts = np.bincount(v, minlength=600)
    chi2 = ((counts - 100.0) ** 2 / 100.0).sum()
    assert abs(chi2 - 599) < 6 * math.sqrt(2 * 599)


def test_float64_closed_form():
    u = [int(v) for v in O.pcg_uint64s(11, 12, 1000)]
    f = O.pcg_float64s(11, 12, 1000)
    want = np.array([(v & ((1 << 53) - 1)) / float(1 << 53) for v in u])
    assert np.array_equal(f, want)
    assert (f >= 0).all() and (f < 1).all()


def test_normalize_closed_form():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((50, 33)).astype(np.float32) * rng.uniform(0.01, 100, (50, 1)).astype(np.float32)
    x[7] = 0
    y = O.cluster_normalize(x)
    xd = x.astype(np.float64)
    nrm = np.sqrt((xd * xd).sum(1, keepdims=True))
    nrm[nrm == 0] = 1
    np.testing.assert_allclose(y, xd / nrm, rtol=0, atol=1e-6)
    assert (y[7] == 0).all()


def test_nearest_brute_force():
    rng = np.random.default_rng(2)
    x = O.cluster_normalize(rng.standard_normal((300, 40)).astype(np.float32))
    c = O.cluster_normalize(rng.standard_normal((9, 40)).astype(np.float32))
    c[5] = c[2]  # equal scores: the first index wins
    idx, sim = O.cluster_nearest(x, c)
    s = x.astype(np.float64) @ c.astype(np.float64).T
    srt = np.sort(s, 1)
    clear = srt[:, -1] - srt[:, -2] > 1e-5
    assert (idx[clear] == s.argmax(1)[clear]).all()
    assert not (idx == 5).any()
    np.testing.assert_allclose(sim, s[np.arange(300), idx], atol=1e-6)


def planted(rng, n, d, groups=3, noise=0.05):
    """cluster_test.go:12-26: rows around well-separated unit centres."""
    cd = O.cluster_normalize(rng.standard_normal((groups, d)).astype(np.float32))
    truth = np.arange(n) % groups
    data = cd[truth] + (rng.standard_normal((n, d)) * noise).astype(np.float32)
    return O.cluster_normalize(data.astype(np.float32)), truth


def inertia(sim):
    return sum(1 - float(v) for v in sim) / len(sim)


def test_kmeans_recovers_planted_clusters():
    """TestKMeansRecoversPlantedClusters (cluster_test.go:28-65) restated."""
    rng = np.random.default_rng(12)
    x, truth = planted(rng, 600, 64)
    r = O.cluster_kmeans(x, 3, 20, 7)
    mapping = {}
    for g, a in zip(truth.tolist(), r["assignment"].tolist()):
        assert mapping.setdefault(g, a) == a, "group split between centres"
    assert len(set(mapping.values())) == 3, "groups merged"
    assert (r["similarity"] >= 0.85).all()
    idx, sim = O.cluster_nearest(x[:3], r["centres"])
    assert (sim >= 0.85).all() and (idx == r["assignment"][:3]).all()
    _, sim = O.cluster_nearest(O.cluster_normalize(rng.standard_normal((1, 64)).astype(np.float32)), r["centres"])
    assert sim[0] <= 0.6
    assert inertia(r["similarity"]) <= 0.1


def test_kmeans_fixed_point_invariants():
    rng = np.random.default_rng(4)
    x, _ = planted(rng, 400, 16, groups=5, noise=0.2)
    r = O.cluster_kmeans(x, 5, 100, 3)
    assert 1 < r["iterations"] < 100  # converged: the last round changed nothing
    a, c = r["assignment"], r["centres"].astype(np.float64)
    assert (r["sizes"] == np.bincount(a, minlength=5)).all()
    xd = x.astype(np.float64)
    for j in range(5):
        s = xd[a == j].sum(0)
        np.testing.assert_allclose(c[j], s / np.linalg.norm(s), atol=1e-6)
    s = xd @ c.T
    np.testing.assert_allclose(r["similarity"], s[np.arange(400), a], atol=1e-6)
    srt = np.sort(s, 1)
    clear = srt[:, -1] - srt[:, -2] > 1e-5
    assert (a[clear] == s.argmax(1)[clear]).all()


def test_kmeans_plus_plus_takes_every_row_when_k_is_n():
    rng = np.random.default_rng(5)
    x = O.cluster_normalize(rng.standard_normal((12, 6)).astype(np.float32))
    r = O.cluster_kmeans(x, 12, 1, 99)
    assert sorted(r["chosen"].tolist()) == list(range(12))
    assert (r["sizes"] == 1).all()


def test_kmeans_plus_plus_zero_total_picks_row_zero():
    e = np.eye(3, dtype=np.float32)
    x = np.stack([e[1], e[1], e[2]])  # two distinct rows; k = 3 forces a pick with every weight 0
    for seed in range(5):
        r = O.cluster_kmeans(x, 3, 0, seed)
        assert r["chosen"][2] == 0
        assert set(r["chosen"][:2].tolist()) in ({0, 2}, {1, 2})


def test_kmeans_plus_plus_weights_are_squared_distances():
    # rows e0, e1, -e0: with e0 first, the second pick has weights 0, 1, 4
    e = np.eye(2, dtype=np.float32)
    x = np.stack([e[0], e[1], -e[0]])
    picks = []
    for seed in range(3000):
        r = O.cluster_kmeans(x, 2, 0, seed)
        if r["chosen"][0] == 0:
            picks.append(r["chosen"][1])
    picks = np.array(picks)
    p = (picks == 2).mean()
    assert abs(p - 0.8) < 4 * math.sqrt(0.16 / len(picks)), p
    assert not (picks == 0).any()


def basis_rows():
    """Rows with one nonzero dyadic coordinate: every product and sum of the
    algorithm on them is exact."""
    e = np.eye(4, dtype=np.float32)
    return np.stack([e[0], e[0], e[1], 0.5 * e[1], e[2], e[3], 0.25 * e[3], 0.5 * e[0]]).astype(np.float32)


def test_kmeans_empty_centre_restart_by_hand():
    x = basis_rows()
    r = O.cluster_kmeans(x, 4, 1, 0)
    # seeding (fixed by the PCG stream): rows 4 (e2), 6 (e3/4), 2 (e1), 6 again
    assert r["chosen"].tolist() == [4, 6, 2, 6]
    # first iteration: centres e2, e3, e1, e3; e0 rows score 0 everywhere -> centre 0
    assert r["assignment"].tolist() == [0, 0, 2, 2, 0, 1, 1, 0]
    assert r["sizes"].tolist() == [4, 2, 2, 0]
    # centre 3 restarts on the worst row: row 0 (similarity 0, first of the
    # minima), whose similarity becomes 1
    assert r["similarity"].tolist() == [1.0, 0.0, 1.0, 0.5, 1.0, 1.0, 0.25, 0.0]
    s0 = x[0] + x[1] + x[4] + x[7]
    want = np.stack([s0 / np.linalg.norm(s0), np.eye(4)[3], np.eye(4)[1], np.eye(4)[0]]).astype(np.float32)
    np.testing.assert_array_equal(r["centres"], want)


def test_kmeans_errors_and_zero_iterations():
    x = basis_rows()
    with pytest.raises(ValueError):
        O.cluster_kmeans(x, 0, 5, 1)
    with pytest.raises(ValueError):
        O.cluster_kmeans(x, 9, 5, 1)
    r = O.cluster_kmeans(x, 3, 0, 1)
    assert r["iterations"] == 0 and (r["assignment"] == 0).all() and (r["sizes"] == 0).all()
    np.testing.assert_array_equal(r["centres"], O.cluster_normalize(x[r["chosen"]]))
