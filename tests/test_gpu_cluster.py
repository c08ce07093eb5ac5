"""cluster on the GPU (fa_cluster_*: Normalize, Nearest, KMeans) against the
CPU oracle (oracle/fa_oracle.cpp, pinned by tests/test_cluster_oracle.py).

Bars: Normalize within 1e-6; Nearest's index identical wherever the float64
top-2 margin exceeds 1e-5, similarity within 1e-5; KMeans on well-separated
planted data identical in assignment, sizes and iterations, centres and
similarities within 1e-5 (the seeding's picks depend on the data only
through products that differ by rounding); KMeans on rows with one nonzero
dyadic coordinate (every step exact, empty-centre restarts included)
bit-identical.
"""
import time

import numpy as np
import pytest

import oracle_lib as O
from ai_amd import cluster as CL
from ai_amd.tensor import TensorError

pytestmark = pytest.mark.gpu


def unit_rows(rng, n, d):
    return O.cluster_normalize(rng.standard_normal((n, d)).astype(np.float32))


def planted(rng, n, d, groups, noise):
    cd = unit_rows(rng, groups, d)
    truth = np.arange(n) % groups
    data = cd[truth] + (rng.standard_normal((n, d)) * noise).astype(np.float32)
    return O.cluster_normalize(data.astype(np.float32)), truth


def basis_rows():
    e = np.eye(4, dtype=np.float32)
    return np.stack([e[0], e[0], e[1], 0.5 * e[1], e[2], e[3], 0.25 * e[3], 0.5 * e[0]]).astype(np.float32)


def test_normalize():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1000, 768)).astype(np.float32) * rng.uniform(0.01, 50, (1000, 1)).astype(np.float32)
    x[3] = 0
    got = CL.Normalize(x)
    np.testing.assert_allclose(got, O.cluster_normalize(x), rtol=0, atol=1e-6)
    assert (got[3] == 0).all()
    assert CL.Normalize(np.zeros((0, 5), np.float32)).shape == (0, 5)


@pytest.mark.parametrize("n,k,d", [(20000, 40, 768), (777, 3, 64), (64, 1, 9), (300, 130, 33)])
def test_nearest(n, k, d):
    rng = np.random.default_rng(n + k)
    x, c = unit_rows(rng, n, d), unit_rows(rng, k, d)
    print(f"nearest n={n} k={k} d={d}", flush=True)
    idx, sim = CL.Nearest(x, c)
    oi, osim = O.cluster_nearest(x, c)
    s = x.astype(np.float64) @ c.astype(np.float64).T
    if k > 1:
        srt = np.sort(s, 1)
        clear = srt[:, -1] - srt[:, -2] > 1e-5
    else:
        clear = np.ones(n, bool)
    assert (idx[clear] == oi[clear]).all()
    np.testing.assert_allclose(sim, osim, atol=1e-5)


def test_nearest_equal_scores_take_the_first_centre():
    e = np.eye(4, dtype=np.float32)
    c = np.stack([e[1], e[0], e[2], e[0], e[1]])
    idx, sim = CL.Nearest(basis_rows(), c)
    oi, osim = O.cluster_nearest(basis_rows(), c)
    assert idx.tolist() == oi.tolist() == [1, 1, 0, 0, 2, 0, 0, 1]
    np.testing.assert_array_equal(sim, osim)


def compare_kmeans(x, k, iters, seed, atol):
    print(f"kmeans n={x.shape[0]} d={x.shape[1]} k={k} iters={iters} seed={seed}", flush=True)
    g = CL.KMeans(x, k, iters, seed)
    o = O.cluster_kmeans(x, k, iters, seed)
    assert g.Iterations == o["iterations"]
    assert (g.Assignment == o["assignment"]).all()
    assert (g.Sizes == o["sizes"]).all()
    if atol == 0:
        np.testing.assert_array_equal(g.Centres, o["centres"])
        np.testing.assert_array_equal(g.Similarity, o["similarity"])
    else:
        np.testing.assert_allclose(g.Centres, o["centres"], rtol=0, atol=atol)
        np.testing.assert_allclose(g.Similarity, o["similarity"], rtol=0, atol=atol)
    return g


def test_kmeans_recovers_planted_clusters():
    """TestKMeansRecoversPlantedClusters (cluster_test.go:28-65) on the GPU,
    and identical to the oracle."""
    rng = np.random.default_rng(12)
    x, truth = planted(rng, 600, 64, 3, 0.05)
    r = compare_kmeans(x, 3, 20, 7, 1e-5)
    mapping = {}
    for g, a in zip(truth.tolist(), r.Assignment.tolist()):
        assert mapping.setdefault(g, a) == a
    assert len(set(mapping.values())) == 3
    assert (r.Similarity >= 0.85).all()
    idx, sim = CL.Nearest(x[:3], r.Centres)
    assert (sim >= 0.85).all() and (idx == r.Assignment[:3]).all()
    _, sim = CL.Nearest(unit_rows(rng, 1, 64), r.Centres)
    assert sim[0] <= 0.6
    assert r.Inertia() <= 0.1


@pytest.mark.parametrize("n,d,k,iters,seed", [(20000, 768, 40, 10, 3), (5000, 128, 200, 8, 11), (3000, 33, 7, 30, 5),
                                               (300000, 8, 4, 5, 21)])
def test_kmeans_matches_oracle(n, d, k, iters, seed):
    rng = np.random.default_rng(seed)
    x, _ = planted(rng, n, d, k, 0.3 / np.sqrt(d) * 8)
    compare_kmeans(x, k, iters, seed, 1e-5)


@pytest.mark.parametrize("k", [4, 5, 6, 8])
@pytest.mark.parametrize("seed", [0, 1, 2, 17])
def test_kmeans_exact_with_empty_centres(k, seed):
    compare_kmeans(basis_rows(), k, 10, seed, 0)


def test_kmeans_zero_iterations_and_errors():
    x = basis_rows()
    compare_kmeans(x, 3, 0, 1, 0)
    with pytest.raises(CL.ClusterError):
        CL.KMeans(x, 0, 5, 1)
    with pytest.raises(CL.ClusterError):
        CL.KMeans(x, 9, 5, 1)
    with pytest.raises(TensorError):
        CL.Nearest(x, np.zeros((0, 4), np.float32))


def test_cosine_and_similarities():
    """TestCosine and TestSimilarities (cluster_test.go:88-132) restated."""
    a = [1, 2, 3, 4]
    assert abs(CL.Cosine(a, a) - 1) <= 1e-6
    assert abs(CL.Cosine(a, [-1, -2, -3, -4]) + 1) <= 1e-6
    assert CL.Cosine([1, 0], [0, 1]) == 0
    assert CL.Cosine(a, [0, 0, 0, 0]) == 0
    assert CL.Cosine([], []) == 0
    rng = np.random.default_rng(9)
    for n in (1, 7, 8, 9, 768, 1001):
        x, y = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
        xd, yd = x.astype(np.float64), y.astype(np.float64)
        want = (xd @ yd) / np.sqrt((xd @ xd) * (yd @ yd))
        assert abs(CL.Cosine(x, y) - want) <= 1e-5
    with pytest.raises(CL.ClusterError):
        CL.Cosine([1, 2], [1])
    q, dm = unit_rows(rng, 5, 64), unit_rows(rng, 7, 64)
    s = CL.Similarities(q, dm)
    assert s.shape == (5, 7)
    for i in range(5):
        for j in range(7):
            assert abs(s[i, j] - CL.Cosine(q[i], dm[j])) <= 1e-5
    with pytest.raises(CL.ClusterError):
        CL.Similarities(q, unit_rows(rng, 7, 63))


def test_nearest_and_kmeans_speed():
    """TestNearestSpeed (cluster_test.go:67-84): 50 000 x 768 against 40
    centres; the reference bounds one call at 200 ms on its CPU."""
    rng = np.random.default_rng(0)
    x, c = unit_rows(rng, 50000, 768), unit_rows(rng, 40, 768)
    CL.Nearest(x, c)
    t = time.perf_counter()
    CL.Nearest(x, c)
    el = time.perf_counter() - t
    print(f"Nearest 50000x768 vs 40 (host arrays, PCIe included): {el * 1e3:.1f} ms", flush=True)
    assert el < 0.2
    t = time.perf_counter()
    r = CL.KMeans(x, 40, 20, 1)
    print(f"KMeans 50000x768 k=40 iters={r.Iterations}: {(time.perf_counter() - t) * 1e3:.1f} ms", flush=True)
