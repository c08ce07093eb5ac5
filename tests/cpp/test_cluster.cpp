// cluster package of the C++ host mirror (ai_amd/host/cluster.hpp) on the
// GPU, restating the reference's own tests (cluster/cluster_test.go, file:line
// of each below). Run by tests/test_cpp_host.py on an MI355X.
#include <chrono>
#include <cmath>
#include <map>
#include <random>

#include "cluster.hpp"
#include "testing.hpp"

using namespace fiber;
using tensor::Tensor;

static Tensor randn(std::mt19937_64& rng, int64_t n, int64_t d) {
  std::normal_distribution<double> nd(0.0, 1.0);
  std::vector<float> v((size_t)(n * d));
  for (auto& x : v) x = (float)nd(rng);
  return Tensor::New(std::move(v), {n, d});
}

// cluster_test.go:12-26: n rows around three well-separated unit vectors.
static Tensor planted(std::mt19937_64& rng, int n, int d, std::vector<int>* truth) {
  const std::vector<float> cd = cluster::Normalize(randn(rng, 3, d)).Float32s();
  std::normal_distribution<double> nd(0.0, 1.0);
  std::vector<float> data((size_t)n * d);
  truth->resize(n);
  for (int i = 0; i < n; i++) {
    const int g = i % 3;
    (*truth)[i] = g;
    for (int j = 0; j < d; j++) data[(size_t)i * d + j] = cd[(size_t)g * d + j] + (float)nd(rng) * 0.05f;
  }
  return cluster::Normalize(Tensor::New(std::move(data), {n, d}));
}

// cluster_test.go:28-65
TEST(TestKMeansRecoversPlantedClusters) {
  std::mt19937_64 rng(12);
  std::vector<int> truth;
  const Tensor x = planted(rng, 600, 64, &truth);
  const cluster::Result res = cluster::KMeans(x, 3, 20, 7);
  std::map<int, int> mapping;
  for (size_t i = 0; i < res.Assignment.size(); i++) {
    auto it = mapping.find(truth[i]);
    if (it != mapping.end() && it->second != res.Assignment[i])
      FATAL("group %d split between centres %d and %d", truth[i], it->second, res.Assignment[i]);
    mapping[truth[i]] = res.Assignment[i];
  }
  if (mapping.size() != 3) FATAL("groups merged: %zu centres", mapping.size());
  for (size_t i = 0; i < res.Similarity.size(); i++)
    if (res.Similarity[i] < 0.85f) FATAL("row %zu similarity %g to its centre", i, res.Similarity[i]);
  const std::vector<float> xv = x.Float32s();
  std::vector<float> first3(xv.begin(), xv.begin() + 3 * 64);
  auto [idx, sim] = cluster::Nearest(Tensor::New(first3, {3, 64}), res.Centres);
  for (int i = 0; i < 3; i++)
    if (sim[i] < 0.85f || idx[i] != res.Assignment[i]) FATAL("Nearest disagrees at %d: %d %g", i, idx[i], sim[i]);
  auto [ridx, rsim] = cluster::Nearest(cluster::Normalize(randn(rng, 1, 64)), res.Centres);
  (void)ridx;
  if (rsim[0] > 0.6f) FATAL("random vector too similar: %g", rsim[0]);
  if (res.Inertia() > 0.1) FATAL("inertia %g", res.Inertia());
  if (res.Iterations < 1 || res.Iterations > 20) FATAL("iterations %d", res.Iterations);
}

// cluster_test.go:67-84 (the reference bounds one call at 200 ms on its CPU)
TEST(TestNearestSpeed) {
  std::mt19937_64 rng(1);
  const Tensor x = cluster::Normalize(randn(rng, 50000, 768));
  const Tensor c = cluster::Normalize(randn(rng, 40, 768));
  cluster::Nearest(x, c);  // warm up
  const auto t0 = std::chrono::steady_clock::now();
  cluster::Nearest(x, c);
  const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  std::printf("    50 000 x 768 against 40 centres: %.1f ms (host arrays, PCIe included)\n", ms);
  if (ms > 200) FATAL("took %.1f ms", ms);
}

// cluster_test.go:86-116
TEST(TestCosine) {
  const std::vector<float> a = {1, 2, 3, 4};
  if (std::fabs(cluster::Cosine(a, a) - 1) > 1e-6) FATAL("same direction: %g", cluster::Cosine(a, a));
  if (std::fabs(cluster::Cosine(a, {-1, -2, -3, -4}) + 1) > 1e-6) FATAL("opposite");
  if (cluster::Cosine({1, 0}, {0, 1}) != 0) FATAL("orthogonal");
  if (cluster::Cosine(a, {0, 0, 0, 0}) != 0) FATAL("zero vector");
  std::mt19937_64 rng(9);
  std::normal_distribution<double> nd(0.0, 1.0);
  for (int n : {1, 7, 8, 9, 768, 1001}) {
    std::vector<float> x(n + 1), y(n + 1);
    for (auto& v : x) v = (float)nd(rng);
    for (auto& v : y) v = (float)nd(rng);
    double dot = 0, nx = 0, ny = 0;
    for (int i = 0; i <= n; i++) {
      dot += (double)x[i] * y[i];
      nx += (double)x[i] * x[i];
      ny += (double)y[i] * y[i];
    }
    const double want = dot / std::sqrt(nx * ny);
    if (std::fabs(cluster::Cosine(x, y) - want) > 1e-5) FATAL("n=%d: %g vs %g", n + 1, cluster::Cosine(x, y), want);
  }
  bool threw = false;
  try {
    cluster::Cosine({1, 2}, {1});
  } catch (const cluster::Error&) {
    threw = true;
  }
  if (!threw) FATAL("lengths 2 and 1 did not panic");
}

// cluster_test.go:118-132
TEST(TestSimilarities) {
  std::mt19937_64 rng(3);
  const Tensor q = cluster::Normalize(randn(rng, 5, 64));
  const Tensor d = cluster::Normalize(randn(rng, 7, 64));
  const Tensor s = cluster::Similarities(q, d);
  if (s.Dim(0) != 5 || s.Dim(1) != 7) FATAL("shape [%lld %lld]", (long long)s.Dim(0), (long long)s.Dim(1));
  const auto qd = q.Float32s(), dd = d.Float32s();
  for (int i = 0; i < 5; i++)
    for (int j = 0; j < 7; j++) {
      const float want = cluster::Cosine(std::vector<float>(qd.begin() + i * 64, qd.begin() + (i + 1) * 64),
                                         std::vector<float>(dd.begin() + j * 64, dd.begin() + (j + 1) * 64));
      if (std::fabs(s.At({i, j}) - want) > 1e-5) FATAL("(%d,%d): %g vs %g", i, j, s.At({i, j}), want);
    }
}

TEST(TestKMeansPanics) {
  std::mt19937_64 rng(4);
  const Tensor x = cluster::Normalize(randn(rng, 5, 8));
  for (int k : {0, 6}) {
    bool threw = false;
    try {
      cluster::KMeans(x, k, 3, 1);
    } catch (const cluster::Error& e) {
      threw = std::string(e.what()) == "cluster: k must be between 1 and the number of rows";
    }
    if (!threw) FATAL("k=%d did not panic with the reference's message", k);
  }
}

int main(int argc, char** argv) { return ctest::run_all(argc, argv); }
