#include "cluster.hpp"

#include <cmath>
#include <limits>
#include <string>

namespace fiber::cluster {

namespace {

std::string shape_str(const tensor::Shape& s) {
  std::string o = "[";
  for (size_t i = 0; i < s.size(); i++) o += (i ? " " : "") + std::to_string(s[i]);
  return o + "]";
}

void call(const char* op, int rc) {
  if (rc == FA_OK) return;
  const std::string msg = fa_last_error(device());
  if (rc == FA_ERR_ARG) throw tensor::Error(op, msg);
  throw std::runtime_error(std::string("fa_rocm: ") + op + ": " + msg);
}

void need_2d(const char* op, const tensor::Tensor& x) {
  if (x.Dims() != 2) throw tensor::Error(op, "want a 2-D tensor, got " + shape_str(x.shape()));
}

}  // namespace

tensor::Tensor Normalize(const tensor::Tensor& x) {
  need_2d("Normalize", x);
  const tensor::Tensor xc = x.Contiguous();
  tensor::Tensor out = tensor::Tensor::Zeros(x.shape());
  call("Normalize",
       fa_cluster_normalize(device(), xc.base(), x.Dim(0), (int32_t)x.Dim(1), const_cast<float*>(out.base())));
  return out;
}

double Result::Inertia() const {
  if (Similarity.empty()) return std::numeric_limits<double>::quiet_NaN();
  double s = 0;
  for (float v : Similarity) s += 1 - (double)v;
  return s / (double)Similarity.size();
}

Result KMeans(const tensor::Tensor& x, int k, int iters, uint64_t seed) {
  need_2d("KMeans", x);
  const int64_t n = x.Dim(0), d = x.Dim(1);
  if (k <= 0 || k > n) throw Error("cluster: k must be between 1 and the number of rows");
  const tensor::Tensor xc = x.Contiguous();
  Result r;
  std::vector<float> centres((size_t)k * d);
  std::vector<int32_t> assign((size_t)n), sizes((size_t)k);
  r.Similarity.resize((size_t)n);
  int32_t it = 0;
  call("KMeans", fa_cluster_kmeans(device(), xc.base(), n, (int32_t)d, k, iters, seed, centres.data(), assign.data(),
                                   r.Similarity.data(), sizes.data(), &it));
  r.Centres = tensor::Tensor::New(std::move(centres), {k, d});
  r.Assignment.assign(assign.begin(), assign.end());
  r.Sizes.assign(sizes.begin(), sizes.end());
  r.Iterations = it;
  return r;
}

std::pair<std::vector<int>, std::vector<float>> Nearest(const tensor::Tensor& x, const tensor::Tensor& centres) {
  need_2d("MatMul", x);
  need_2d("MatMul", centres);
  if (x.Dim(1) != centres.Dim(1))
    throw tensor::Error("MatMul", "shape mismatch " + shape_str(x.shape()) + " · " + shape_str(centres.T().shape()));
  const int64_t n = x.Dim(0);
  const tensor::Tensor xc = x.Contiguous(), cc = centres.Contiguous();
  std::vector<int32_t> idx((size_t)n);
  std::vector<float> sim((size_t)n);
  call("Nearest", fa_cluster_nearest(device(), xc.base(), n, cc.base(), centres.Dim(0), (int32_t)x.Dim(1),
                                     idx.data(), sim.data()));
  return {std::vector<int>(idx.begin(), idx.end()), std::move(sim)};
}

float Cosine(const std::vector<float>& a, const std::vector<float>& b) {
  if (a.size() != b.size())
    throw Error("cluster: Cosine: lengths " + std::to_string(a.size()) + " and " + std::to_string(b.size()) +
                " differ");
  if (a.empty()) return 0;
  // a.b, a.a and b.b from one product of the stacked pair with its transpose
  std::vector<float> pair(a);
  pair.insert(pair.end(), b.begin(), b.end());
  const int64_t n = (int64_t)a.size();
  const tensor::Tensor p = tensor::Tensor::New(std::move(pair), {2, n});
  const tensor::Tensor g = tensor::MatMul(p, p.T());
  const float dot = g.At({0, 1}), na = g.At({0, 0}), nb = g.At({1, 1});
  if (na == 0 || nb == 0) return 0;
  return (float)((double)dot / std::sqrt((double)na * (double)nb));
}

tensor::Tensor Similarities(const tensor::Tensor& queries, const tensor::Tensor& docs) {
  if (queries.Dims() != 2 || docs.Dims() != 2 || queries.Dim(1) != docs.Dim(1))
    throw Error("cluster: Similarities: shapes " + shape_str(queries.shape()) + " and " + shape_str(docs.shape()));
  return tensor::MatMul(queries, docs.T());
}

}  // namespace fiber::cluster
