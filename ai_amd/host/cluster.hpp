// cluster.hpp — C++ host mirror of fiber/ai's cluster package
// (cluster/cluster.go), computed on the GPU through the C ABI
// (fa_cluster_* and fa_matmul_fused of include/fa_rocm.h).
//
//   cluster.Normalize                 cluster.go:17-28
//   cluster.KMeans, Result, Inertia   cluster.go:30-131, 148-159
//   cluster.Nearest                   cluster.go:134-146
//   cluster.Cosine                    cluster.go:161-178
//   cluster.Similarities              cluster.go:180-190
// The reference's panic("cluster: ...") is thrown as fiber::cluster::Error;
// shape errors of the tensor layer as fiber::tensor::Error.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <utility>
#include <vector>

#include "fiber.hpp"

namespace fiber::cluster {

struct Error : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// Every row scaled to unit length; rows of length zero stay zero.
tensor::Tensor Normalize(const tensor::Tensor& x);

struct Result {
  tensor::Tensor Centres;        // [k x d], unit length
  std::vector<int> Assignment;   // centre index per row
  std::vector<float> Similarity; // similarity of each row to its centre
  std::vector<int> Sizes;        // rows per centre
  int Iterations = 0;
  // Mean cosine distance of rows to their centres (NaN without rows).
  double Inertia() const;
};

// k-means++ seeding (Go's math/rand/v2 PCG seeded (seed, seed ^
// 0x9e3779b97f4a7c15)) and up to iters assignment/update rounds over the
// unit-length rows of x; stops when no row changes centre.
Result KMeans(const tensor::Tensor& x, int k, int iters, uint64_t seed);

// For every row, the index of the most similar centre and that similarity.
std::pair<std::vector<int>, std::vector<float>> Nearest(const tensor::Tensor& x, const tensor::Tensor& centres);

// Cosine similarity of two equal-length vectors (0 for an all-zero vector
// or empty input).
float Cosine(const std::vector<float>& a, const std::vector<float>& b);

// [q x n] dot products of unit-length rows: one product.
tensor::Tensor Similarities(const tensor::Tensor& queries, const tensor::Tensor& docs);

}  // namespace fiber::cluster
