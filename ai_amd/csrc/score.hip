// Per-row top-k selection over a score matrix [nq x nd] (the config-5
// nearest-neighbour step after cluster.Similarities, cluster/cluster.go:
// 185-190). Order: larger score first; equal scores by lower index (the
// first-max rule of (*Tensor).Argmax, tensor/reduce.go:269-297); NaN scores
// are never selected.
//
// Two passes, one wavefront per workgroup. Pass 1: each (query, chunk of
// the row) wave scans its chunk with four coalesced loads in flight per
// lane, every lane keeping its best KK (value, index) pairs sorted in
// registers (a candidate below the lane's k-th is dropped at once), then k
// rounds of a wave-wide arg-best over the lanes' list heads (shuffles, no
// barriers) write the chunk's top k. Pass 2: one wave per query merges the
// chunks' candidates the same way. Every comparison uses the full order
// (value, then index), so the result does not depend on the chunking.
#include <algorithm>
#include <cstdint>

#include "fa_internal.h"

namespace fa {
namespace {

constexpr int kMaxK = 32;
constexpr int kChunk = 4096;    // scores per pass-1 wave
constexpr int kMaxChunks = 64;  // per row

__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

// A lane's best k candidates, sorted, in the first k of KK registers; (tv,
// ti) is the k-th (the admission threshold).
template <int KK>
struct LaneList {
  float lv[KK];
  int li[KK];
  float tv = -INFINITY;
  int ti = INT32_MAX;
  __device__ __forceinline__ LaneList() {
#pragma unroll
    for (int i = 0; i < KK; i++) {
      lv[i] = -INFINITY;
      li[i] = INT32_MAX;
    }
  }
  __device__ __forceinline__ void insert(int k, float v, int j) {
    if (!better(v, j, tv, ti)) return;  // also drops NaN
    float cv = v;
    int ci = j;
    bool shifting = false;  // past the insertion point every entry moves down one
#pragma unroll
    for (int i = 0; i < KK; i++) {
      if (i < k && (shifting || better(cv, ci, lv[i], li[i]))) {
        shifting = true;
        const float t = lv[i];
        const int u = li[i];
        lv[i] = cv;
        li[i] = ci;
        cv = t;
        ci = u;
      }
    }
#pragma unroll
    for (int i = 0; i < KK; i++)
      if (i == k - 1) {
        tv = lv[i];
        ti = li[i];
      }
  }
};

// k rounds of a wave-wide arg-best over the lanes' list heads; lane 0
// writes result r to out_v[r] (if out_v) and out_i[r]
template <int KK>
__device__ __forceinline__ void wave_select(LaneList<KK>& L, int k, int lane, float* out_v, int32_t* out_i) {
  float (&lv)[KK] = L.lv;
  int (&li)[KK] = L.li;
  for (int r = 0; r < k; r++) {
    float v = lv[0];
    int i = li[0];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(v, o, 64);
      const int oi = __shfl_xor(i, o, 64);
      if (better(ov, oi, v, i)) {
        v = ov;
        i = oi;
      }
    }
    if (lane == 0) {
      if (out_v) out_v[r] = v;
      out_i[r] = i;
    }
    // the owner (unique index; an exhausted list offers INT32_MAX) pops its head
    if (li[0] == i && lv[0] == v) {
#pragma unroll
      for (int t = 0; t + 1 < KK; t++) {
        lv[t] = lv[t + 1];
        li[t] = li[t + 1];
      }
      lv[KK - 1] = -INFINITY;
      li[KK - 1] = INT32_MAX;
    }
  }
}

template <int KK>
__global__ __launch_bounds__(64) void topk_chunk_kernel(const float* __restrict__ scores, int64_t nd, int k,
                                                        int chunk, float* __restrict__ cv, int32_t* __restrict__ ci) {
  const int c = blockIdx.x, nchunks = gridDim.x;
  const int64_t q = blockIdx.y;
  const int lane = threadIdx.x;
  const float* row = scores + q * nd;
  LaneList<KK> L;
  const int64_t j0 = (int64_t)c * chunk, j1 = min(nd, j0 + chunk);
  for (int64_t j = j0 + lane; j < j1; j += 256) {
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) v[u] = j + 64 * u < j1 ? row[j + 64 * u] : -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; u++)
      if (j + 64 * u < j1) L.insert(k, v[u], (int)(j + 64 * u));
  }
  const int64_t o = (q * nchunks + c) * k;
  wave_select<KK>(L, k, lane, cv + o, ci + o);
}

template <int KK>
__global__ __launch_bounds__(64) void topk_merge_kernel(const float* __restrict__ cv, const int32_t* __restrict__ ci,
                                                        int ncand, int k, int32_t* __restrict__ idx,
                                                        float* __restrict__ val) {
  const int64_t q = blockIdx.x;
  const int lane = threadIdx.x;
  LaneList<KK> L;
  for (int t = lane; t < ncand; t += 64) L.insert(k, cv[q * ncand + t], ci[q * ncand + t]);
  wave_select<KK>(L, k, lane, val ? val + q * k : nullptr, idx + q * k);
}

}  // namespace

int topk_scratch_bytes(int64_t nq, int64_t nd, int32_t topk) {
  const int64_t nchunks = std::min<int64_t>(kMaxChunks, (nd + kChunk - 1) / kChunk);
  return (int)(nq * nchunks * topk * 8);
}

int launch_topk(fa_ctx* ctx, const float* scores, int64_t nq, int64_t nd, int32_t topk, int32_t* idx, float* val,
                void* scratch, hipStream_t s) {
  if (topk < 1 || topk > kMaxK)
    return set_error(ctx, FA_ERR_ARG, "Similarities top-k: k=%d outside 1..%d", topk, kMaxK);
  if (topk > nd) return set_error(ctx, FA_ERR_ARG, "Similarities top-k: k=%d > %lld docs", topk, (long long)nd);
  if (nq == 0) return FA_OK;
  if (nq > 65535) return set_error(ctx, FA_ERR_ARG, "Similarities top-k: %lld queries > 65535", (long long)nq);
  const int64_t nchunks = std::min<int64_t>(kMaxChunks, (nd + kChunk - 1) / kChunk);
  const int64_t chunk = (nd + nchunks - 1) / nchunks;
  float* cv = static_cast<float*>(scratch);
  int32_t* ci = reinterpret_cast<int32_t*>(cv + nq * nchunks * topk);
  const int ncand = (int)(nchunks * topk);
  dim3 g1((unsigned)nchunks, (unsigned)nq);
  if (topk <= 8) {
    hipLaunchKernelGGL(topk_chunk_kernel<8>, g1, dim3(64), 0, s, scores, nd, topk, (int)chunk, cv, ci);
    hipLaunchKernelGGL(topk_merge_kernel<8>, dim3((unsigned)nq), dim3(64), 0, s, cv, ci, ncand, topk, idx, val);
  } else if (topk <= 16) {
    hipLaunchKernelGGL(topk_chunk_kernel<16>, g1, dim3(64), 0, s, scores, nd, topk, (int)chunk, cv, ci);
    hipLaunchKernelGGL(topk_merge_kernel<16>, dim3((unsigned)nq), dim3(64), 0, s, cv, ci, ncand, topk, idx, val);
  } else {
    hipLaunchKernelGGL(topk_chunk_kernel<32>, g1, dim3(64), 0, s, scores, nd, topk, (int)chunk, cv, ci);
    hipLaunchKernelGGL(topk_merge_kernel<32>, dim3((unsigned)nq), dim3(64), 0, s, cv, ci, ncand, topk, idx, val);
  }
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

}  // namespace fa
