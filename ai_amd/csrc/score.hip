// Per-row top-k selection over a score matrix [nq x nd] (the config-5
// nearest-neighbour step after cluster.Similarities, cluster/cluster.go:
// 185-190). Order: larger score first; equal scores by lower index (the
// first-max rule of (*Tensor).Argmax, tensor/reduce.go:269-297); NaN scores
// are never selected.
//
// Two passes, one wavefront per workgroup. Pass 1: each (query, chunk of
// up to 16 384 scores) wave scans its chunk with eight 16-byte loads in
// flight per lane, keeping the chunk's best k so far as one sorted list spread over
// lanes 0..k-1; a ballot against the list's k-th entry filters each step's
// 64 scores, so after the first few hundred scores a step costs a load, a
// compare and a ballot, and the rare survivors are inserted one at a time
// with shuffles. Pass 2: one wave per query merges the chunks' candidates
// the same way. Every comparison uses the full order (value, then index),
// so the result does not depend on the chunking.
#include <algorithm>
#include <cstdint>

#include "fa_internal.h"

namespace fa {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxK = 32;
constexpr int kChunk = 16384;   // scores per pass-1 wave
constexpr int kMaxChunks = 64;  // per row

__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

// The wave's best k candidates so far as one sorted list spread over lanes
// 0..k-1 (lane r holds the r-th best; lanes >= k hold nothing that
// matters), with the k-th best (the admission threshold) in every lane.
// A step offers one candidate per lane: a ballot finds the lanes whose
// candidate beats the threshold (after the first few hundred scores, rarely
// any), and each of those is inserted in lane order: its rank is the number
// of list entries better than it, entries from that rank on move up one lane.
struct WaveList {
  float lv = -INFINITY;
  int li = INT32_MAX;
  float tv = -INFINITY;
  int ti = INT32_MAX;

  __device__ __forceinline__ void offer(int k, int lane, float v, int j) {
    uint64_t mask = __ballot(better(v, j, tv, ti));  // NaN never passes
    while (mask) {
      const int src = __ffsll((unsigned long long)mask) - 1;
      mask &= mask - 1;
      const float cv = __shfl(v, src, 64);
      const int ci = __shfl(j, src, 64);
      if (!better(cv, ci, tv, ti)) continue;  // the threshold rose meanwhile
      const uint64_t above = __ballot(lane < k && better(lv, li, cv, ci));
      const int pos = __popcll((unsigned long long)above);
      const float uv = __shfl_up(lv, 1, 64);
      const int ui = __shfl_up(li, 1, 64);
      if (lane > pos) {
        lv = uv;
        li = ui;
      } else if (lane == pos) {
        lv = cv;
        li = ci;
      }
      tv = __shfl(lv, k - 1, 64);
      ti = __shfl(li, k - 1, 64);
    }
  }
};

// Pass 1: the top k of scores[q, c*chunk .. min(nd, (c+1)*chunk)) to
// cv/ci[(q * nchunks + c) * k ..]. VEC = 4 (rows and chunks 16-byte
// aligned): eight 16-byte loads per lane, 2 048 scores per round, the next
// round loading while the current one is offered; VEC = 1: four 4-byte loads.
template <int VEC>
__global__ __launch_bounds__(64) void topk_chunk_kernel(const float* __restrict__ scores, int64_t nd, int k,
                                                        int chunk, float* __restrict__ cv, int32_t* __restrict__ ci) {
  constexpr int U = VEC == 4 ? 8 : 4;  // loads in flight per lane
  constexpr int ROUND = 64 * VEC * U;  // scores per round
  const int c = blockIdx.x, nchunks = gridDim.x;
  const int64_t q = blockIdx.y;
  const int lane = threadIdx.x;
  const float* row = scores + q * nd;
  WaveList W;
  const int64_t j0 = (int64_t)c * chunk, j1 = min(nd, j0 + chunk);
  if constexpr (VEC == 4) {
    // the next round's loads are issued before the current round's offers
    auto load = [&](f32x4 (&v)[U], int64_t base) {
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int64_t j = base + 4 * (lane + 64 * u);  // j1 is a multiple of 4
        v[u] = j < j1 ? *reinterpret_cast<const f32x4*>(row + j) : f32x4{NAN, NAN, NAN, NAN};
      }
    };
    auto offer_all = [&](const f32x4 (&v)[U], int64_t base) {
#pragma unroll
      for (int u = 0; u < U; u++)
#pragma unroll
        for (int e = 0; e < 4; e++) W.offer(k, lane, v[u][e], (int)(base + 4 * (lane + 64 * u) + e));
    };
    f32x4 va[U], vb[U];
    load(va, j0);
    for (int64_t base = j0; base < j1; base += 2 * ROUND) {
      load(vb, base + ROUND);
      offer_all(va, base);
      if (base + ROUND >= j1) break;
      load(va, base + 2 * ROUND);
      offer_all(vb, base + ROUND);
    }
  } else {
    for (int64_t base = j0; base < j1; base += ROUND) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; u++) {
        const int64_t j = base + lane + 64 * u;
        v[u] = j < j1 ? row[j] : NAN;
      }
#pragma unroll
      for (int u = 0; u < U; u++) W.offer(k, lane, v[u], (int)(base + lane + 64 * u));
    }
  }
  if (lane < k) {
    const int64_t o = (q * nchunks + c) * k + lane;
    cv[o] = W.lv;
    ci[o] = W.li;
  }
}

// Pass 2: one wave per query merges its chunks' ncand candidates.
__global__ __launch_bounds__(64) void topk_merge_kernel(const float* __restrict__ cv, const int32_t* __restrict__ ci,
                                                        int ncand, int k, int32_t* __restrict__ idx,
                                                        float* __restrict__ val) {
  const int64_t q = blockIdx.x;
  const int lane = threadIdx.x;
  WaveList W;
  for (int t0 = 0; t0 < ncand; t0 += 64) {
    const int t = t0 + lane;
    const bool ok = t < ncand;
    W.offer(k, lane, ok ? cv[q * ncand + t] : NAN, ok ? ci[q * ncand + t] : INT32_MAX);
  }
  if (lane < k) {
    if (val) val[q * k + lane] = W.lv;
    idx[q * k + lane] = W.li;
  }
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
  const bool vec = nd % 4 == 0 && (reinterpret_cast<uintptr_t>(scores) & 15) == 0;
  const int64_t chunk = ((nd + nchunks - 1) / nchunks + 3) / 4 * 4;  // a multiple of 4
  float* cv = static_cast<float*>(scratch);
  int32_t* ci = reinterpret_cast<int32_t*>(cv + nq * nchunks * topk);
  const int ncand = (int)(nchunks * topk);
  dim3 g1((unsigned)nchunks, (unsigned)nq);
  if (vec)
    hipLaunchKernelGGL(topk_chunk_kernel<4>, g1, dim3(64), 0, s, scores, nd, topk, (int)chunk, cv, ci);
  else
    hipLaunchKernelGGL(topk_chunk_kernel<1>, g1, dim3(64), 0, s, scores, nd, topk, (int)chunk, cv, ci);
  hipLaunchKernelGGL(topk_merge_kernel, dim3((unsigned)nq), dim3(64), 0, s, cv, ci, ncand, topk, idx, val);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

}  // namespace fa
