// Per-row top-k selection over a score matrix [nq x nd] (the config-5
// nearest-neighbour step after cluster.Similarities, cluster/cluster.go:
// 185-190). Order: larger score first; equal scores by lower index (the
// first-max rule of (*Tensor).Argmax, tensor/reduce.go:269-297).
//
// One workgroup per query row. Each thread scans a strided slice of the row
// keeping a sorted list of its best K in registers (indices increase along
// the scan, so an equal score never displaces an earlier one), then K rounds
// of a workgroup-wide arg-best over the threads' list heads pick the result.
#include "fa_internal.h"

namespace fa {
namespace {

constexpr int kMaxK = 32;
constexpr int kThreads = 256;

__device__ __forceinline__ bool better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

__global__ __launch_bounds__(kThreads) void topk_kernel(const float* __restrict__ scores, int64_t nd, int k,
                                                        int32_t* __restrict__ idx, float* __restrict__ val) {
  const int64_t q = blockIdx.x;
  const float* row = scores + q * nd;
  float lv[kMaxK];
  int li[kMaxK];
#pragma unroll
  for (int i = 0; i < kMaxK; i++) {
    lv[i] = -INFINITY;
    li[i] = INT32_MAX;
  }
  float thr = -INFINITY;  // the list's k-th value
  for (int64_t j = threadIdx.x; j < nd; j += kThreads) {
    const float v = row[j];
    if (!(v > thr)) continue;  // also drops NaN
    // insert keeping order (strictly greater moves past equal earlier entries)
    float cv = v;
    int ci = (int)j;
    bool shifting = false;  // past the insertion point every entry moves down one
#pragma unroll
    for (int i = 0; i < kMaxK; i++) {
      if (i < k && (shifting || cv > lv[i])) {
        shifting = true;
        float tv = lv[i];
        int ti = li[i];
        lv[i] = cv;
        li[i] = ci;
        cv = tv;
        ci = ti;
      }
    }
#pragma unroll
    for (int i = 0; i < kMaxK; i++)
      if (i == k - 1) thr = lv[i];
  }
  __shared__ float sv[kThreads];
  __shared__ int si[kThreads];
  __shared__ int owner[kThreads];
  int head = 0;
  for (int r = 0; r < k; r++) {
    // this thread's candidate
    float v = -INFINITY;
    int ii = INT32_MAX;
#pragma unroll
    for (int i = 0; i < kMaxK; i++)
      if (i == head) {
        v = lv[i];
        ii = li[i];
      }
    sv[threadIdx.x] = v;
    si[threadIdx.x] = ii;
    owner[threadIdx.x] = threadIdx.x;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
      if (threadIdx.x < s) {
        const int o = threadIdx.x + s;
        if (better(sv[o], si[o], sv[threadIdx.x], si[threadIdx.x])) {
          sv[threadIdx.x] = sv[o];
          si[threadIdx.x] = si[o];
          owner[threadIdx.x] = owner[o];
        }
      }
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      idx[q * k + r] = si[0];
      if (val) val[q * k + r] = sv[0];
    }
    if (owner[0] == (int)threadIdx.x) head++;
    __syncthreads();
  }
}

}  // namespace

int launch_topk(fa_ctx* ctx, const float* scores, int64_t nq, int64_t nd, int32_t topk, int32_t* idx, float* val,
                hipStream_t s) {
  if (topk < 1 || topk > kMaxK)
    return set_error(ctx, FA_ERR_ARG, "Similarities top-k: k=%d outside 1..%d", topk, kMaxK);
  if (topk > nd) return set_error(ctx, FA_ERR_ARG, "Similarities top-k: k=%d > %lld docs", topk, (long long)nd);
  if (nq == 0) return FA_OK;
  hipLaunchKernelGGL(topk_kernel, dim3((unsigned)nq), dim3(kThreads), 0, s, scores, nd, topk, idx, val);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

}  // namespace fa
