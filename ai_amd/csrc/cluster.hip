// k-means and nearest-centre search over embedding rows on gfx950: the
// drop-in for fiber/ai's cluster package (cluster/cluster.go:17-146).
//
// Nearest = one fp32-MFMA product sim = x . centres^T [n x k] (the GEMM of
// gemm.hip) + a per-row first-max argmax (tensor/reduce.go:269-297).
//
// KMeans keeps every step on the device; the host only draws the random
// numbers (Go's math/rand/v2 PCG, whose draws do not depend on the data, so
// all of them are drawn up front) and reads the per-iteration change count
// and centre sizes for the early stop and the empty-centre restarts.
//   k-means++ (cluster.go:51-85): per new centre, kpp_weights_kernel scores
//     every row against the newest centre, keeps the best similarity and
//     writes the float64 weight (1 - best)^2; block_sums_kernel sums the
//     weights in blocks of 256; kpp_pick_kernel (one workgroup) scans the
//     block sums, scales the uniform draw by the total, finds the block and
//     then the row where the running subtraction crosses zero, and copies
//     that row into the centre list.
//   Lloyd rounds (cluster.go:86-129): sim product, argmax_rows_kernel
//     (assignment, similarity), count_kernel (per-chunk centre counts and
//     change counts), a stable counting sort of the row indices by centre
//     (chunk_scan_kernel, offsets_kernel, scatter_kernel), then
//     colsum_kernel adds each centre's rows in increasing row order, one
//     lane per (centre, column): the same float32 additions in the same
//     order as the reference's loop, so the centre sums are bit-identical
//     given the same assignment. Empty centres restart on the worst-fitting
//     row (worst_kernel, in increasing centre order), and
//     normalize_rows_kernel renormalises.
#include <cmath>
#include <cstring>
#include <vector>

#include "device_math.h"
#include "fa_internal.h"

namespace fa {
namespace {

constexpr int kRowWG = 256;        // one wave per row, 4 rows per workgroup
constexpr int kChunk = 256;        // rows per counting-sort chunk (one per thread of count_kernel)
constexpr int kCntWindow = 8192;   // centres per LDS counter window
constexpr int kPickThreads = 1024;
constexpr int kSumBlock = 256;     // weights per partial sum of the k-means++ pick
constexpr int kColTile = 32;       // rows loaded ahead by colsum_kernel

inline unsigned row_blocks(int64_t n) { return (unsigned)((n + 3) / 4); }

// cluster.Normalize (cluster.go:17-28): x / sqrt(sum x^2), a zero norm
// replaced by 1 (zero rows stay zero). In place allowed (out == x).
__global__ __launch_bounds__(kRowWG) void normalize_rows_kernel(const float* x, int64_t n, int d, float* out) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n) return;
  const float* xr = x + row * d;
  float ss = 0.f;
  for (int j = lane; j < d; j += 64) {
    const float v = xr[j];
    ss += v * v;
  }
  float nrm = sqrtf(wave_sum(ss));
  if (nrm == 0.f) nrm = 1.f;
  float* orow = out + row * d;
  for (int j = lane; j < d; j += 64) orow[j] = xr[j] / nrm;
}

// First-max argmax of each row of sim [n x k] with the sequential rule of
// (*Tensor).Argmax: the first index holding the maximum; NaN never wins
// except at index 0, where the sequential scan starts.
__global__ __launch_bounds__(kRowWG) void argmax_rows_kernel(const float* __restrict__ sim, int64_t n, int k,
                                                             int32_t* __restrict__ assign,
                                                             float* __restrict__ simil) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n) return;
  const float* sr = sim + row * k;
  float bv = -INFINITY;
  int bi = INT32_MAX;
  for (int j = lane; j < k; j += 64) {
    const float v = sr[j];
    if (v > bv) {
      bv = v;
      bi = j;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane != 0) return;
  if (bi == INT32_MAX || isnan(sr[0])) bi = 0;
  assign[row] = bi;
  simil[row] = sr[bi];
}

// Per chunk of kChunk rows: rows per centre (chunk_cnt[c][ch], centre-major)
// and rows whose centre differs from the previous round's
// (chunk_changed[ch]); then the previous assignment is brought up to date.
__global__ __launch_bounds__(kChunk) void count_kernel(const int32_t* __restrict__ cur, int32_t* __restrict__ prev,
                                                       int64_t n, int k, int nchunks, int32_t* __restrict__ chunk_cnt,
                                                       int32_t* __restrict__ chunk_changed) {
  __shared__ int32_t cnt[kCntWindow];
  __shared__ int32_t nchanged;
  const int t = threadIdx.x;
  const int64_t ch = blockIdx.x;
  const int64_t row = ch * kChunk + t;
  const int a = row < n ? cur[row] : -1;
  if (t == 0) nchanged = 0;
  __syncthreads();
  if (row < n && prev[row] != a) atomicAdd(&nchanged, 1);
  for (int w0 = 0; w0 < k; w0 += kCntWindow) {
    const int w1 = min(k, w0 + kCntWindow);
    for (int c = t; c < w1 - w0; c += kChunk) cnt[c] = 0;
    __syncthreads();
    if (a >= w0 && a < w1) atomicAdd(&cnt[a - w0], 1);
    __syncthreads();
    for (int c = t; c < w1 - w0; c += kChunk) chunk_cnt[(int64_t)(w0 + c) * nchunks + ch] = cnt[c];
    __syncthreads();
  }
  if (row < n) prev[row] = a;
  if (t == 0) chunk_changed[ch] = nchanged;
}

// k-means++ step over all rows: s = x[i] . c, best[i] = max(best[i], s),
// w[i] = float64(1 - best[i])^2 (cluster.go:62-72).
__global__ __launch_bounds__(kRowWG) void kpp_weights_kernel(const float* __restrict__ x, int64_t n, int d,
                                                             const float* __restrict__ c, float* best, double* w) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= n) return;
  const float* xr = x + row * d;
  float s = 0.f;
  if ((d & 3) == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(c)) & 15) == 0) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    const f4* xv = reinterpret_cast<const f4*>(xr);
    const f4* cv = reinterpret_cast<const f4*>(c);
    for (int j = lane; j < d / 4; j += 64) {
      const f4 a = xv[j], b = cv[j];
      s += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
    }
  } else {
    for (int j = lane; j < d; j += 64) s += xr[j] * c[j];
  }
  s = wave_sum(s);
  if (lane != 0) return;
  float b = best[row];
  if (s > b) b = s;
  best[row] = b;
  const double om = (double)(1.f - b);
  w[row] = om * om;
}

// part[b] = sum of w[b*kSumBlock ...] in a fixed tree order.
__global__ __launch_bounds__(kSumBlock) void block_sums_kernel(const double* __restrict__ w, int64_t n,
                                                               double* __restrict__ part) {
  __shared__ double buf[kSumBlock];
  const int t = threadIdx.x;
  const int64_t i = (int64_t)blockIdx.x * kSumBlock + t;
  buf[t] = i < n ? w[i] : 0.0;
  __syncthreads();
  for (int o = kSumBlock / 2; o > 0; o >>= 1) {
    if (t < o) buf[t] += buf[t + o];
    __syncthreads();
  }
  if (t == 0) part[blockIdx.x] = buf[0];
}

// k-means++ pick (cluster.go:73-82): pick = u * total; the chosen row is
// the first i where pick - w[0] - ... - w[i] <= 0 (n-1 when rounding leaves
// it positive). The block partial sums' inclusive prefix locates the
// crossing block, whose weights are then walked one by one. The row is
// copied to centre_out.
__global__ __launch_bounds__(kPickThreads) void kpp_pick_kernel(const double* __restrict__ w, int64_t n,
                                                                const double* __restrict__ part, int nparts, double u,
                                                                const float* __restrict__ x, int d,
                                                                float* __restrict__ centre_out, int32_t* chosen) {
  __shared__ double scan[kPickThreads];
  __shared__ double wblk[kSumBlock];
  __shared__ double carry, total_s;
  __shared__ int first_blk;
  __shared__ int64_t pick_idx;
  const int t = threadIdx.x;
  if (t == 0) {
    carry = 0;
    first_blk = INT32_MAX;
  }
  __syncthreads();
  // total: inclusive scan of the partials in tiles of kPickThreads (pass 1)
  for (int base = 0; base < nparts; base += kPickThreads) {
    scan[t] = base + t < nparts ? part[base + t] : 0.0;
    __syncthreads();
    for (int o = 1; o < kPickThreads; o <<= 1) {
      const double add = t >= o ? scan[t - o] : 0.0;
      __syncthreads();
      scan[t] += add;
      __syncthreads();
    }
    if (t == 0) carry += scan[kPickThreads - 1];
    __syncthreads();
  }
  if (t == 0) total_s = carry;
  __syncthreads();
  const double pick = u * total_s;
  // pass 2: the first block whose inclusive prefix reaches pick (one tile of
  // partials: the scan of pass 1 is still in LDS)
  const bool one_tile = nparts <= kPickThreads;
  if (t == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < nparts; base += kPickThreads) {
    if (!one_tile) {
      scan[t] = base + t < nparts ? part[base + t] : 0.0;
      __syncthreads();
      for (int o = 1; o < kPickThreads; o <<= 1) {
        const double add = t >= o ? scan[t - o] : 0.0;
        __syncthreads();
        scan[t] += add;
        __syncthreads();
      }
    }
    if (base + t < nparts && pick - (carry + scan[t]) <= 0) atomicMin(&first_blk, base + t);
    __syncthreads();
    if (first_blk != INT32_MAX) break;
    if (t == 0) carry += scan[kPickThreads - 1];
    __syncthreads();
  }
  __syncthreads();
  const int fb = first_blk;
  // the prefix before block fb, in the order pass 2 formed it
  if (fb != INT32_MAX && t == 0) {
    const int tile = fb / kPickThreads * kPickThreads;
    total_s = carry + (fb > tile ? scan[fb - tile - 1] : 0.0);
  }
  const int64_t b0 = fb != INT32_MAX ? (int64_t)fb * kSumBlock : n;
  if (t < kSumBlock) wblk[t] = b0 + t < n ? w[b0 + t] : 0.0;
  __syncthreads();
  if (t == 0) {
    int64_t idx = n - 1;
    if (fb != INT32_MAX) {
      double p = pick - total_s;
      int64_t i = b0;
      for (; i < min(n, b0 + kSumBlock); i++) {
        p -= wblk[i - b0];
        if (p <= 0) break;
      }
      if (i >= min(n, b0 + kSumBlock))  // rounding: keep walking
        for (; i < n; i++) {
          p -= w[i];
          if (p <= 0) break;
        }
      if (i < n) idx = i;
    }
    pick_idx = idx;
    *chosen = (int32_t)idx;
  }
  __syncthreads();
  const float* src = x + pick_idx * d;
  for (int j = t; j < d; j += kPickThreads) centre_out[j] = src[j];
}

// chunk_cnt[c][ch] (rows of chunk ch assigned to c) -> exclusive prefix over
// chunks; sizes[c] = total. One workgroup per centre.
__global__ __launch_bounds__(256) void chunk_scan_kernel(int32_t* chunk_cnt, int nchunks, int32_t* sizes) {
  __shared__ int32_t buf[256];
  __shared__ int32_t carry;
  const int t = threadIdx.x;
  int32_t* row = chunk_cnt + (int64_t)blockIdx.x * nchunks;
  if (t == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < nchunks; base += 256) {
    const int32_t v = base + t < nchunks ? row[base + t] : 0;
    buf[t] = v;
    __syncthreads();
    for (int o = 1; o < 256; o <<= 1) {
      const int32_t add = t >= o ? buf[t - o] : 0;
      __syncthreads();
      buf[t] += add;
      __syncthreads();
    }
    if (base + t < nchunks) row[base + t] = carry + buf[t] - v;
    __syncthreads();
    if (t == 0) carry += buf[255];
    __syncthreads();
  }
  if (t == 0) sizes[blockIdx.x] = carry;
}

// offsets[c] = sizes[0] + ... + sizes[c-1]; *changed = sum of the chunks'
// change counts. One workgroup.
__global__ __launch_bounds__(1024) void offsets_kernel(const int32_t* sizes, int k, int32_t* offsets,
                                                       const int32_t* chunk_changed, int nchunks, int32_t* changed) {
  __shared__ int32_t buf[1024];
  __shared__ int32_t carry;
  const int t = threadIdx.x;
  if (t == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base < k; base += 1024) {
    const int32_t v = base + t < k ? sizes[base + t] : 0;
    buf[t] = v;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {  // inclusive Hillis-Steele scan
      const int32_t add = t >= o ? buf[t - o] : 0;
      __syncthreads();
      buf[t] += add;
      __syncthreads();
    }
    if (base + t < k) offsets[base + t] = carry + buf[t] - v;
    __syncthreads();
    if (t == 0) carry += buf[1023];
    __syncthreads();
  }
  int32_t s = 0;
  for (int ch = t; ch < nchunks; ch += 1024) s += chunk_changed[ch];
  buf[t] = s;
  __syncthreads();
  for (int o = 512; o > 0; o >>= 1) {
    if (t < o) buf[t] += buf[t + o];
    __syncthreads();
  }
  if (t == 0) *changed = buf[0];
}

// Stable scatter of row indices by centre: list[offsets[a] + (rows of a in
// earlier chunks) + (rows of a earlier in this chunk)] = row. One wave per
// chunk walks its rows in order 64 at a time; the rank among equal lanes
// comes from shuffles, the running count per centre from LDS (centre
// windows of kCntWindow).
__global__ __launch_bounds__(64) void scatter_kernel(const int32_t* __restrict__ assign, int64_t n, int k,
                                                     int nchunks, const int32_t* __restrict__ offsets,
                                                     const int32_t* __restrict__ chunk_pre, int32_t* __restrict__ list) {
  __shared__ int32_t cnt[kCntWindow];
  const int lane = threadIdx.x;
  const int64_t ch = blockIdx.x;
  const int64_t r0 = ch * kChunk;
  for (int w0 = 0; w0 < k; w0 += kCntWindow) {
    const int w1 = min(k, w0 + kCntWindow);
    for (int c = lane; c < w1 - w0; c += 64) cnt[c] = 0;
    __syncthreads();
    for (int sub = 0; sub < kChunk; sub += 64) {
      const int64_t row = r0 + sub + lane;
      int a = row < n ? assign[row] : -1;
      if (a < w0 || a >= w1) a = -1;
      int rank = 0, later = 0;
      for (int j = 0; j < 64; j++) {
        const int aj = __shfl(a, j, 64);
        if (aj == a) {
          rank += j < lane;
          later += j > lane;
        }
      }
      if (a >= 0) list[offsets[a] + chunk_pre[(int64_t)a * nchunks + ch] + cnt[a - w0] + rank] = (int32_t)row;
      __syncthreads();
      if (a >= 0 && later == 0) cnt[a - w0] += rank + 1;
      __syncthreads();
    }
  }
}

// sums[c][j] = sum over c's rows in increasing row order of x[row][j],
// accumulated in float32 from 0 (cluster.go:100-112). One wave per (centre,
// 64 columns); kColTile rows are loaded ahead of their additions.
__global__ __launch_bounds__(64) void colsum_kernel(const float* __restrict__ x, int d,
                                                    const int32_t* __restrict__ list,
                                                    const int32_t* __restrict__ offsets,
                                                    const int32_t* __restrict__ sizes, float* __restrict__ sums) {
  const int c = blockIdx.x;
  const int j = blockIdx.y * 64 + threadIdx.x;
  if (j >= d) return;
  const int32_t* rows = list + offsets[c];
  const int m = sizes[c];
  float acc = 0.f;
  int p = 0;
  for (; p + kColTile <= m; p += kColTile) {
    float v[kColTile];
#pragma unroll
    for (int u = 0; u < kColTile; u++) v[u] = x[(int64_t)rows[p + u] * d + j];
#pragma unroll
    for (int u = 0; u < kColTile; u++) acc += v[u];
  }
  for (; p < m; p++) acc += x[(int64_t)rows[p] * d + j];
  sums[(int64_t)c * d + j] = acc;
}

// Empty-centre restart (cluster.go:113-124): worst = the first index of the
// minimum similarity (index 0 when no element compares below simil[0]);
// its row becomes the centre's sum and its similarity is set to 1.
__global__ __launch_bounds__(1024) void worst_kernel(float* simil, int64_t n, const float* __restrict__ x, int d,
                                                     float* __restrict__ sums_row) {
  __shared__ float sv[1024];
  __shared__ int64_t si[1024];
  const int t = threadIdx.x;
  float bv = INFINITY;
  int64_t bi = INT64_MAX;
  for (int64_t i = t; i < n; i += 1024) {
    const float v = simil[i];
    if (v < bv) {
      bv = v;
      bi = i;
    }
  }
  sv[t] = bv;
  si[t] = bi;
  __syncthreads();
  for (int o = 512; o > 0; o >>= 1) {
    if (t < o) {
      const float ov = sv[t + o];
      const int64_t oi = si[t + o];
      if (ov < sv[t] || (ov == sv[t] && oi < si[t])) {
        sv[t] = ov;
        si[t] = oi;
      }
    }
    __syncthreads();
  }
  const int64_t worst = (si[0] == INT64_MAX || isnan(simil[0])) ? 0 : si[0];
  __syncthreads();
  if (t == 0) simil[worst] = 1.f;
  const float* src = x + worst * d;
  for (int j = t; j < d; j += 1024) sums_row[j] = src[j];
}

__global__ void fill_f32_kernel(float* p, int64_t n, float v) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace
}  // namespace fa

// ---- host side -----------------------------------------------------------------

namespace fa {
namespace {

// Go's math/rand/v2 generator as cluster.KMeans seeds it
// (rand.New(rand.NewPCG(seed, seed^0x9e3779b97f4a7c15)), cluster.go:47):
// a 128-bit LCG (pcg-cpp's default multiplier and increment) whose new
// state goes through the DXSM output function; IntN is Lemire's
// multiply-shift with rejection (a mask for powers of two), Float64 the top
// 53 bits of a draw over 2^53.
struct GoPCG {
  uint64_t hi, lo;
  uint64_t Uint64() {
    typedef unsigned __int128 u128;
    const u128 mul = ((u128)2549297995355413924ULL << 64) | 4865540595714422341ULL;
    const u128 inc = ((u128)6364136223846793005ULL << 64) | 1442695040888963407ULL;
    const u128 s = ((((u128)hi) << 64) | lo) * mul + inc;
    hi = (uint64_t)(s >> 64);
    lo = (uint64_t)s;
    uint64_t h = hi;
    h ^= h >> 32;
    h *= 0xda942042e4dd58b5ULL;
    h ^= h >> 48;
    return h * (lo | 1);
  }
  uint64_t IntN(uint64_t n) {
    typedef unsigned __int128 u128;
    if ((n & (n - 1)) == 0) return Uint64() & (n - 1);
    u128 m = (u128)Uint64() * n;
    if ((uint64_t)m < n) {
      const uint64_t thresh = (0 - n) % n;
      while ((uint64_t)m < thresh) m = (u128)Uint64() * n;
    }
    return (uint64_t)(m >> 64);
  }
  double Float64() { return (double)(Uint64() << 11 >> 11) / 9007199254740992.0; }
};

size_t align256(size_t b) { return (b + 255) & ~size_t(255); }

int check_rows(fa_ctx* ctx, const char* op, int64_t n, int64_t d) {
  if (n < 0 || d < 0 || n > INT32_MAX || d > INT32_MAX)
    return set_error(ctx, FA_ERR_ARG, "%s: shape [%lld x %lld] outside this build's int32 row/column range", op,
                     (long long)n, (long long)d);
  return FA_OK;
}

int launch_normalize(fa_ctx* ctx, const float* x, int64_t n, int d, float* out) {
  if (n == 0 || d == 0) return FA_OK;
  hipLaunchKernelGGL(normalize_rows_kernel, dim3(row_blocks(n)), dim3(kRowWG), 0, ctx->stream, x, n, d, out);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

// sim = x . c^T [n x k] on the fp32 MFMA GEMM.
int launch_sim(fa_ctx* ctx, const float* x, int64_t n, const float* c, int64_t k, int d, float* sim) {
  GemmArgs g;
  g.m = n;
  g.n = k;
  g.k = d;
  g.a = x;
  g.lda = d;
  g.b = c;
  g.ldb = d;
  g.b_dtype = FA_DT_F32;
  g.b_layout = FA_B_NK;
  g.c = sim;
  g.ldc = k;
  return launch_gemm(ctx, g, ctx->stream);
}

}  // namespace
}  // namespace fa

using fa::set_error;
using namespace fa::slots;

extern "C" {

int fa_cluster_normalize_dev(fa_ctx* ctx, const float* x, int64_t n, int32_t d, float* out) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "cluster: ctx is NULL");
  int rc;
  if ((rc = fa::check_rows(ctx, "Normalize", n, d))) return rc;
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "cluster");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  return fa::launch_normalize(ctx, x, n, d, out);
}

int fa_cluster_normalize(fa_ctx* ctx, const float* x, int64_t n, int32_t d, float* out) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "cluster: ctx is NULL");
  int rc;
  if ((rc = fa::check_rows(ctx, "Normalize", n, d))) return rc;
  if (n == 0 || d == 0) return FA_OK;
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "cluster");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  void* dx;
  const size_t bytes = (size_t)n * d * 4;
  if ((rc = fa::stage_h2d(ctx, S_CL_X, x, bytes, &dx))) return rc;
  if ((rc = fa::launch_normalize(ctx, (const float*)dx, n, d, (float*)dx))) return rc;
  FA_HIP_CHECK(ctx, hipMemcpyAsync(out, dx, bytes, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

int fa_cluster_nearest_dev(fa_ctx* ctx, const float* x, int64_t n, const float* centres, int64_t k, int32_t d,
                           int32_t* index, float* similarity) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "cluster: ctx is NULL");
  int rc;
  if ((rc = fa::check_rows(ctx, "Nearest", n, d))) return rc;
  if (k <= 0 || k > INT32_MAX)
    return set_error(ctx, FA_ERR_ARG, "Argmax: cannot reduce empty dimension 1 of shape [%lld %lld]", (long long)n,
                     (long long)k);
  if (d <= 0) return set_error(ctx, FA_ERR_ARG, "Nearest: rows of length %d", d);
  if (n == 0) return FA_OK;
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "Nearest");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  fa::DevBuf& ws = ctx->slot(S_CL_WORK);
  if ((rc = ws.ensure(ctx, (size_t)n * k * 4))) return rc;
  float* sim = ws.as<float>();
  if ((rc = fa::launch_sim(ctx, x, n, centres, k, d, sim))) return rc;
  hipLaunchKernelGGL(fa::argmax_rows_kernel, dim3(fa::row_blocks(n)), dim3(fa::kRowWG), 0, ctx->stream, sim, n,
                     (int)k, index, similarity);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int fa_cluster_nearest(fa_ctx* ctx, const float* x, int64_t n, const float* centres, int64_t k, int32_t d,
                       int32_t* index, float* similarity) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "cluster: ctx is NULL");
  int rc;
  if ((rc = fa::check_rows(ctx, "Nearest", n, d))) return rc;
  if (k <= 0 || k > INT32_MAX)
    return set_error(ctx, FA_ERR_ARG, "Argmax: cannot reduce empty dimension 1 of shape [%lld %lld]", (long long)n,
                     (long long)k);
  if (d <= 0) return set_error(ctx, FA_ERR_ARG, "Nearest: rows of length %d", d);
  if (n == 0) return FA_OK;
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "Nearest");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  void *dx, *dc;
  if ((rc = fa::stage_h2d(ctx, S_CL_X, x, (size_t)n * d * 4, &dx))) return rc;
  if ((rc = fa::stage_h2d(ctx, S_CL_C, centres, (size_t)k * d * 4, &dc))) return rc;
  fa::DevBuf& ob = ctx->slot(S_CL_OUT);
  if ((rc = ob.ensure(ctx, (size_t)n * 8))) return rc;
  int32_t* di = ob.as<int32_t>();
  float* ds = (float*)(di + n);
  if ((rc = fa_cluster_nearest_dev(ctx, (const float*)dx, n, (const float*)dc, k, d, di, ds))) return rc;
  FA_HIP_CHECK(ctx, hipMemcpyAsync(index, di, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipMemcpyAsync(similarity, ds, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

int fa_cluster_kmeans_dev(fa_ctx* ctx, const float* x, int64_t n, int32_t d, int32_t k, int32_t iters,
                          uint64_t seed, float* centres, int32_t* assignment, float* similarity, int32_t* sizes,
                          int32_t* iterations) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "cluster: ctx is NULL");
  int rc;
  if ((rc = fa::check_rows(ctx, "KMeans", n, d))) return rc;
  if (k <= 0 || k > n) return set_error(ctx, FA_ERR_ARG, "cluster: k must be between 1 and the number of rows");
  if (d <= 0) return set_error(ctx, FA_ERR_ARG, "KMeans: rows of length %d", d);
  if (!iterations) return set_error(ctx, FA_ERR_ARG, "KMeans: iterations is NULL");
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "cluster");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  hipStream_t st = ctx->stream;
  const int nchunks = (int)((n + fa::kChunk - 1) / fa::kChunk);

  // workspace: raw centres, sums [k x d]; best [n]; w [n] f64; partial
  // sums of w; sim [n x k]; chunk counts [nchunks x k]; chunk change counts;
  // offsets [k]; list [n]; previous assignment [n]; changed; chosen [k]
  const int nparts = (int)((n + fa::kSumBlock - 1) / fa::kSumBlock);
  size_t off = 0;
  auto take = [&off](size_t bytes) {
    const size_t o = off;
    off += fa::align256(bytes);
    return o;
  };
  const size_t o_raw = take((size_t)k * d * 4), o_sums = take((size_t)k * d * 4), o_best = take((size_t)n * 4),
               o_w = take((size_t)n * 8), o_part = take((size_t)nparts * 8), o_sim = take((size_t)n * k * 4),
               o_cnt = take((size_t)nchunks * k * 4), o_chg = take((size_t)nchunks * 4), o_offs = take((size_t)k * 4),
               o_list = take((size_t)n * 4), o_prev = take((size_t)n * 4), o_changed = take(4),
               o_chosen = take((size_t)k * 4);
  fa::DevBuf& ws = ctx->slot(S_CL_WORK);
  if ((rc = ws.ensure(ctx, off))) return rc;
  char* base = ws.as<char>();
  float* raw = (float*)(base + o_raw);
  float* sums = (float*)(base + o_sums);
  float* best = (float*)(base + o_best);
  double* w = (double*)(base + o_w);
  double* part = (double*)(base + o_part);
  float* sim = (float*)(base + o_sim);
  int32_t* cnt = (int32_t*)(base + o_cnt);
  int32_t* chg = (int32_t*)(base + o_chg);
  int32_t* offs = (int32_t*)(base + o_offs);
  int32_t* list = (int32_t*)(base + o_list);
  int32_t* prev = (int32_t*)(base + o_prev);
  int32_t* changed = (int32_t*)(base + o_changed);
  int32_t* chosen = (int32_t*)(base + o_chosen);

  // k-means++ seeding (cluster.go:47-85); every draw up front
  fa::GoPCG rng{seed, seed ^ 0x9e3779b97f4a7c15ULL};
  const int64_t first = (int64_t)rng.IntN((uint64_t)n);
  std::vector<double> u((size_t)k, 0.0);
  for (int r = 1; r < k; r++) u[r] = rng.Float64();
  FA_HIP_CHECK(ctx, hipMemcpyAsync(raw, x + first * d, (size_t)d * 4, hipMemcpyDeviceToDevice, st));
  hipLaunchKernelGGL(fa::fill_f32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, best, n, -1.f);
  FA_CHECK_LAUNCH(ctx);
  for (int r = 1; r < k; r++) {
    hipLaunchKernelGGL(fa::kpp_weights_kernel, dim3(fa::row_blocks(n)), dim3(fa::kRowWG), 0, st, x, n, (int)d,
                       (const float*)(raw + (size_t)(r - 1) * d), best, w);
    FA_CHECK_LAUNCH(ctx);
    hipLaunchKernelGGL(fa::block_sums_kernel, dim3((unsigned)nparts), dim3(fa::kSumBlock), 0, st, (const double*)w,
                       n, part);
    FA_CHECK_LAUNCH(ctx);
    hipLaunchKernelGGL(fa::kpp_pick_kernel, dim3(1), dim3(fa::kPickThreads), 0, st, (const double*)w, n,
                       (const double*)part, nparts, u[r], x, (int)d, raw + (size_t)r * d, chosen + r);
    FA_CHECK_LAUNCH(ctx);
  }
  if ((rc = fa::launch_normalize(ctx, raw, k, d, centres))) return rc;

  // Lloyd rounds (cluster.go:86-129)
  FA_HIP_CHECK(ctx, hipMemsetAsync(assignment, 0, (size_t)n * 4, st));
  FA_HIP_CHECK(ctx, hipMemsetAsync(prev, 0, (size_t)n * 4, st));
  FA_HIP_CHECK(ctx, hipMemsetAsync(similarity, 0, (size_t)n * 4, st));
  FA_HIP_CHECK(ctx, hipMemsetAsync(sizes, 0, (size_t)k * 4, st));
  std::vector<int32_t> host((size_t)k + 1);
  int it_done = 0;
  for (int it = 1; it <= iters; it++) {
    it_done = it;
    if ((rc = fa::launch_sim(ctx, x, n, centres, k, d, sim))) return rc;
    hipLaunchKernelGGL(fa::argmax_rows_kernel, dim3(fa::row_blocks(n)), dim3(fa::kRowWG), 0, st,
                       (const float*)sim, n, (int)k, assignment, similarity);
    FA_CHECK_LAUNCH(ctx);
    hipLaunchKernelGGL(fa::count_kernel, dim3((unsigned)nchunks), dim3(fa::kChunk), 0, st,
                       (const int32_t*)assignment, prev, n, (int)k, nchunks, cnt, chg);
    FA_CHECK_LAUNCH(ctx);
    hipLaunchKernelGGL(fa::chunk_scan_kernel, dim3((unsigned)k), dim3(256), 0, st, cnt, nchunks, sizes);
    FA_CHECK_LAUNCH(ctx);
    hipLaunchKernelGGL(fa::offsets_kernel, dim3(1), dim3(1024), 0, st, (const int32_t*)sizes, (int)k, offs,
                       (const int32_t*)chg, nchunks, changed);
    FA_CHECK_LAUNCH(ctx);
    hipLaunchKernelGGL(fa::scatter_kernel, dim3((unsigned)nchunks), dim3(64), 0, st, (const int32_t*)assignment, n,
                       (int)k, nchunks, (const int32_t*)offs, (const int32_t*)cnt, list);
    FA_CHECK_LAUNCH(ctx);
    hipLaunchKernelGGL(fa::colsum_kernel, dim3((unsigned)k, (unsigned)((d + 63) / 64)), dim3(64), 0, st, x, (int)d,
                       (const int32_t*)list, (const int32_t*)offs, (const int32_t*)sizes, sums);
    FA_CHECK_LAUNCH(ctx);
    FA_HIP_CHECK(ctx, hipMemcpyAsync(host.data(), sizes, (size_t)k * 4, hipMemcpyDeviceToHost, st));
    FA_HIP_CHECK(ctx, hipMemcpyAsync(host.data() + k, changed, 4, hipMemcpyDeviceToHost, st));
    FA_HIP_CHECK(ctx, hipStreamSynchronize(st));
    for (int c = 0; c < k; c++) {
      if (host[c] != 0) continue;
      hipLaunchKernelGGL(fa::worst_kernel, dim3(1), dim3(1024), 0, st, similarity, n, x, (int)d,
                         sums + (size_t)c * d);
      FA_CHECK_LAUNCH(ctx);
    }
    if ((rc = fa::launch_normalize(ctx, sums, k, d, centres))) return rc;
    if (host[k] == 0 && it > 1) break;
  }
  *iterations = it_done;
  return FA_OK;
}

int fa_cluster_kmeans(fa_ctx* ctx, const float* x, int64_t n, int32_t d, int32_t k, int32_t iters, uint64_t seed,
                      float* centres, int32_t* assignment, float* similarity, int32_t* sizes, int32_t* iterations) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "cluster: ctx is NULL");
  int rc;
  if ((rc = fa::check_rows(ctx, "KMeans", n, d))) return rc;
  if (k <= 0 || k > n) return set_error(ctx, FA_ERR_ARG, "cluster: k must be between 1 and the number of rows");
  if (d <= 0) return set_error(ctx, FA_ERR_ARG, "KMeans: rows of length %d", d);
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "cluster");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  void* dx;
  if ((rc = fa::stage_h2d(ctx, S_CL_X, x, (size_t)n * d * 4, &dx))) return rc;
  fa::DevBuf& ob = ctx->slot(S_CL_OUT);
  const size_t cb = fa::align256((size_t)k * d * 4), nb = fa::align256((size_t)n * 4);
  if ((rc = ob.ensure(ctx, cb + 2 * nb + (size_t)k * 4))) return rc;
  char* o = ob.as<char>();
  float* dcent = (float*)o;
  int32_t* dassign = (int32_t*)(o + cb);
  float* dsim = (float*)(o + cb + nb);
  int32_t* dsizes = (int32_t*)(o + cb + 2 * nb);
  int32_t it = 0;
  if ((rc = fa_cluster_kmeans_dev(ctx, (const float*)dx, n, d, k, iters, seed, dcent, dassign, dsim, dsizes, &it)))
    return rc;
  FA_HIP_CHECK(ctx, hipMemcpyAsync(centres, dcent, (size_t)k * d * 4, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipMemcpyAsync(assignment, dassign, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipMemcpyAsync(similarity, dsim, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipMemcpyAsync(sizes, dsizes, (size_t)k * 4, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  if (iterations) *iterations = it;
  return FA_OK;
}

}  // extern "C"
