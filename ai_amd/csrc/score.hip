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
#include <mutex>
#include <type_traits>

#include "fa_internal.h"
#include "device_math.h"

namespace fa {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

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
    if (val) val[q * k + lane] = W.li == INT32_MAX ? NAN : W.lv;
    idx[q * k + lane] = W.li == INT32_MAX ? -1 : W.li;
  }
}

// ---------------------------------------------------------------------------
// Fused scoring: similarities and top-k without a score matrix.
//
// Per block of up to 256 queries, three launches:
//  1. score_qsplit_kernel: each query row split into hi + mid bf16 planes
//     (hi = the row with its low 16 bits cleared, mid the same of the
//     remainder) and its float64 norm.
//  2. score_stage1_kernel: one workgroup per range of 32-doc blocks; tiles of
//     256 queries x 128 docs on v_mfma_f32_32x32x16_bf16 with the docs split
//     into hi + mid as they are staged in LDS and three products per pair
//     (hi.hi + hi.mid + mid.hi, fp32 accumulate): an approximate score s'
//     within eps(d) * |q| * |doc| of the exact dot product. Each lane keeps,
//     for its two queries, the best four (s', index) of the docs it owns (the
//     MFMA C layout gives a lane 16 docs of every 32-doc block); any doc a
//     lane drops is no better than its list's fourth entry, which the lane
//     reports as its discard bound. Doc norms are taken during the split.
//  3. score_merge_kernel: one workgroup per query merges the 16 candidates of
//     every stage-1 workgroup to the best 16 by s', rescoring them exactly
//     (float64 dot products rounded to float32) and ordering them by (value
//     desc, index asc). The result is exact when the k-th rescored value
//     exceeds every discard bound (lanes' and the merge's own 16th) plus eps
//     * |q| * max|doc|: then no dropped doc can reach the top k. Otherwise
//     (near-ties of more than a few docs around the k-th score, e.g.
//     duplicated rows) the same workgroup scans every doc exactly.
// The output is the exact top k by float32-rounded dot product, larger first,
// equal values by lower index (tensor/reduce.go:269-297); NaN scores rank
// below every number.
constexpr int kSQB = 256;    // queries per block
constexpr int kSDB = 128;    // docs per tile
constexpr int kSKL = 4;      // entries per lane list
constexpr int kSCand = 16;   // candidates per (query, workgroup): 2 doc waves x 2 lane halves x kSKL
constexpr int kSMerge = 16;  // candidates rescored per query
constexpr int kSMaxK = 16;
constexpr int kSMaxWG = 256;

typedef __bf16 sbf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t su32x4 __attribute__((ext_vector_type(4)));

// LDS slabs (ROWS rows of 32 bf16) chunk-major: chunk c of row r at 16-byte
// slot c * ROWS + (r ^ 2c), conflict-free for the 16-byte staging writes
// (four lanes per row) and operand reads (consecutive rows of one chunk) on
// gfx950's LDS (the layout of the split GEMM, gemm.hip).
template <int ROWS>
__device__ __forceinline__ int s_chunk(int r, int c) { return (c * ROWS + (r ^ (2 * c))) * 8; }

// 1. One wave per query row of the block: hi/mid planes [kSQB x d] (zero rows
// past nq) and |q| in float64 rounded up to float32.
__global__ __launch_bounds__(64) void score_qsplit_kernel(const float* __restrict__ q, int64_t ldq, int nq, int d,
                                                          uint16_t* __restrict__ qh, uint16_t* __restrict__ qm,
                                                          float* __restrict__ qnorm) {
  const int r = blockIdx.x, lane = threadIdx.x;
  double ss = 0;
  for (int t = lane; t < d; t += 64) {
    const float x = r < nq ? q[(int64_t)r * ldq + t] : 0.f;
    const Split3 sp = split3(x);
    qh[(int64_t)r * d + t] = (uint16_t)(sp.h >> 16);
    qm[(int64_t)r * d + t] = (uint16_t)(sp.m >> 16);
    ss += (double)x * x;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if (lane == 0) qnorm[r] = (float)(sqrt(ss) * (1.0 + 1e-6));
}

struct Stage1Params {
  const uint16_t* qh;
  const uint16_t* qm;
  const float* docs;
  int64_t ldd, nd;
  int d, nq, nwg;
  int64_t nblocks;  // 32-doc blocks
  float* cv;
  int32_t* ci;
  float* bound;
  float* wgnorm;
};

// 2. Workgroup w: docs [32*b0, min(32*b1, nd)) with b = w*nblocks/nwg. Eight
// waves: wave (wq, wd) owns queries 64*wq .. +63 (two 32-column blocks) and
// docs 64*wd .. +63 of each 128-doc tile (two 32-row blocks). K advances in
// 32-wide slabs over (tile, slab) items: item i in LDS buffer i&1, item i+1
// split from registers during item i's MFMAs, item i+2 loading.
__global__ __launch_bounds__(512) void score_stage1_kernel(Stage1Params p) {
  __shared__ __attribute__((aligned(16))) uint16_t Dp[2][2][kSDB * 32];
  __shared__ __attribute__((aligned(16))) uint16_t Qp[2][2][kSQB * 32];
  __shared__ float red[8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wq = wave >> 1, wd = wave & 1;
  const int w = blockIdx.x;
  const int64_t b0 = (int64_t)w * p.nblocks / p.nwg, b1 = (int64_t)(w + 1) * p.nblocks / p.nwg;
  const int64_t dbeg = b0 * 32, dend = min(b1 * 32, p.nd);
  const int ntile = (int)((b1 - b0 + 3) / 4);
  const int nk = p.d / 32;
  const int d = p.d;

  // staging: doc row tid/4, chunk tid%4 (8 floats); query rows (tid + 512 i)/4
  const int srow = tid >> 2, sc = tid & 3;
  struct Regs {
    f32x4 a[2];
    su32x4 b[4];
  };
  auto load = [&](Regs& g, int item) {
    const int t = item / nk, kt = item - t * nk;
    const int64_t row = min(dbeg + (int64_t)t * kSDB + srow, p.nd - 1);
    const float* src = p.docs + row * p.ldd + kt * 32 + sc * 8;
    g.a[0] = *reinterpret_cast<const f32x4*>(src);
    g.a[1] = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int idx = tid + 512 * (i & 1), qr = idx >> 2, c = idx & 3;
      const uint16_t* pl = (i < 2) ? p.qh : p.qm;
      g.b[i] = *reinterpret_cast<const su32x4*>(pl + (int64_t)qr * d + kt * 32 + c * 8);
    }
  };
  float ss = 0.f, mx = 0.f;
  auto split_store = [&](const Regs& g, int buf, int item) {
    const int t = item / nk, kt = item - t * nk;
    uint32_t h[8], m[8];
    if (kt == 0) ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float x = g.a[e >> 2][e & 3];
      const Split3 sp = split3(x);
      h[e] = sp.h;
      m[e] = sp.m;
      ss = fmaf(x, x, ss);
    }
    const int o = s_chunk<kSDB>(srow, sc);
    *reinterpret_cast<uint4*>(&Dp[buf][0][o]) =
        make_uint4(pack_hi16(h[0], h[1]), pack_hi16(h[2], h[3]), pack_hi16(h[4], h[5]), pack_hi16(h[6], h[7]));
    *reinterpret_cast<uint4*>(&Dp[buf][1][o]) =
        make_uint4(pack_hi16(m[0], m[1]), pack_hi16(m[2], m[3]), pack_hi16(m[4], m[5]), pack_hi16(m[6], m[7]));
    if (kt == nk - 1) {  // the row's sum of squares is complete: four threads hold its parts
      float tot = ss + __shfl_xor(ss, 1, 64);
      tot += __shfl_xor(tot, 2, 64);
      if (dbeg + (int64_t)t * kSDB + srow < dend) mx = fmaxf(mx, tot);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int idx = tid + 512 * (i & 1), qr = idx >> 2, c = idx & 3;
      *reinterpret_cast<su32x4*>(&Qp[buf][i >> 1][s_chunk<kSQB>(qr, c)]) = g.b[i];
    }
  };
  const int hh = lane >> 5;
  auto read_ops = [&](int buf, int s, sbf16x8 (&oa)[2][2], sbf16x8 (&ob)[2][2]) {
    // 32 rows further is 32 slots further
    const int ca = s_chunk<kSDB>(wd * 64 + (lane & 31), 2 * s + hh);
    const int cb = s_chunk<kSQB>(wq * 64 + (lane & 31), 2 * s + hh);
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int i = 0; i < 2; i++) {
        oa[t][i] = *reinterpret_cast<const sbf16x8*>(&Dp[buf][t][ca + 32 * 8 * i]);
        ob[t][i] = *reinterpret_cast<const sbf16x8*>(&Qp[buf][t][cb + 32 * 8 * i]);
      }
  };
  f32x16 acc[2][2];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
  };
  zero_acc();
  // doc blocks of this wave inside the range in the item's tile (0, 1 or 2)
  auto nvalid = [&](int item) {
    const int t = item / nk;
    const int64_t blk0 = dbeg + (int64_t)t * kSDB + wd * 64;
    return (int)min<int64_t>(2, max<int64_t>(0, (dend - blk0 + 31) / 32));
  };
  // NV: doc blocks of this wave inside the range (a tile's constant, so the
  // slab loop below is compiled once per value and has no branch)
  auto mfma_step = [&](const sbf16x8 (&oa)[2][2], const sbf16x8 (&ob)[2][2], auto nvc) {
    constexpr int NV = decltype(nvc)::value;
    // mid.hi, hi.mid, then hi.hi (smallest first)
#pragma unroll
    for (int i = 0; i < NV; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(oa[1][i], ob[0][j], acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(oa[0][i], ob[1][j], acc[i][j], 0, 0, 0);
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(oa[0][i], ob[0][j], acc[i][j], 0, 0, 0);
      }
  };
  // lane lists: query column j of this wave, best kSKL (value desc, index asc)
  float lv[2][kSKL];
  int li[2][kSKL];
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int e = 0; e < kSKL; e++) {
      lv[j][e] = -INFINITY;
      li[j][e] = INT32_MAX;
    }
  // C element (i, j, r) of lane l: doc row 8*(r/4) + 4*(l/32) + r%4 of block i,
  // query column l%32 of block j
  auto epilogue = [&](int item) {
    const int t = item / nk;
    const int64_t tile0 = dbeg + (int64_t)t * kSDB + wd * 64 + 4 * hh;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int64_t doc = tile0 + i * 32 + 8 * (r >> 2) + (r & 3);
        const bool ok = doc < dend;
#pragma unroll
        for (int j = 0; j < 2; j++) {
          float cv = ok ? acc[i][j][r] : NAN;
          int ci = (int)doc;
#pragma unroll
          for (int e = 0; e < kSKL; e++) {
            const bool b = better(cv, ci, lv[j][e], li[j][e]);
            const float tv = lv[j][e];
            const int ti = li[j][e];
            lv[j][e] = b ? cv : tv;
            li[j][e] = b ? ci : ti;
            cv = b ? tv : cv;
            ci = b ? ti : ci;
          }
        }
      }
    zero_acc();
  };
  // items i0 .. last of one tile (nk slabs)
  auto body = [&](int item, int last, auto nvc, const Regs& use, Regs& fill) {
    const int buf = item & 1;
    load(fill, min(item + 2, last));
    sbf16x8 a0[2][2], b0[2][2], a1[2][2], b1[2][2];
    read_ops(buf, 0, a0, b0);
    read_ops(buf, 1, a1, b1);
    mfma_step(a0, b0, nvc);
    split_store(use, buf ^ 1, item + 1);
    mfma_step(a1, b1, nvc);
    __syncthreads();
  };
  auto tile = [&](int i0, auto nvc) {
    const int last = i0 + nk - 1;
    Regs rA, rB;
    load(rA, i0);
    split_store(rA, i0 & 1, i0);
    load(rA, min(i0 + 1, last));
    __syncthreads();
    int item = i0;
    for (; item + 2 <= last; item += 2) {
      body(item, last, nvc, rA, rB);
      body(item + 1, last, nvc, rB, rA);
    }
    if (item + 1 <= last) {
      body(item, last, nvc, rA, rB);
      item++;
    }
    sbf16x8 a0[2][2], b0[2][2], a1[2][2], b1[2][2];
    read_ops(item & 1, 0, a0, b0);
    read_ops(item & 1, 1, a1, b1);
    mfma_step(a0, b0, nvc);
    mfma_step(a1, b1, nvc);
  };
  for (int t = 0; t < ntile; t++) {
    const int i0 = t * nk;
    const int nv = nvalid(i0);
    // a wave with no doc block in range computes one (the epilogue ignores it)
    if (nv == 2) tile(i0, std::integral_constant<int, 2>{});
    else tile(i0, std::integral_constant<int, 1>{});
    epilogue(i0);
    __syncthreads();  // the next tile's first slab overwrites the buffers read above
  }
  // candidates and discard bounds of this workgroup
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int qr = wq * 64 + j * 32 + (lane & 31);
    if (qr < p.nq) {
      const int64_t base = ((int64_t)qr * p.nwg + w) * kSCand + wd * 8 + hh * kSKL;
#pragma unroll
      for (int e = 0; e < kSKL; e++) {
        p.cv[base + e] = lv[j][e];
        p.ci[base + e] = li[j][e];
      }
      p.bound[((int64_t)qr * p.nwg + w) * 4 + wd * 2 + hh] = lv[j][kSKL - 1];
    }
  }
  mx = wave_max(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  if (tid == 0) {
    float m = red[0];
    for (int i = 1; i < 8; i++) m = fmaxf(m, red[i]);
    p.wgnorm[w] = m;
  }
}

// float64 dot product of two float32 rows of length d (d % 4 == 0, 16-byte
// aligned), rounded to float32.
__device__ __forceinline__ float exact_dot(const float* __restrict__ a, const float* __restrict__ b, int d) {
  double s = 0;
  for (int t = 0; t < d; t += 4) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(a + t), y = *reinterpret_cast<const f32x4*>(b + t);
    s = fma((double)x[0], (double)y[0], s);
    s = fma((double)x[1], (double)y[1], s);
    s = fma((double)x[2], (double)y[2], s);
    s = fma((double)x[3], (double)y[3], s);
  }
  return (float)s;
}

struct MergeParams {
  const float* cv;
  const int32_t* ci;
  const float* bound;
  const float* wgnorm;
  const float* qnorm;
  const float* q;
  int64_t ldq;
  const float* docs;
  int64_t ldd, nd;
  int nwg, d, k;
  float eps;  // score error bound of stage 1 per |q| |doc|
  int32_t* idx;
  float* val;
  int32_t* flag;
};

// Sorting networks over (value, index) pairs in the full order (value desc,
// index asc). NaN candidates enter as (-inf, INT32_MAX), below every pair
// that stands for a doc.
__device__ __forceinline__ void cas_desc(float& va, int& ia, float& vb, int& ib) {
  // after the call (va, ia) is the better of the two
  const bool sw = better(vb, ib, va, ia);
  const float tv = va;
  const int ti = ia;
  va = sw ? vb : va;
  ia = sw ? ib : ia;
  vb = sw ? tv : vb;
  ib = sw ? ti : ib;
}

// Bitonic sort of N register pairs, best first.
template <int N>
__device__ __forceinline__ void sort_list(float (&v)[N], int (&ix)[N]) {
#pragma unroll
  for (int k = 2; k <= N; k *= 2)
#pragma unroll
    for (int j = k / 2; j > 0; j /= 2)
#pragma unroll
      for (int i = 0; i < N; i++) {
        const int l = i ^ j;
        if (l > i) {
          if ((i & k) == 0) cas_desc(v[i], ix[i], v[l], ix[l]);
          else cas_desc(v[l], ix[l], v[i], ix[i]);
        }
      }
}

// Two sorted lists (best first) -> the best N of their union, sorted: the
// pairwise better of A[i] and B[N-1-i] is a bitonic sequence holding those
// N, then half-cleaners sort it.
template <int N>
__device__ __forceinline__ void merge_lists(float (&v)[N], int (&ix)[N], const float (&bv)[N], const int (&bi)[N]) {
#pragma unroll
  for (int i = 0; i < N; i++)
    if (better(bv[N - 1 - i], bi[N - 1 - i], v[i], ix[i])) {
      v[i] = bv[N - 1 - i];
      ix[i] = bi[N - 1 - i];
    }
#pragma unroll
  for (int j = N / 2; j > 0; j /= 2)
#pragma unroll
    for (int i = 0; i < N; i++) {
      const int l = i ^ j;
      if (l > i) cas_desc(v[i], ix[i], v[l], ix[l]);
    }
}

// 3. Four waves per query: each thread loads and sorts kSMerge candidates,
// the lanes of a wave merge their lists pairwise (lane ^ 1, ^ 2, ... ^ 32)
// until every lane holds the wave's best kSMerge, wave 0 merges the four
// waves' lists, rescores them exactly and checks the bound.
__global__ __launch_bounds__(256) void score_merge_kernel(MergeParams p) {
  __shared__ float sv[4][kSMerge];
  __shared__ int si[4][kSMerge];
  __shared__ float sx[4], sd[4];
  __shared__ int s_flag;
  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ncand = p.nwg * kSCand;  // at most kSMaxWG * kSCand = kSMerge per thread
  static_assert(kSMaxWG * kSCand == 256 * kSMerge, "one list of kSMerge candidates per thread");
  float v[kSMerge];
  int ix[kSMerge];
#pragma unroll
  for (int u = 0; u < kSMerge; u++) {
    const int t = tid + 256 * u;
    const bool ok = t < ncand;
    const float c = ok ? p.cv[q * ncand + t] : NAN;
    const bool nan = !(c == c);
    v[u] = nan ? -INFINITY : c;
    ix[u] = (ok && !nan) ? p.ci[q * ncand + t] : INT32_MAX;
  }
  float xb = -INFINITY, dn2 = 0.f;
  for (int t = tid; t < p.nwg * 4; t += 256) xb = fmaxf(xb, p.bound[q * p.nwg * 4 + t]);
  for (int t = tid; t < p.nwg; t += 256) dn2 = fmaxf(dn2, p.wgnorm[t]);
  sort_list(v, ix);
#pragma unroll
  for (int m = 1; m < 64; m *= 2) {
    float bv[kSMerge];
    int bi[kSMerge];
#pragma unroll
    for (int u = 0; u < kSMerge; u++) {
      bv[u] = __shfl_xor(v[u], m, 64);
      bi[u] = __shfl_xor(ix[u], m, 64);
    }
    merge_lists(v, ix, bv, bi);
  }
  xb = wave_max(xb);
  dn2 = wave_max(dn2);
  if (lane == 0) {
#pragma unroll
    for (int u = 0; u < kSMerge; u++) {
      sv[wave][u] = v[u];
      si[wave][u] = ix[u];
    }
    sx[wave] = xb;
    sd[wave] = dn2;
  }
  __syncthreads();
  if (wave == 0) {
    for (int w2 = 1; w2 < 4; w2++) {
      float bv[kSMerge];
      int bi[kSMerge];
#pragma unroll
      for (int u = 0; u < kSMerge; u++) {
        bv[u] = sv[w2][u];
        bi[u] = si[w2][u];
      }
      merge_lists(v, ix, bv, bi);
      xb = fmaxf(xb, sx[w2]);
      dn2 = fmaxf(dn2, sd[w2]);
    }
    xb = fmaxf(xb, v[kSMerge - 1]);  // the merge's own discards
    // exact rescoring: float64 dot products of the query with the kSMerge
    // candidates, the wave's lanes taking four columns each per 256, rounded to
    // float32; lane u keeps candidate u's value
    double part[kSMerge];
#pragma unroll
    for (int u = 0; u < kSMerge; u++) part[u] = 0.0;
    const float* qrow = p.q + q * p.ldq;
    for (int t = 4 * lane; t < p.d; t += 256) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(qrow + t);
#pragma unroll
      for (int u = 0; u < kSMerge; u++) {
        // an empty slot reads doc 0 and is ignored below: no branch, so the
        // loads of all slots are in flight together
        const int64_t row = ix[u] == INT32_MAX ? 0 : ix[u];
        const f32x4 y = *reinterpret_cast<const f32x4*>(p.docs + row * p.ldd + t);
        part[u] = fma((double)x[0], (double)y[0], part[u]);
        part[u] = fma((double)x[1], (double)y[1], part[u]);
        part[u] = fma((double)x[2], (double)y[2], part[u]);
        part[u] = fma((double)x[3], (double)y[3], part[u]);
      }
    }
    float e = -INFINITY;
    int me = INT32_MAX;
#pragma unroll
    for (int u = 0; u < kSMerge; u++) {
      double t = part[u];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) t += __shfl_xor(t, o, 64);
      if (lane == u && ix[u] != INT32_MAX) {
        e = (float)t;
        me = ix[u];
      }
    }
    // rank of this lane's exact value among the kSMerge
    int rank = 0;
#pragma unroll
    for (int u = 0; u < kSMerge; u++) {
      const float eu = __shfl(e, u, 64);
      const int iu = __shfl(me, u, 64);
      rank += better(eu, iu, e, me) ? 1 : 0;
    }
    // the k-th best exact value: the lane of rank k-1
    const uint64_t at = __ballot(lane < kSMerge && rank == p.k - 1);
    const int src = at ? __ffsll((unsigned long long)at) - 1 : 0;
    const float ek = __shfl(e, src, 64);
    const int ik = __shfl(me, src, 64);
    const float margin = p.eps * p.qnorm[q] * sqrtf(dn2) * (1.f + 1e-4f);
    // no lane of rank k-1: fewer than k candidates stand for docs
    const bool exact = at != 0 && ik != INT32_MAX && ek > xb + margin;  // false for NaN: flagged
    if (exact && lane < kSMerge && rank < p.k) {
      p.idx[q * p.k + rank] = me;
      if (p.val) p.val[q * p.k + rank] = e;
    }
    if (lane == 0) {
      p.flag[q] = exact ? 0 : 1;
      s_flag = exact ? 0 : 1;
    }
  }  // wave 0
  __syncthreads();
  if (s_flag == 0) return;
  // flagged (near-ties of more than a lane list, or fewer than k
  // candidates): the exact scan, float64 dot products against every doc,
  // each wave a list of the best k, merged into wave 0's in wave order
  WaveList W;
  const float* qrow = p.q + q * p.ldq;
  for (int64_t base = 0; base < p.nd; base += 256) {
    const int64_t j = base + tid;
    const bool ok = j < p.nd;
    W.offer(p.k, lane, ok ? exact_dot(qrow, p.docs + j * p.ldd, p.d) : NAN, ok ? (int)j : INT32_MAX);
  }
  __syncthreads();  // every wave is done with sv / si
  if (lane < p.k) {
    sv[wave][lane] = W.lv;
    si[wave][lane] = W.li;
  }
  __syncthreads();
  if (wave == 0) {
    for (int w2 = 1; w2 < 4; w2++)
      W.offer(p.k, lane, lane < p.k ? sv[w2][lane] : NAN, lane < p.k ? si[w2][lane] : INT32_MAX);
    if (lane < p.k) {
      p.idx[q * p.k + lane] = W.li == INT32_MAX ? -1 : W.li;
      if (p.val) p.val[q * p.k + lane] = W.li == INT32_MAX ? NAN : W.lv;
    }
  }
}

struct ScoreScratch {
  uint16_t *qh, *qm;
  float *qnorm, *cv, *bound, *wgnorm;
  int32_t *ci, *flag;
};

size_t score_layout(int d, int nwg, char* base, ScoreScratch* s) {
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* ptr = base ? base + off : nullptr;
    off += (bytes + 255) & ~(size_t)255;
    return ptr;
  };
  ScoreScratch t;
  t.qh = (uint16_t*)take((size_t)kSQB * d * 2);
  t.qm = (uint16_t*)take((size_t)kSQB * d * 2);
  t.qnorm = (float*)take(kSQB * 4);
  t.cv = (float*)take((size_t)kSQB * nwg * kSCand * 4);
  t.ci = (int32_t*)take((size_t)kSQB * nwg * kSCand * 4);
  t.bound = (float*)take((size_t)kSQB * nwg * 4 * 4);
  t.wgnorm = (float*)take((size_t)nwg * 4);
  t.flag = (int32_t*)take(kSQB * 4);
  if (s) *s = t;
  return off;
}

}  // namespace

int score_workgroups(int64_t nd, int cus) {
  const int64_t nb = (nd + 31) / 32;
  return (int)std::max<int64_t>(1, std::min<int64_t>({nb, (int64_t)kSMaxWG, (int64_t)std::max(cus, 1)}));
}

size_t score_scratch_bytes(int d, int nwg) { return score_layout(d, nwg, nullptr, nullptr); }

bool score_fused_ok(const float* q, int64_t ldq, const float* docs, int64_t ldd, int d, int topk) {
  auto al = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
  return d > 0 && d % 32 == 0 && topk >= 1 && topk <= kSMaxK && al(q) && al(docs) && ldq % 4 == 0 && ldd % 4 == 0;
}

int launch_score_topk(fa_ctx* ctx, const float* q, int64_t nq, int64_t ldq, const float* docs, int64_t nd,
                      int64_t ldd, int d, int topk, int32_t* idx, float* val, void* scratch, int nwg,
                      hipStream_t s) {
  if (!score_fused_ok(q, ldq, docs, ldd, d, topk))
    return set_error(ctx, FA_ERR_ARG, "Similarities: fused scoring needs d %% 32 == 0, 1 <= k <= %d and 16-byte "
                     "aligned rows", kSMaxK);
  ScoreScratch sc;
  score_layout(d, nwg, static_cast<char*>(scratch), &sc);
  // stage-1 error per |q| |doc|: the dropped split terms (3 * 2^-14 + 2 * 2^-21
  // + 2^-28) and fp32 accumulation over 3d products (3d * 2^-24, times 1.02 for
  // the kept terms' magnitude), plus the rounding of a rescored value
  const float eps = (float)(3.0 * std::ldexp(1.0, -14) + 2.0 * std::ldexp(1.0, -21) + std::ldexp(1.0, -28) +
                            1.02 * 3.0 * d * std::ldexp(1.0, -24) + std::ldexp(1.0, -22));
  for (int64_t q0 = 0; q0 < nq; q0 += kSQB) {
    const int nb = (int)std::min<int64_t>(kSQB, nq - q0);
    const float* qb = q + q0 * ldq;
    hipLaunchKernelGGL(score_qsplit_kernel, dim3(kSQB), dim3(64), 0, s, qb, ldq, nb, d, sc.qh, sc.qm, sc.qnorm);
    Stage1Params p1;
    p1.qh = sc.qh; p1.qm = sc.qm; p1.docs = docs; p1.ldd = ldd; p1.nd = nd; p1.d = d; p1.nq = nb; p1.nwg = nwg;
    p1.nblocks = (nd + 31) / 32; p1.cv = sc.cv; p1.ci = sc.ci; p1.bound = sc.bound; p1.wgnorm = sc.wgnorm;
    hipLaunchKernelGGL(score_stage1_kernel, dim3(nwg), dim3(512), 0, s, p1);
    MergeParams pm;
    pm.cv = sc.cv; pm.ci = sc.ci; pm.bound = sc.bound; pm.wgnorm = sc.wgnorm; pm.qnorm = sc.qnorm; pm.q = qb;
    pm.ldq = ldq; pm.docs = docs; pm.ldd = ldd; pm.nwg = nwg; pm.d = d; pm.k = topk; pm.eps = eps;
    pm.idx = idx + q0 * topk; pm.val = val ? val + q0 * topk : nullptr; pm.flag = sc.flag;
    pm.nd = nd;
    hipLaunchKernelGGL(score_merge_kernel, dim3(nb), dim3(256), 0, s, pm);
  }
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

// ---------------------------------------------------------------------------
// Scratch of fa_similarities_topk_dev_noalloc: the fused path's query planes,
// norms, candidates, discard bounds, doc norms and flags for one block of 256
// queries, in a fixed array of each device (held until the process ends). Its
// device address comes from hipGetSymbolAddress once per device, at context
// creation on that device; host code never passes the array's name itself.
// The array of a device belongs to the first context that calls the entry
// point there, until that context is destroyed: calls from other contexts
// on that device are refused (FA_ERR_STATE) instead of racing on it, and the
// owner's calls are ordered by its one stream. No kernel relies on the
// array's previous contents (every value read in a call is written earlier
// in the same call).
constexpr size_t kNoAllocScratchBytes = (size_t)12 << 20;
__device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
const fa_ctx* g_scratch_owner[kMaxDevices] = {};
}  // namespace

void noalloc_release(const fa_ctx* ctx) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  for (auto& o : g_scratch_owner)
    if (o == ctx) o = nullptr;
}

// Claims the device's array for ctx (or finds it already ctx's).
int noalloc_claim(fa_ctx* ctx) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  const fa_ctx*& o = g_scratch_owner[ctx->device];
  if (o && o != ctx)
    return set_error(ctx, FA_ERR_STATE,
                     "Similarities (no-alloc): the fixed scratch of device %d belongs to another context until that "
                     "context is destroyed (calls from two contexts would race on it)",
                     ctx->device);
  o = ctx;
  return FA_OK;
}

int noalloc_scratch_init(fa_ctx* ctx) {
  const int dev = ctx->device;
  if (dev < 0 || dev >= kMaxDevices) return set_error(ctx, FA_ERR_UNSUPPORTED, "device %d outside 0..%d", dev,
                                                      kMaxDevices - 1);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev]) return FA_OK;
  void* ptr = nullptr;
  FA_HIP_CHECK(ctx, hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));  // the device is current (fa_create)
  g_scratch_ptr[dev] = ptr;
  return FA_OK;
}

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

extern "C" int fa_similarities_topk_dev_noalloc(fa_ctx* ctx, const float* queries, int64_t nq, const float* docs,
                                                int64_t nd, int32_t d, int32_t topk, int32_t* idx, float* val) {
  using fa::set_error;
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "Similarities: ctx is NULL");
  if (nq < 0 || nd <= 0 || d <= 0)
    return set_error(ctx, FA_ERR_ARG, "Similarities: shapes [%lld x %d] and [%lld x %d]", (long long)nq, d,
                     (long long)nd, d);
  if (topk < 1 || topk > fa::kSMaxK || topk > nd)
    return set_error(ctx, FA_ERR_ARG, "Similarities (no-alloc): k=%d outside 1..min(%d, %lld)", topk, fa::kSMaxK,
                     (long long)nd);
  if (nq == 0) return FA_OK;
  if (!queries || !docs || !idx) return set_error(ctx, FA_ERR_ARG, "Similarities: NULL buffer");
  if (d > 2048) return set_error(ctx, FA_ERR_ARG, "Similarities (no-alloc): d=%d exceeds the fixed scratch's 2048", d);
  if (!fa::score_fused_ok(queries, d, docs, d, d, topk))
    return set_error(ctx, FA_ERR_ARG, "Similarities (no-alloc): needs d %% 32 == 0 and 16-byte aligned rows, got d=%d",
                     d);
  const int nwg = fa::score_workgroups(nd, ctx->cu_count);
  const size_t need = fa::score_scratch_bytes(d, nwg);
  if (need > fa::kNoAllocScratchBytes)
    return set_error(ctx, FA_ERR_ARG, "Similarities (no-alloc): d=%d needs %zu bytes of scratch, the fixed array has %zu "
                     "(d <= 2048 fits)", d, need, fa::kNoAllocScratchBytes);
  void* ptr = ctx->device >= 0 && ctx->device < fa::kMaxDevices ? fa::g_scratch_ptr[ctx->device] : nullptr;
  if (!ptr) return set_error(ctx, FA_ERR_STATE, "Similarities (no-alloc): scratch address of device %d unknown",
                             ctx->device);
  if (const int rc = fa::noalloc_claim(ctx)) return rc;
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  return fa::launch_score_topk(ctx, queries, nq, d, docs, nd, d, d, topk, idx, val, ptr, nwg, ctx->stream);
}
