// Bidirectional attention for gfx950.
//
// attention_varlen_kernel (the model path): packed variable-length
// sequences, grouped-query heads (every query head h reads key/value head
// h / (H/Hkv)), head_dim 256 or 512, optional sliding window |i-j| < window, padding
// implied by the packing (a sequence's keys are exactly its valid tokens).
// Computes softmax(scale * q.k^T) . v with an online softmax over key tiles,
// never materialising scores or masks. Masked keys get weight exactly 0, and
// so does any weight whose exponent is below -87 (the reference's flush,
// internal/kernel/generic.go:278-307), as in tensor.AttentionScaled
// (tensor/attention.go:67-83) + blas.AttentionBlock (internal/blas/
// attention.go:61-136) with PaddingMask + WindowMask (attention.go:33-42,
// 97-107; models/gemma/embed.go:168-186).
//
// Formulation (v_mfma_f32_16x16x4_f32; lane l of a 16x16 result holds
// column l%16 and rows 4*(l/16)+r, r=0..3). A work item is (sequence, block
// of 32 queries, head); its workgroup is four waves: waves 2b and 2b+1 own
// the same 16 queries (block b) and the two halves of the head dimension.
// Per tile of 16 keys each wave computes the partial scores over its 128
// dimensions as S^T[key, query] = K . Q^T (A = K rows from LDS, B = Q in
// VGPRs), so lane l holds the scores of query l%16 against keys
// 4*(l/16)+r; the pair exchanges partial scores through LDS and adds them
// in one order (half 0 + half 1), so both hold the same scores and softmax
// statistics (lane-local plus two shuffles). The probabilities are already
// the A operand of O[query, d] += P . V (B = V rows from LDS) when the k
// index of MFMA c in lane group g is taken as key 4g+c, and each wave
// accumulates its half of O. Splitting the head dimension halves the Q and
// O registers per wave (two waves per SIMD) and doubles the waves over a
// batch.
//
// K and V tiles reach LDS by direct global->LDS loads (global_load_lds,
// one 1 KB row per wave instruction) into two buffers, the next tile
// loading while the current one is computed; a row's 16-byte chunks are
// XOR-swizzled by row so the operand reads hit distinct banks. The
// barriers use explicit counter waits so the exchange barrier does not wait
// for the next tile's loads.
//
// attention_generic_kernel (the tensor.AttentionScaled drop-in): arbitrary
// B, H, T, S, D <= 512, strides and an additive mask tensor, one wavefront
// per query row, the reference's algebra: raw scores, + mask/scale, max,
// exp(scale*row - scale*max) with the flush, P.V, times 1/sum.

#include <cstdlib>

#include "fa_internal.h"
#include "device_math.h"

namespace fa {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int QW = 16;                   // queries per wave pair
constexpr int QBLK = 2 * QW;             // queries per work item (two pairs)
constexpr int KT = 16;                   // keys per tile
constexpr float kNegBig = -1e30f;

struct VarlenParams {
  const float* qkv;
  float* out;
  const int32_t* cu;
  const int32_t* items;  // triples (seq, q0, head)
  int32_t H, Hkv;
  int32_t window;
  float scale;
  int64_t row0;  // packed row of qkv's and out's first row
  // kparts > 1: each item's key range is cut into kparts runs of whole
  // tiles, one workgroup each; they write unnormalised partial outputs and
  // (max, sum) pairs to part for attention_combine_kernel
  int32_t kparts;
  int64_t rows;  // rows of qkv and out (the partial buffers' row count)
  float* part;
};

// ---- the model path's kernel ------------------------------------------------
// Direct-to-LDS tile loads: each 1 KB of a K or V row of a tile (256
// floats; a row is 1 KB at head_dim 256, 2 KB at 512) is one
// global_load_lds_dwordx4 of a wave (64 lanes x 16 bytes, LDS address =
// base + 16 * lane), into two LDS buffers. A row's 16-byte chunk c is stored
// at position c ^ (row & 15) (the XOR stays within each 1 KB part), so the
// score reads (16 rows, one chunk each) and the V reads (4 rows x 4 chunks)
// hit distinct banks. Keys past the range load the last valid row (finite
// values; their weights are 0).
constexpr int DL_NT = 256;

__device__ __forceinline__ int dl_pos(int row, int chunk) { return chunk ^ (row & 15); }

// Workgroup barrier with an explicit counter wait (s_waitcnt encoding WAIT)
// instead of __syncthreads()'s release fence, which would also wait for the
// next tile's loads to LDS. The signal fences keep the compiler from moving
// LDS accesses across it.
template <int WAIT>
__device__ __forceinline__ void dl_barrier() {
  __builtin_amdgcn_s_waitcnt(WAIT);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int HD>
__global__ __launch_bounds__(DL_NT) void attention_varlen_kernel(VarlenParams p) {
  constexpr int HALF = HD / 2;  // head dimensions per wave
  constexpr int ROWF = HD;      // floats per LDS row (unpadded)
  // separate objects per buffer, so the compiler can tell the tile being
  // read from the one being loaded and need not wait for the loads
  __shared__ __attribute__((aligned(16))) float K0[KT * ROWF];
  __shared__ __attribute__((aligned(16))) float V0[KT * ROWF];
  __shared__ __attribute__((aligned(16))) float K1[KT * ROWF];
  __shared__ __attribute__((aligned(16))) float V1[KT * ROWF];
  __shared__ __attribute__((aligned(16))) float Sx[4][64 * 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int qb = wave >> 1, half = wave & 1;
  const int g = lane >> 4;
  const int lq = lane & 15;

  const int item = blockIdx.x / p.kparts, part = blockIdx.x % p.kparts;
  const int seq = p.items[3 * item];
  const int q0 = p.items[3 * item + 1];
  const int h = p.items[3 * item + 2];
  const int hk = h / (p.H / p.Hkv);
  const int L = p.cu[seq + 1] - p.cu[seq];
  const int64_t start = p.cu[seq] - p.row0;  // the sequence's first row in qkv and out
  const int W = (p.H + 2 * p.Hkv) * HD;
  const int dofs = half * HALF;
  const float* qbase = p.qkv + (int64_t)start * W + (int64_t)h * HD + dofs;
  const float* kbase = p.qkv + (int64_t)start * W + (int64_t)(p.H + hk) * HD;
  const float* vbase = p.qkv + (int64_t)start * W + (int64_t)(p.H + p.Hkv + hk) * HD;

  const int qw0 = q0 + qb * QW;
  const int qi = qw0 + lq;
  const bool qvalid = qi < L;
  f32x4 qreg[HALF / 16];
  {
    const float* qr = qbase + (int64_t)(qvalid ? qi : 0) * W;
#pragma unroll
    for (int sg = 0; sg < HALF / 16; sg++) {
      f32x4 v = *reinterpret_cast<const f32x4*>(qr + sg * 16 + g * 4);
      qreg[sg] = qvalid ? v : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  f32x4 oacc[HALF / 16];
#pragma unroll
  for (int db = 0; db < HALF / 16; db++) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegBig;
  float l_part = 0.f;

  const int qlast = min(q0 + QBLK, L) - 1;
  int kbeg = 0, kend = L;
  if (p.window > 0) {
    kbeg = max(0, q0 - p.window + 1);
    kend = min(L, qlast + p.window);
  }
  if (p.kparts > 1) {  // this part's run of tiles (possibly none)
    const int per = ((kend - kbeg + KT - 1) / KT + p.kparts - 1) / p.kparts;
    const int kb = kbeg + part * per * KT;
    kend = min(kend, kb + per * KT);
    kbeg = kb;
  }

  // wave w loads rows w, w+4, w+8, w+12 of K and of V, 1 KB (64 lanes x 16
  // bytes) per instruction
  auto issue_tile = [&](int k0, float* Kb, float* Vb) {
#pragma unroll
    for (int j = 0; j < KT / 4; j++) {
      const int r = wave + 4 * j;
      const int64_t key = min(k0 + r, kend - 1);
#pragma unroll
      for (int part = 0; part < HD / 256; part++) {
        const int chunk = dl_pos(r, part * 64 + lane);  // the global chunk that lands at this position
        __builtin_amdgcn_global_load_lds(kbase + key * W + chunk * 4,
                                         (__attribute__((address_space(3))) void*)&Kb[r * ROWF + part * 256], 16, 0,
                                         0);
        __builtin_amdgcn_global_load_lds(vbase + key * W + chunk * 4,
                                         (__attribute__((address_space(3))) void*)&Vb[r * ROWF + part * 256], 16, 0,
                                         0);
      }
    }
  };
  if (kbeg < kend) issue_tile(kbeg, K0, V0);

  auto step = [&](int k0, const float* Kc, const float* Vc, float* Kn, float* Vn) {
    // this wave's loads of the tile have landed; after the barrier, every
    // wave's have, and the other buffer is free (its tile was consumed)
    dl_barrier<0x0070>();  // vmcnt(0) lgkmcnt(0): the tile landed, the scores were read
    if (k0 + KT < kend) issue_tile(k0 + KT, Kn, Vn);

    f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
    {
      const float* krow = &Kc[lq * ROWF];
      auto kfrag = [&](int sg) {
        return *reinterpret_cast<const f32x4*>(krow + dl_pos(lq, (dofs + sg * 16 + g * 4) >> 2) * 4);
      };
      f32x4 a = kfrag(0);  // operands of step sg+1 are read while step sg computes
#pragma unroll
      for (int sg = 0; sg < HALF / 16; sg++) {
        const f32x4 an = sg + 1 < HALF / 16 ? kfrag(sg + 1) : a;
#pragma unroll
        for (int c = 0; c < 4; c++) sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c], qreg[sg][c], sacc, 0, 0, 0);
        a = an;
      }
    }
    *reinterpret_cast<f32x4*>(&Sx[wave][lane * 4]) = sacc;
    dl_barrier<0xC07F>();  // lgkmcnt(0) only: the next tile's loads stay in flight
    {
      const f32x4 other = *reinterpret_cast<const f32x4*>(&Sx[wave ^ 1][lane * 4]);
      const f32x4 lo = half == 0 ? sacc : other, hi = half == 0 ? other : sacc;
#pragma unroll
      for (int r = 0; r < 4; r++) sacc[r] = lo[r] + hi[r];
    }

    float tmax = kNegBig;
    bool valid[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int j = k0 + g * 4 + r;
      bool ok = qvalid && j < kend;
      if (p.window > 0) ok = ok && (qi - j < p.window) && (j - qi < p.window);
      valid[r] = ok;
      const float t = sacc[r] * p.scale;
      sacc[r] = t;
      if (ok) tmax = fmaxf(tmax, t);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp_flush(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float pv = valid[r] ? exp_flush(sacc[r] - m_new) : 0.f;
      sacc[r] = pv;
      psum += pv;
    }
    l_part = l_part * alpha + psum;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float ar = __shfl(alpha, 4 * g + r, 64);
#pragma unroll
      for (int db = 0; db < HALF / 16; db++) oacc[db][r] *= ar;
    }
#pragma unroll
    for (int db = 0; db < HALF / 16; db++) {
      const int f = dofs + db * 16 + lq;
      f32x4 b;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int row = 4 * g + c;
        b[c] = Vc[row * ROWF + dl_pos(row, f >> 2) * 4 + (f & 3)];
      }
#pragma unroll
      for (int c = 0; c < 4; c++) oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(sacc[c], b[c], oacc[db], 0, 0, 0);
    }
  };
  for (int k0 = kbeg; k0 < kend; k0 += 2 * KT) {
    step(k0, K0, V0, K1, V1);
    if (k0 + KT < kend) step(k0 + KT, K1, V1, K0, V0);
  }

  float l_tot = l_part + __shfl_xor(l_part, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  const int OW = p.H * HD;
  if (p.kparts > 1) {
    // unnormalised O of this key run; lane lq < 16 of the first wave of the
    // pair holds query lq's running max and sum
    float* po = p.part + (int64_t)part * p.rows * OW;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int qr = qw0 + 4 * g + r;
      if (qr < L) {
        float* orow = po + (int64_t)(start + qr) * OW + (int64_t)h * HD + dofs;
#pragma unroll
        for (int db = 0; db < HALF / 16; db++) orow[db * 16 + lq] = oacc[db][r];
      }
    }
    if (half == 0 && g == 0 && qvalid) {
      float2* pml = reinterpret_cast<float2*>(p.part + (int64_t)p.kparts * p.rows * OW);
      pml[((int64_t)part * p.rows + start + qi) * p.H + h] = make_float2(m_run, l_tot);
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int qr = qw0 + 4 * g + r;
    const float inv = 1.f / __shfl(l_tot, 4 * g + r, 64);
    if (qr < L) {
      float* orow = p.out + (int64_t)(start + qr) * OW + (int64_t)h * HD + dofs;
#pragma unroll
      for (int db = 0; db < HALF / 16; db++) orow[db * 16 + lq] = oacc[db][r] * inv;
    }
  }
}

// Sums the key runs of a split item: with M the largest run max, O =
// (sum_p e^(m_p - M) O_p) / (sum_p e^(m_p - M) l_p), runs added in order.
// One wave per (row, head), 16 bytes per lane per 256 dimensions.
template <int HD>
__global__ __launch_bounds__(256) void attention_combine_kernel(const float* __restrict__ part, int kparts,
                                                                int64_t rows, int H, float* __restrict__ out) {
  const int64_t id = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // row * H + head
  if (id >= rows * H) return;
  const int lane = threadIdx.x & 63;
  const int64_t OW = (int64_t)H * HD;
  const int64_t row = id / H, h = id % H;
  const float2* ml = reinterpret_cast<const float2*>(part + (int64_t)kparts * rows * OW);
  float M = kNegBig;
  for (int q = 0; q < kparts; q++) M = fmaxf(M, ml[q * rows * H + id].x);
  float Lsum = 0.f;
  f32x4 acc[HD / 256];
#pragma unroll
  for (int c = 0; c < HD / 256; c++) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int q = 0; q < kparts; q++) {
    const float2 v = ml[q * rows * H + id];
    const float w = exp_flush(v.x - M);
    Lsum += w * v.y;
    const float* src = part + (q * rows + row) * OW + h * HD + lane * 4;
#pragma unroll
    for (int c = 0; c < HD / 256; c++) {
      const f32x4 o = *reinterpret_cast<const f32x4*>(src + c * 256);
#pragma unroll
      for (int e = 0; e < 4; e++) acc[c][e] += w * o[e];
    }
  }
  const float inv = 1.f / Lsum;
  float* dst = out + row * OW + h * HD + lane * 4;
#pragma unroll
  for (int c = 0; c < HD / 256; c++) {
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = acc[c][e] * inv;
    *reinterpret_cast<f32x4*>(dst + c * 256) = o;
  }
}

// ---- split-bf16 model-path kernel (head_dim 256) --------------------------------
// attention_planes_kernel computes what attention_varlen_kernel<256> does on
// the bf16 MFMA (v_mfma_f32_16x16x32_bf16, 16x the fp32 MFMA's rate) with
// fp32 accuracy: every fp32 operand x is the exact sum of three bf16 terms
// x0 + x1 + x2 (split3: 8 mantissa bits each), and a product a.b is the sum
// of the six term products ai.bj with i + j <= 2 (the three dropped ones
// are below 2^-24 relative), accumulated in fp32.
//
// Operands. q (fp32, normed and rotated in qkv) is split in registers once
// per work item. Keys and values arrive split, written by
// qkv_planes_kernel: keys [row][kv head][term][256]; values in quads
// of four keys of one sequence (every sequence starts a quad, cu_quads),
// [quad][kv head][dim][16]: per dimension the two 16-byte windows (V0|V1)
// and (V0|V2) of the four keys' terms, in that order for dims with bit 3
// clear and swapped otherwise (the 16 lanes reading one window per
// instruction then cover all LDS banks).
//
// Formulation (lane l: g = l / 16, lq = l % 16). A work item is (sequence,
// block of 64 queries, head), eight waves in four pairs; as in
// attention_varlen_kernel, waves 2b and 2b+1 own queries q0 + 16b .. +15
// and the two 128-dim halves. Per tile of 16 keys:
//   S^T[key, query] = K . Q^T over the wave's 128 dims: A = a key term from
//   LDS (lane: key lq, dims 8g..8g+7 of a 32-dim chunk), B = a q term;
//   4 chunks x 6 term pairs = 24 MFMAs; lane l ends with query lq's scores
//   against keys 4g+r. The pair adds its partial scores through LDS in one
//   fixed order, then the online softmax (lane-local + two shuffles).
//   O^T[dim, query] += V^T . P^T: the 32 k-slots of one MFMA carry two term
//   pairs of the 16 keys (slot 8g+j: key 4g+(j&3) of the first pair for
//   j < 4, of the second for j >= 4), so A is one window read (lane: dim lq
//   of the 16-dim block, quad g) and B the lane's own four probabilities'
//   terms: (V0|V2)x(P2|P0), (V0|V1)x(P1|P1), (V0|V1)x(P0|P0) cover the six
//   pairs in 3 MFMAs per 16 dims. Query lq sits in lane l of the O^T
//   accumulator, so the softmax rescale (skipped while no row maximum of
//   the wave moved) and the final 1/sum are lane-local.
// MFMA time per tile and wave: 48 x 16 cycles, against 64 x 32 for the
// fp32-MFMA kernel.
//
// Loads: buffer loads straight to LDS (a buffer resource per operand; the
// per-lane offsets are fixed per work item and the tile offset is a scalar,
// so no address arithmetic per tile; reads past the buffer return zeros).
// One key buffer (three terms of 16 rows x 512 bytes, 16-byte chunks
// XOR-swizzled by row) and one value buffer (four quads of 8 KB), 65 KB per
// workgroup of eight waves, shared by 64 queries: the tiles' loads to LDS,
// not the MFMAs, bound this kernel at 32 queries per tile. Capped at 128
// VGPRs (a 16-byte spill) for two workgroups per CU, four waves per SIMD:
// C4 14.05 -> 13.19 ms, C3 32.3 -> 30.6 ms per forward against 142 VGPRs. Per tile: barrier (the tile's keys
// landed, every wave is done with the previous values), load the tile's
// values, scores, exchange barrier (every wave is done with the keys, the
// values landed), load the next tile's keys, softmax, P.V.
constexpr int PL_VQ = 4096 + 64;  // uint16 per quad of values in LDS: 8 KB + 128 B
constexpr int PL_W = 8;                 // waves per workgroup: four pairs
constexpr int PL_NT = 64 * PL_W;
constexpr int PL_QBLK = QW * PL_W / 2;  // queries per work item

struct PlanesParams {
  const float* qkv;
  const uint16_t* kp;
  const uint16_t* vp;
  float* out;
  const int32_t* cu;
  const int32_t* cu4;
  const int32_t* items;
  int32_t kp_bytes, vp_bytes;  // buffer extents (loads past them return zeros)
  int32_t H, Hkv;
  int32_t window;
  float scale;
  int64_t row0;  // packed row of qkv's and out's first row (kp and vp are indexed by absolute row and quad)
};

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return *reinterpret_cast<const bf16x8*>(&v); }

// raw buffer of `bytes` bytes (stride 0: offsets are byte offsets, range-checked)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base, int32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

__global__ __launch_bounds__(PL_NT, 4) void attention_planes_kernel(PlanesParams p) {
  constexpr int HD = 256, HALF = 128;
  __shared__ __attribute__((aligned(16))) uint16_t Kb[3 * KT * HD];
  __shared__ __attribute__((aligned(16))) uint16_t Vq[4 * PL_VQ];
  __shared__ __attribute__((aligned(16))) float Sx[PL_NT / 64][64 * 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: LDS load addresses in scalars
  const int qb = wave >> 1, half = wave & 1;
  const int g = lane >> 4;
  const int lq = lane & 15;

  const int seq = p.items[3 * blockIdx.x];
  const int q0 = p.items[3 * blockIdx.x + 1];
  const int h = p.items[3 * blockIdx.x + 2];
  const int hk = h / (p.H / p.Hkv);
  const int start_abs = p.cu[seq];
  const int L = p.cu[seq + 1] - start_abs;
  const int64_t start = start_abs - p.row0;  // the sequence's first row in qkv and out
  const int quad0 = p.cu4[seq];
  const int W = (p.H + 2 * p.Hkv) * HD;
  const int dofs = half * HALF;

  const int qw0 = q0 + qb * QW;
  const int qi = qw0 + lq;
  const bool qvalid = qi < L;
  // q terms: query lq, dims dofs + 32c + 8g .. +7
  bf16x8 qt[3][HALF / 32];
  {
    const float* qr = p.qkv + (int64_t)(start + (qvalid ? qi : 0)) * W + (int64_t)h * HD + dofs + 8 * g;
#pragma unroll
    for (int c = 0; c < HALF / 32; c++) {
      f32x4 x0 = *reinterpret_cast<const f32x4*>(qr + 32 * c);
      f32x4 x1 = *reinterpret_cast<const f32x4*>(qr + 32 * c + 4);
      if (!qvalid) x0 = x1 = f32x4{0.f, 0.f, 0.f, 0.f};
      uint32_t t0[8], t1[8], t2[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const Split3 sp = split3(e < 4 ? x0[e] : x1[e - 4]);
        t0[e] = sp.h;
        t1[e] = sp.m;
        t2[e] = sp.l;
      }
      qt[0][c] = as_bf16x8(u32x4{pack_hi16(t0[0], t0[1]), pack_hi16(t0[2], t0[3]), pack_hi16(t0[4], t0[5]),
                                 pack_hi16(t0[6], t0[7])});
      qt[1][c] = as_bf16x8(u32x4{pack_hi16(t1[0], t1[1]), pack_hi16(t1[2], t1[3]), pack_hi16(t1[4], t1[5]),
                                 pack_hi16(t1[6], t1[7])});
      qt[2][c] = as_bf16x8(u32x4{pack_hi16(t2[0], t2[1]), pack_hi16(t2[2], t2[3]), pack_hi16(t2[4], t2[5]),
                                 pack_hi16(t2[6], t2[7])});
    }
  }
  f32x4 oacc[HALF / 16];  // O^T: dims dofs + 16db + 4g + r of query lq
#pragma unroll
  for (int db = 0; db < HALF / 16; db++) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegBig;
  float l_part = 0.f;

  const int qlast = min(q0 + PL_QBLK, L) - 1;
  int kbeg = 0, kend = L;
  if (p.window > 0) {
    // tiles start on a quad; keys below q0 - window + 1 fail every query's window test
    kbeg = max(0, q0 - p.window + 1) & ~3;
    kend = min(L, qlast + p.window);
  }

  const __amdgpu_buffer_rsrc_t krs = raw_rsrc(p.kp, p.kp_bytes), vrs = raw_rsrc(p.vp, p.vp_bytes);
  // keys: 24 loads of 1 KB per tile (term, pair of rows), three per wave;
  // byte offsets relative to the tile's first key row
  int kvo[24 / PL_W];
#pragma unroll
  for (int j = 0; j < 24 / PL_W; j++) {
    const int i = wave + PL_W * j;
    const int term = i >> 3, rp = i & 7;
    const int r = 2 * rp + (lane >> 5);
    const int chunk = (lane & 31) ^ (r & 15);  // the global chunk that lands at this position
    kvo[j] = ((r * p.Hkv * 3 + term) * HD + chunk * 8) * 2;
  }
  const int krow_bytes = p.Hkv * 3 * HD * 2;
  const int kbase = (start_abs * p.Hkv + hk) * 3 * HD * 2;
  // values: 32 loads of 1 KB per tile (quad, eighth of the quad), four per wave
  int vvo[32 / PL_W];
#pragma unroll
  for (int j = 0; j < 32 / PL_W; j++) {
    const int i = wave + PL_W * j;
    vvo[j] = ((i >> 3) * p.Hkv * 4096 + (i & 7) * 512 + lane * 8) * 2;
  }
  const int vquad_bytes = p.Hkv * 4096 * 2;
  const int vbase = (quad0 * p.Hkv + hk) * 4096 * 2;

  auto issue_k = [&](int k0) {
    const int so = kbase + k0 * krow_bytes;
#pragma unroll
    for (int j = 0; j < 24 / PL_W; j++) {
      const int i = wave + PL_W * j;
      const int term = i >> 3, rp = i & 7;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(krs, (__attribute__((address_space(3))) void*)&Kb[(term * KT + 2 * rp) * HD],
                                               16, kvo[j], so, 0, 0);
    }
  };
  auto issue_v = [&](int k0) {
    const int so = vbase + (k0 >> 2) * vquad_bytes;
#pragma unroll
    for (int j = 0; j < 32 / PL_W; j++) {
      const int i = wave + PL_W * j;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vrs, (__attribute__((address_space(3))) void*)&Vq[(i >> 3) * PL_VQ + (i & 7) * 512],
                                               16, vvo[j], so, 0, 0);
    }
  };
  issue_k(kbeg);

  const int w0 = (lq & 8) ? 8 : 0;  // position of the (V0|V1) window of this lane's dims
  for (int k0 = kbeg; k0 < kend; k0 += KT) {
    // the tile's keys landed (own loads, then everyone's); every wave is done
    // with the previous tile's values
    dl_barrier<0x0070>();
    issue_v(k0);

    f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < HALF / 32; c++) {
      const int pos = ((dofs >> 3) + 4 * c + g) ^ lq;
      const bf16x8 k0v = *reinterpret_cast<const bf16x8*>(&Kb[(0 * KT + lq) * HD + pos * 8]);
      const bf16x8 k1v = *reinterpret_cast<const bf16x8*>(&Kb[(1 * KT + lq) * HD + pos * 8]);
      const bf16x8 k2v = *reinterpret_cast<const bf16x8*>(&Kb[(2 * KT + lq) * HD + pos * 8]);
      // smallest terms first
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k2v, qt[0][c], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1v, qt[1][c], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0v, qt[2][c], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1v, qt[0][c], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0v, qt[1][c], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0v, qt[0][c], sacc, 0, 0, 0);
    }
    *reinterpret_cast<f32x4*>(&Sx[wave][lane * 4]) = sacc;
    // partial scores written, every wave is done with the keys, the values landed
    dl_barrier<0x0070>();
    // the next tile's keys (past the last tile: a redundant load, so that no
    // load is conditional)
    issue_k(k0 + KT);
    {
      const f32x4 other = *reinterpret_cast<const f32x4*>(&Sx[wave ^ 1][lane * 4]);
      const f32x4 lo = half == 0 ? sacc : other, hi = half == 0 ? other : sacc;
#pragma unroll
      for (int r = 0; r < 4; r++) sacc[r] = lo[r] + hi[r];
    }

    float tmax = kNegBig;
    bool valid[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int j = k0 + g * 4 + r;
      bool ok = qvalid && j < kend;
      if (p.window > 0) ok = ok && (qi - j < p.window) && (j - qi < p.window);
      valid[r] = ok;
      const float t = sacc[r] * p.scale;
      sacc[r] = t;
      if (ok) tmax = fmaxf(tmax, t);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const bool moved = m_new != m_run;
    const float alpha = exp_flush(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
    uint32_t p0[4], p1[4], p2[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float pv = valid[r] ? exp_flush(sacc[r] - m_new) : 0.f;
      psum += pv;
      const Split3 sp = split3(pv);
      p0[r] = sp.h;
      p1[r] = sp.m;
      p2[r] = sp.l;
    }
    l_part = l_part * alpha + psum;
    if (__any(moved)) {
#pragma unroll
      for (int db = 0; db < HALF / 16; db++) oacc[db] *= alpha;
    }
    const uint32_t a0 = pack_hi16(p0[0], p0[1]), b0 = pack_hi16(p0[2], p0[3]);
    const uint32_t a1 = pack_hi16(p1[0], p1[1]), b1 = pack_hi16(p1[2], p1[3]);
    const uint32_t a2 = pack_hi16(p2[0], p2[1]), b2 = pack_hi16(p2[2], p2[3]);
    const bf16x8 B1 = as_bf16x8(u32x4{a0, b0, a0, b0});  // P0 | P0
    const bf16x8 B2 = as_bf16x8(u32x4{a1, b1, a1, b1});  // P1 | P1
    const bf16x8 B3 = as_bf16x8(u32x4{a2, b2, a0, b0});  // P2 | P0
#pragma unroll
    for (int db = 0; db < HALF / 16; db++) {
      const uint16_t* vr = &Vq[g * PL_VQ + (dofs + db * 16 + lq) * 16];
      const bf16x8 A01 = *reinterpret_cast<const bf16x8*>(vr + w0);      // V0 | V1
      const bf16x8 A02 = *reinterpret_cast<const bf16x8*>(vr + 8 - w0);  // V0 | V2
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A02, B3, oacc[db], 0, 0, 0);
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A01, B2, oacc[db], 0, 0, 0);
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A01, B1, oacc[db], 0, 0, 0);
    }
  }

  __builtin_amdgcn_s_waitcnt(0x0070);  // no load to LDS outstanding at exit
  float l_tot = l_part + __shfl_xor(l_part, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (qvalid) {
    const float inv = 1.f / l_tot;
    float* orow = p.out + (int64_t)(start + qi) * (p.H * HD) + (int64_t)h * HD + dofs + 4 * g;
#pragma unroll
    for (int db = 0; db < HALF / 16; db++) *reinterpret_cast<f32x4*>(orow + db * 16) = oacc[db] * inv;
  }
}


// ---- generic attention (per-op drop-in) ------------------------------------------
constexpr int GMAXD = 512;

__global__ __launch_bounds__(256) void attention_generic_kernel(AttnGenericArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t rowid = (int64_t)blockIdx.x * 4 + wave;
  const int64_t nrows = (int64_t)a.B * a.H * a.T;
  if (rowid >= nrows) return;
  const int i = (int)(rowid % a.T);
  const int hh = (int)((rowid / a.T) % a.H);
  const int b = (int)(rowid / ((int64_t)a.T * a.H));
  const int D = a.D, S = a.S;
  const float* q = a.q + b * a.q_sb + hh * a.q_sh + (int64_t)i * D;
  const float* k = a.k + b * a.k_sb + hh * a.k_sh;
  const float* v = a.v + b * a.v_sb + hh * a.v_sh;
  const float* mrow = a.mask ? a.mask + b * a.m_sb + hh * a.m_sh + (int64_t)i * a.m_sr : nullptr;
  // reference algebra (internal/blas/attention.go:105-122)
  float sa = a.scale, invScale = 1.f;
  const bool pos = a.scale > 0.f;
  if (pos) invScale = 1.f / a.scale; else sa = 1.f;
  float m_run = -INFINITY, l_run = 0.f;
  float o[GMAXD / 64];
#pragma unroll
  for (int c = 0; c < GMAXD / 64; c++) o[c] = 0.f;
  for (int j0 = 0; j0 < S; j0 += 64) {
    const int j = j0 + lane;
    const bool ok = j < S;
    float row = -INFINITY;
    if (ok) {
      const float* kj = k + (int64_t)j * D;
      float s = 0.f;
      for (int d = 0; d < D; d++) s = fmaf(q[d], kj[d], s);
      row = s;
      if (!pos) row = __fmul_rn(row, a.scale);
      if (mrow) row = __fadd_rn(__fmul_rn(invScale, mrow[(int64_t)j * a.m_sc]), row);
    }
    const float bmax = wave_max(row);
    const float m_new = fmaxf(m_run, bmax);
    const float alpha = (m_run == -INFINITY) ? 0.f : exp_flush(sa * m_run - sa * m_new);
    const float pj = ok ? exp_flush(__fadd_rn(__fmul_rn(sa, row), -sa * m_new)) : 0.f;
    l_run = l_run * alpha + wave_sum(pj);
    m_run = m_new;
#pragma unroll
    for (int c = 0; c < GMAXD / 64; c++) o[c] *= alpha;
    const int nj = min(64, S - j0);
    for (int jj = 0; jj < nj; jj++) {
      const float pw = __shfl(pj, jj, 64);
      if (pw == 0.f) continue;  // uniform across the wave
      const float* vj = v + (int64_t)(j0 + jj) * D;
#pragma unroll
      for (int c = 0; c < GMAXD / 64; c++) {
        const int d = lane + 64 * c;
        if (d < D) o[c] = fmaf(pw, vj[d], o[c]);
      }
    }
  }
  const float inv = 1.f / l_run;
  float* out = a.out + rowid * D;
#pragma unroll
  for (int c = 0; c < GMAXD / 64; c++) {
    const int d = lane + 64 * c;
    if (d < D) out[d] = o[c] * inv;
  }
}

}  // namespace

int launch_attention_varlen_items(fa_ctx* ctx, const AttnVarlenArgs& a, const int32_t* d_items, int32_t n_items,
                                  hipStream_t s) {
  if (a.D != 256 && a.D != 512)
    return set_error(ctx, FA_ERR_UNSUPPORTED, "attention: head_dim %d not 256 or 512", a.D);
  if (a.Hkv <= 0 || a.H % a.Hkv != 0)
    return set_error(ctx, FA_ERR_ARG, "attention: %d query heads not a multiple of %d kv heads", a.H, a.Hkv);
  if (n_items == 0) return FA_OK;
  if (a.kparts < 1 || a.kparts > kMaxKeyParts || (a.kparts > 1 && (!a.part || a.rows <= 0)))
    return set_error(ctx, FA_ERR_ARG, "attention: %d key parts (1..%d, > 1 needs a partial buffer)", a.kparts,
                     kMaxKeyParts);
  VarlenParams p;
  p.qkv = a.qkv; p.out = a.out; p.cu = a.cu_seqlens; p.items = d_items; p.row0 = a.row0;
  p.H = a.H; p.Hkv = a.Hkv; p.window = a.window; p.scale = a.scale;
  p.kparts = a.kparts; p.rows = a.rows; p.part = a.part;
  const dim3 grid((unsigned)((int64_t)n_items * a.kparts));
  if (a.D == 256)
    hipLaunchKernelGGL(attention_varlen_kernel<256>, grid, dim3(DL_NT), 0, s, p);
  else
    hipLaunchKernelGGL(attention_varlen_kernel<512>, grid, dim3(DL_NT), 0, s, p);
  if (a.kparts > 1) {
    const dim3 g2((unsigned)((a.rows * a.H + 3) / 4));
    if (a.D == 256)
      hipLaunchKernelGGL(attention_combine_kernel<256>, g2, dim3(256), 0, s, a.part, a.kparts, a.rows, a.H, a.out);
    else
      hipLaunchKernelGGL(attention_combine_kernel<512>, g2, dim3(256), 0, s, a.part, a.kparts, a.rows, a.H, a.out);
  }
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_attention_planes(fa_ctx* ctx, const AttnPlanesArgs& a, const int32_t* d_items, int32_t n_items,
                            hipStream_t s) {
  if (a.Hkv <= 0 || a.H % a.Hkv != 0)
    return set_error(ctx, FA_ERR_ARG, "attention: %d query heads not a multiple of %d kv heads", a.H, a.Hkv);
  if (n_items == 0) return FA_OK;
  if (a.kp_bytes <= 0 || a.vp_bytes <= 0 || a.kp_bytes > INT32_MAX - (1 << 22) || a.vp_bytes > INT32_MAX - (1 << 22))
    return set_error(ctx, FA_ERR_ARG, "attention: key/value planes of %lld / %lld bytes outside 1..2^31 - 4 MB",
                     (long long)a.kp_bytes, (long long)a.vp_bytes);
  PlanesParams p;
  p.qkv = a.qkv; p.kp = a.kp; p.vp = a.vp; p.out = a.out; p.cu = a.cu_seqlens; p.cu4 = a.cu_quads;
  p.kp_bytes = (int32_t)a.kp_bytes; p.vp_bytes = (int32_t)a.vp_bytes;
  p.items = d_items; p.H = a.H; p.Hkv = a.Hkv; p.window = a.window; p.scale = a.scale; p.row0 = a.row0;
  hipLaunchKernelGGL(attention_planes_kernel, dim3((unsigned)n_items), dim3(PL_NT), 0, s, p);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}


int attention_varlen_qblock() { return QBLK; }
int attention_planes_qblock() { return PL_QBLK; }

int launch_attention_generic(fa_ctx* ctx, const AttnGenericArgs& a, hipStream_t s) {
  if (a.D > GMAXD) return set_error(ctx, FA_ERR_UNSUPPORTED, "Attention: head dimension %d > %d", a.D, GMAXD);
  const int64_t rows = (int64_t)a.B * a.H * a.T;
  if (rows == 0) return FA_OK;
  hipLaunchKernelGGL(attention_generic_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, a);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

}  // namespace fa
