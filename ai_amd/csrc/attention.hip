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
  const int32_t* items;  // triples (seq, q0, head)
  const int32_t* ext;    // per item (sequence's first packed row, length, first tile, 0)
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
// Max and sum over lanes l, l^16, l^32 and l^48 (the four row groups of a
// 16x16 MFMA column) with v_permlane16_swap / v_permlane32_swap: a swap of
// a value with itself leaves the lane's own value in one result and its
// partner's in the other, so no LDS round trip (ds_bpermute) is needed and
// the reduction does not wait behind outstanding LDS reads.
__device__ __forceinline__ float rows4_max(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
// x_l + x_{l^16}, then the same over l^32 (each sum commutes exactly)
__device__ __forceinline__ float rows4_sum(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

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
  const int q0 = p.items[3 * item + 1];
  const int h = p.items[3 * item + 2];
  const int hk = h / (p.H / p.Hkv);
  const int4 e = reinterpret_cast<const int4*>(p.ext)[item];
  const int32_t seq_row = e.x, L = e.y;  // the sequence's first packed row and length
  const int64_t start = seq_row - p.row0;  // the sequence's first row in qkv and out
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
    tmax = rows4_max(tmax);
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

  const float l_tot = rows4_sum(l_part);
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
                                                                int64_t rows, int64_t row_off, int64_t n, int H,
                                                                float* __restrict__ out) {
  // rows: the partial buffers' row count; this launch sums rows row_off ..
  // row_off + n - 1 of them into out's rows 0 .. n - 1
  const int64_t lid = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);  // local row * H + head
  if (lid >= n * H) return;
  const int lane = threadIdx.x & 63;
  const int64_t OW = (int64_t)H * HD;
  const int64_t lrow = lid / H, h = lid % H;
  const int64_t row = row_off + lrow, id = row * H + h;
  const float2* ml = reinterpret_cast<const float2*>(part + (int64_t)kparts * rows * OW);
  // every run's (max, sum) and partial O loaded before the first use (one
  // round trip instead of one per run; kparts <= kMaxKeyParts, checked by
  // the launchers), then combined in run order
  float2 mlv[kMaxKeyParts];
  f32x4 ov[kMaxKeyParts][HD / 256];
#pragma unroll
  for (int q = 0; q < kMaxKeyParts; q++) {
    if (q < kparts) {
      mlv[q] = ml[q * rows * H + id];
      const float* src = part + (q * rows + row) * OW + h * HD + lane * 4;
#pragma unroll
      for (int c = 0; c < HD / 256; c++) ov[q][c] = *reinterpret_cast<const f32x4*>(src + c * 256);
    }
  }
  float M = kNegBig;
#pragma unroll
  for (int q = 0; q < kMaxKeyParts; q++)
    if (q < kparts) M = fmaxf(M, mlv[q].x);
  float Lsum = 0.f;
  f32x4 acc[HD / 256];
#pragma unroll
  for (int c = 0; c < HD / 256; c++) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int q = 0; q < kMaxKeyParts; q++) {
    if (q < kparts) {
      const float w = exp_flush(mlv[q].x - M);
      Lsum += w * mlv[q].y;
#pragma unroll
      for (int c = 0; c < HD / 256; c++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[c][e] += w * ov[q][c][e];
    }
  }
  const float inv = 1.f / Lsum;
  float* dst = out + lrow * OW + h * HD + lane * 4;
#pragma unroll
  for (int c = 0; c < HD / 256; c++) {
    f32x4 o;
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = acc[c][e] * inv;
    *reinterpret_cast<f32x4*>(dst + c * 256) = o;
  }
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return *reinterpret_cast<const bf16x8*>(&v); }

// ---- split-bf16 model-path kernel over key/value tile images (head_dim 256) -----
// attention_tiles_kernel computes attention_varlen_kernel<256>'s result on
// the bf16 MFMA (v_mfma_f32_16x16x32_bf16) with fp32 accuracy: every fp32
// operand is the exact sum of three bf16 terms (split3) and a product a.b
// the sum of the six term products ai.bj with i + j <= 2 (the three dropped
// ones are below 2^-24 relative), accumulated in fp32.
//
// Rows. The query rows of kv head hk are the pairs (token t, query head
// hk*G + g) of the G = H/Hkv heads that share it, numbered r = t*G + g. A
// work item is (sequence, 128 or 64 consecutive rows, hk[, run of key
// tiles]); its waves own 16 rows each (eight waves for 128 rows; for 64
// rows eight waves in pairs that split the head dimension, or four), so
// one key/value tile in LDS serves every query head of the group (and a
// short sequence fills an item's rows G times sooner than with one head
// per item).
//
// Operands. Keys and values arrive as LDS images written once per layer by
// kv_tiles_kernel: per (tile of 32 keys of one sequence, kv head) a key
// image [term][key][256] whose 16-byte chunk c of key k sits at c ^ k, and
// a value image [term][dim][32 slots] whose slot 8g + 4h + r holds key 16h +
// 4g + r (chunk g of dim d at position g ^ ((d >> 1) & 3)); 48 KB each,
// copied to LDS unchanged by direct global->LDS loads (1 KB per wave
// instruction). One key buffer and two value buffers: 144 KB (160 KB with
// the wave pairs' partial-score exchange), one workgroup per CU (two waves
// per SIMD with eight waves, one with four).
//
// Formulation (lane l: lq = l % 16, g = l / 16). The q terms stay in
// registers: lane l holds row lq's dims 32c + 8g .. +7 (c = 0..7), three
// terms, 96 VGPRs.
//   S^T[key, row] = K . Q^T per block of 16 keys: A = a key term (lane l:
//   key lq, dims 32c + 8g ..), B = a q term; 8 chunks x 6 term pairs per
//   block. Lane l ends with row lq's scores against keys 4g + r and 16 + 4g
//   + r: the row's softmax is lane-local plus two exchanges (xor 16, 32).
//   O^T[dim, row] += V^T . P^T, one 32-key step per block of 16 dims x 6
//   pairs: the lane's own eight probabilities are B (slot 8g + e: key 4g + e
//   for e < 4, 16 + 4g + e - 4 after), A one 16-byte value-image read per
//   term (dim 16db + lq, slots 8g ..). Row lq's O sits in the lanes with
//   that lq (dims 16db + 4g + r), so the rescale and the final 1/sum are
//   lane-local.
// Lazy maximum: a row's exponent offset m moves only when a tile's maximum
// exceeds it by more than 8 (O and the sum are then scaled by e^(m_old -
// m_new)), so weights stay below e^8 and O is rarely touched outside the
// MFMAs. A weight is 0 when its exponent t - m is below -87 (the reference
// flushes against the row's final maximum; the two differ only in weights
// below e^-87 of the row's largest).
//
// Per tile tt (software pipeline, detailed at the loop): barrier (keys of
// tt and values of tt-1 landed; every wave done with iteration tt-1), load
// the values of tt, scores of tt, barrier (every wave done reading the
// keys), load the keys of tt+1 (past the last tile: the last again, so no
// load is conditional), then P.V of tile tt-1 with tile tt's softmax spread
// among its blocks.
constexpr int TL_KEYS = 32;              // keys per tile
constexpr int TL_IMG = 3 * 32 * 256;     // bf16 per key or value image
constexpr float TL_TAU = 8.f;            // lazy-maximum slack

struct TilesParams {
  const float* qkv;
  const uint16_t* img;   // [tile][Hkv][key image | value image]
  float* out;
  const int32_t* items;  // triples (sequence, first row, kv head)
  const int32_t* ext;    // per item (sequence's first packed row, length, first tile, 0)
  int32_t H, Hkv;
  int32_t window;
  float scale;
  int64_t row0;  // packed row of qkv's and out's first row
  // kparts > 1: each item's tiles are cut into kparts runs, one workgroup
  // each, written unnormalised with (max, sum) per row and head to part
  // [kparts][rows][H * 256] (rows: packed rows of the whole batch, indexed
  // by absolute row) for attention_combine_kernel
  int32_t kparts;
  int64_t rows;
  float* part;
  // q's RMSNorm gain (1 + g) and RoPE tables [positions][128], applied as q is loaded
  const float* gq;
  const float *cs, *sn;
  float eps;
};

__device__ __forceinline__ void split_pack8(const f32x4& x0, const f32x4& x1, bf16x8& t0, bf16x8& t1, bf16x8& t2) {
  uint32_t h[8], m[8], l[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const Split3 sp = split3(e < 4 ? x0[e] : x1[e - 4]);
    h[e] = sp.h;
    m[e] = sp.m;
    l[e] = sp.l;
  }
  t0 = as_bf16x8(u32x4{pack_hi16(h[0], h[1]), pack_hi16(h[2], h[3]), pack_hi16(h[4], h[5]), pack_hi16(h[6], h[7])});
  t1 = as_bf16x8(u32x4{pack_hi16(m[0], m[1]), pack_hi16(m[2], m[3]), pack_hi16(m[4], m[5]), pack_hi16(m[6], m[7])});
  t2 = as_bf16x8(u32x4{pack_hi16(l[0], l[1]), pack_hi16(l[2], l[3]), pack_hi16(l[4], l[5]), pack_hi16(l[6], l[7])});
}

// TL_W waves of 16 rows: 8 (128-row items, two waves per SIMD) or 4
// (64-row items, one wave per SIMD: twice the items, each half as long,
// for batches whose 128-row items fill between half a round and a round of
// the CUs; the compiler then keeps what does not fit in 256 VGPRs in AGPRs
// instead of scratch).
// DS = 2 (with TL_W = 8): 64-row items whose head dimension is split over
// a pair of waves, waves w and w + 4 owning the same 16 rows and dims
// [0, 128) and [128, 256) of q (for the scores) and of O (for P.V). Each
// wave's partial scores over its 128 dims go to LDS before the barrier
// that follows the score step, and both waves of the pair add them as
// own + partner's (the same fp32 sum in both: addition commutes exactly),
// so they compute identical probabilities. Per wave: half the MFMAs,
// q terms and O of a four-wave item, at two waves per SIMD.
template <int TL_W, int DS>
__global__ __launch_bounds__(64 * TL_W, TL_W == 8 ? 2 : 1) void attention_tiles_kernel(TilesParams p) {
  static_assert(DS == 1 || (DS == 2 && TL_W == 8), "dim split: eight waves in pairs");
  constexpr int RB = TL_W / DS;       // row blocks of 16 per item
  constexpr int TL_ROWS = 16 * RB;    // query rows per work item
  constexpr int HD = 256;
  constexpr int NC = HD / 32 / DS;    // q chunks of 32 dims per wave
  constexpr int NDB = HD / 16 / DS;   // blocks of 16 O dims per wave
  // operand reads one step ahead of the MFMAs that use them (12 more
  // VGPRs): the wave pairs' kernel has the registers to spare
  constexpr bool TL_PF = DS == 2;
  constexpr int TERM = TL_IMG / 3;  // bf16 per term of an image
  __shared__ __attribute__((aligned(16))) uint16_t Ks[TL_IMG];
  __shared__ __attribute__((aligned(16))) uint16_t Vs0[TL_IMG];
  __shared__ __attribute__((aligned(16))) uint16_t Vs1[TL_IMG];
  // partial scores of each wave (two 16-key blocks x 64 lanes), DS = 2
  __shared__ f32x4 Xs[DS == 2 ? TL_W * 2 * 64 : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the wave's row block and dim half (single waves: the whole head)
  const int rbw = wave % RB, hf = DS == 2 ? wave / RB : 0;
  const int lq = lane & 15, g = lane >> 4;

  const int item = blockIdx.x / p.kparts, part = blockIdx.x % p.kparts;
  const int rb = p.items[3 * item + 1];
  const int hk = p.items[3 * item + 2];
  const int G = p.H / p.Hkv;
  const int4 e = reinterpret_cast<const int4*>(p.ext)[item];
  const int32_t seq_row = e.x, L = e.y, seq_tile = e.z;  // the sequence's first packed row, length and first key tile
  const int64_t start = seq_row - p.row0;  // the sequence's first row in qkv and out
  const int W = (p.H + 2 * p.Hkv) * HD;
  const int nrows = G * L;
  const int row = rb + 16 * rbw + lq;
  const bool qvalid = row < nrows;
  const int tok = (qvalid ? row : rb) / G;
  const int head = hk * G + (qvalid ? row : rb) % G;

  // the item's key tiles: the union of its rows' windows
  const int tok_lo = rb / G, tok_hi = (min(rb + TL_ROWS, nrows) - 1) / G;
  int kbeg = 0, kend = L;
  if (p.window > 0) {
    kbeg = max(0, tok_lo - p.window + 1);
    kend = min(L, tok_hi + p.window);
  }
  int tb = kbeg / TL_KEYS, te = (kend + TL_KEYS - 1) / TL_KEYS;
  if (p.kparts > 1) {  // this part's run of tiles (possibly none)
    const int per = (te - tb + p.kparts - 1) / p.kparts;
    const int nb = tb + part * per;
    te = min(te, nb + per);
    tb = nb;
  }

  const uint16_t* img0 = p.img + ((int64_t)seq_tile * p.Hkv + hk) * (2 * TL_IMG);
  const int64_t tstride = (int64_t)p.Hkv * 2 * TL_IMG;
  // 48 loads of 1 KB per image, six per wave
  auto issue = [&](const uint16_t* src, uint16_t* dst) {
#pragma unroll
    for (int j = 0; j < 48 / TL_W; j++) {
      const int c = wave + TL_W * j;
      __builtin_amdgcn_global_load_lds(src + c * 512 + lane * 8, (__attribute__((address_space(3))) void*)&dst[c * 512],
                                       16, 0, 0);
    }
  };

  // The first tile's key image: issued whole by the second wave of each
  // SIMD (waves TL_W/2 ..) before anything else. Those waves get their q
  // rows after the first waves' anyway (the CU's memory pipeline serves
  // the first waves' loads first), so the image lands while the first
  // waves prepare q, and no wave's q wait covers it but theirs. A run
  // without tiles loads the last tile of the range and waits for it
  // before the exit.
  const bool k_first = wave >= TL_W / 2;
  if (k_first) {
    const uint16_t* src = img0 + min(tb, te - 1) * tstride;
#pragma unroll
    for (int j = 0; j < 96 / TL_W; j++) {
      const int c = (wave - TL_W / 2) + (TL_W / 2) * j;
      __builtin_amdgcn_global_load_lds(src + c * 512 + lane * 8, (__attribute__((address_space(3))) void*)&Ks[c * 512],
                                       16, 0, 0);
    }
  }

  if (rb + 16 * rbw >= nrows) {
    // every row of this wave lies past the sequence's rows (the last item
    // of a sequence): the wave issues its share of each image load and
    // takes part in every barrier of the loop below, in the same order,
    // and computes nothing
    if constexpr (DS == 2) dl_barrier<0xC07F>();  // the pairs' q row exchange below
    if (tb < te) {
      for (int tt = tb; tt < te; tt++) {
        dl_barrier<0x0F70>();
        issue(img0 + tt * tstride + TL_IMG, ((tt - tb) & 1) ? Vs1 : Vs0);
        dl_barrier<0xC07F>();
        issue(img0 + min(tt + 1, te - 1) * tstride, Ks);
      }
      dl_barrier<0x0F70>();
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): a first image issued above
    return;
  }

  bf16x8 qt[3][NC];
  if constexpr (DS == 2) {
    // Wave pairs: each wave norms (RMSNorm, gain) and rotates (RoPE at the
    // token's position) 8 of the pair's 16 rows, all 256 dims: lane l takes
    // row 8 hf + l / 8 and dims 16 (l mod 8) .. + 15 and the same + 128
    // (RoPE's pairs in the lane; the row's sum of squares over its eight
    // lanes), and stores them in LDS (the value buffers, free until the
    // first tile's value loads; 16 KB per pair, 16-byte chunk k of row r at
    // position k ^ (r mod 16)); after the barrier each wave reads its dim
    // half of all 16 rows. Each wave norms and rotates 8 rows, not 16.
    const int rho = 8 * hf + (lane >> 3), s8 = lane & 7;
    const int row2 = rb + 16 * rbw + rho;
    const bool valid2 = row2 < nrows;
    const int tok2 = (valid2 ? row2 : rb) / G;
    const int head2 = hk * G + (valid2 ? row2 : rb) % G;
    const float* qr = p.qkv + (start + tok2) * W + (int64_t)head2 * HD + 16 * s8;
    f32x4 lo[4], hi[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      lo[j] = *reinterpret_cast<const f32x4*>(qr + 4 * j);
      hi[j] = *reinterpret_cast<const f32x4*>(qr + HD / 2 + 4 * j);
    }
    const float* gr = p.gq + 16 * s8;
    const float* cr = p.cs + (int64_t)tok2 * (HD / 2) + 16 * s8;
    const float* sr = p.sn + (int64_t)tok2 * (HD / 2) + 16 * s8;
    f32x4 ga[4], gb[4], co[4], si[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      ga[j] = *reinterpret_cast<const f32x4*>(gr + 4 * j);
      gb[j] = *reinterpret_cast<const f32x4*>(gr + HD / 2 + 4 * j);
      co[j] = *reinterpret_cast<const f32x4*>(cr + 4 * j);
      si[j] = *reinterpret_cast<const f32x4*>(sr + 4 * j);
    }
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) ss = fmaf(lo[j][e], lo[j][e], ss);
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int e = 0; e < 4; e++) ss = fmaf(hi[j][e], hi[j][e], ss);
    // the row's eight lanes: xor 1 and 2 within the quad, then the other
    // quad through the half-row mirror (each sum commutes exactly, so every
    // lane of the row gets the same bits)
    ss = ss + dpp_f32<0xB1>(ss);   // quad_perm [1, 0, 3, 2]
    ss = ss + dpp_f32<0x4E>(ss);   // quad_perm [2, 3, 0, 1]
    ss = ss + dpp_f32<0x141>(ss);  // row_half_mirror
    const float inv = rms_inv(ss, HD, p.eps);
    f32x4* qs = reinterpret_cast<f32x4*>((rbw < 3 ? Vs0 : Vs1) + (rbw % 3) * 8192);  // the pair's 16 rows
#pragma unroll
    for (int j = 0; j < 4; j++) {
      f32x4 yl, yh;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float a = lo[j][e] * inv * ga[j][e], b = hi[j][e] * inv * gb[j][e];
        yl[e] = a * co[j][e] - b * si[j][e];  // y_i = x_i c - x_{i+h} s
        yh[e] = a * si[j][e] + b * co[j][e];  // y_{i+h} = x_i s + x_{i+h} c
      }
      const int k = 4 * s8 + j;  // the 16-byte chunk of dims 16 s8 + 4 j
      qs[rho * 64 + (k ^ (rho & 15))] = yl;
      qs[rho * 64 + ((k + 32) ^ (rho & 15))] = yh;
    }
    dl_barrier<0xC07F>();  // lgkmcnt(0): the pair's rows written; the first key image stays in flight
#pragma unroll
    for (int c = 0; c < NC; c++) {
      // the wave's dim half (chunks NC * hf ..): dims 32 (NC hf + c) + 8 g ..
      const int k = 8 * (NC * hf + c) + 2 * g;
      f32x4 x0 = qs[lq * 64 + (k ^ lq)], x1 = qs[lq * 64 + ((k + 1) ^ lq)];
      if (!qvalid) x0 = x1 = f32x4{0.f, 0.f, 0.f, 0.f};
      split_pack8(x0, x1, qt[0][c], qt[1][c], qt[2][c]);
    }
  } else {
    // q normed (RMSNorm, gain) and rotated (RoPE at the token's position)
    // as it is loaded: the row's dims are spread over the four lanes with
    // this lq (sum of squares: two exchanges), and dims i and i + 128 sit in
    // the same lane (chunks c and c + 4)
    const float* qr = p.qkv + (start + tok) * W + (int64_t)head * HD + 8 * g;
    f32x4 x[HD / 32][2];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < HD / 32; c++) {
      x[c][0] = *reinterpret_cast<const f32x4*>(qr + 32 * c);
      x[c][1] = *reinterpret_cast<const f32x4*>(qr + 32 * c + 4);
    }
#pragma unroll
    for (int c = 0; c < HD / 32; c++)
#pragma unroll
      for (int e = 0; e < 8; e++) ss = fmaf(x[c][e >> 2][e & 3], x[c][e >> 2][e & 3], ss);
    ss = rows4_sum(ss);
    const float inv = rms_inv(ss, HD, p.eps);
    const float* gr = p.gq + 8 * g;
    const float* cr = p.cs + (int64_t)tok * (HD / 2) + 8 * g;
    const float* sr = p.sn + (int64_t)tok * (HD / 2) + 8 * g;
#pragma unroll
    for (int c = 0; c < HD / 64; c++) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const f32x4 ga = *reinterpret_cast<const f32x4*>(gr + 32 * c + 4 * h);
        const f32x4 gb = *reinterpret_cast<const f32x4*>(gr + 32 * (c + HD / 64) + 4 * h);
        const f32x4 co = *reinterpret_cast<const f32x4*>(cr + 32 * c + 4 * h);
        const f32x4 si = *reinterpret_cast<const f32x4*>(sr + 32 * c + 4 * h);
        f32x4& lo = x[c][h];
        f32x4& hi = x[c + HD / 64][h];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float a = lo[e] * inv * ga[e], b = hi[e] * inv * gb[e];
          lo[e] = a * co[e] - b * si[e];  // y_i = x_i c - x_{i+h} s
          hi[e] = a * si[e] + b * co[e];  // y_{i+h} = x_i s + x_{i+h} c
        }
      }
    }
#pragma unroll
    for (int c = 0; c < NC; c++) {
      f32x4 x0 = x[c][0], x1 = x[c][1];
      if (!qvalid) x0 = x1 = f32x4{0.f, 0.f, 0.f, 0.f};
      split_pack8(x0, x1, qt[0][c], qt[1][c], qt[2][c]);
    }
  }

  f32x4 oacc[NDB];  // O^T: dims 16(NDB hf + db) + 4g + r of row lq
#pragma unroll
  for (int db = 0; db < NDB; db++) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegBig;
  float l_part = 0.f;
  const int vsw = (lq >> 1) & 3;
  // the row's valid keys: klo <= j < khi (none for a row past the item)
  int klo = 0, khi = qvalid ? L : 0;
  if (p.window > 0 && qvalid) {
    klo = max(0, tok - p.window + 1);
    khi = min(L, tok + p.window);
  }

  // The six term products of one 16-key block and one 32-dim chunk, in a
  // fixed order (smallest terms first), accumulated into s.
  auto qk_chunk = [&](f32x4& s, const bf16x8& k0, const bf16x8& k1, const bf16x8& k2, int c) {
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k2, qt[0][c], s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qt[2][c], s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qt[1][c], s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qt[0][c], s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qt[1][c], s, 0, 0, 0);
    s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qt[0][c], s, 0, 0, 0);
  };
  auto qk = [&](const uint16_t* Kc, f32x4 (&sacc)[2]) {
    if constexpr (TL_PF) {
      // The two key blocks' chains interleaved (each MFMA's accumulator was
      // written two MFMAs earlier, not one), and the key terms of chunk c + 1
      // read while chunk c's products run. Each block's products keep the
      // order above, so the scores are the same bits.
      sacc[0] = f32x4{0.f, 0.f, 0.f, 0.f};
      sacc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
      bf16x8 kt[2][2][3];  // [chunk parity][key block][term]
      auto rd = [&](int c, bf16x8 (&dst)[2][3]) {
#pragma unroll
        for (int kb = 0; kb < 2; kb++) {
          const int key = 16 * kb + lq;
          const uint16_t* kr = Kc + key * HD + ((4 * (NC * hf + c) + g) ^ key) * 8;
#pragma unroll
          for (int t = 0; t < 3; t++) dst[kb][t] = *reinterpret_cast<const bf16x8*>(kr + t * TERM);
        }
      };
      rd(0, kt[0]);
#pragma unroll
      for (int c = 0; c < NC; c++) {
        if (c + 1 < NC) rd(c + 1, kt[(c + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);  // the next chunk's reads issue before this chunk's products
        const int b = c & 1;
        sacc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[b][0][2], qt[0][c], sacc[0], 0, 0, 0);
        sacc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[b][1][2], qt[0][c], sacc[1], 0, 0, 0);
        sacc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[b][0][0], qt[2][c], sacc[0], 0, 0, 0);
        sacc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[b][1][0], qt[2][c], sacc[1], 0, 0, 0);
        sacc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[b][0][1], qt[1][c], sacc[0], 0, 0, 0);
        sacc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[b][1][1], qt[1][c], sacc[1], 0, 0, 0);
        sacc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[b][0][1], qt[0][c], sacc[0], 0, 0, 0);
        sacc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[b][1][1], qt[0][c], sacc[1], 0, 0, 0);
        sacc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[b][0][0], qt[1][c], sacc[0], 0, 0, 0);
        sacc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[b][1][0], qt[1][c], sacc[1], 0, 0, 0);
        sacc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[b][0][0], qt[0][c], sacc[0], 0, 0, 0);
        sacc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt[b][1][0], qt[0][c], sacc[1], 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < 2; kb++) {
        sacc[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int key = 16 * kb + lq;
        const uint16_t* kr = Kc + key * HD;
#pragma unroll
        for (int c = 0; c < NC; c++) {
          const int pos = ((4 * (NC * hf + c) + g) ^ key) * 8;
          const bf16x8 k0 = *reinterpret_cast<const bf16x8*>(kr + pos);
          const bf16x8 k1 = *reinterpret_cast<const bf16x8*>(kr + TERM + pos);
          const bf16x8 k2 = *reinterpret_cast<const bf16x8*>(kr + 2 * TERM + pos);
          qk_chunk(sacc[kb], k0, k1, k2, c);
        }
      }
    }
  };
  // O^T += V^T . P^T for one tile (terms b0, b1, b2 of the probabilities)
  // the value terms of block db (with TL_PF read one block ahead)
  auto vread = [&](const uint16_t* Vc, int db, bf16x8 (&dst)[3]) {
    const uint16_t* vr = Vc + (16 * (NDB * hf + db) + lq) * 32 + (g ^ vsw) * 8;
#pragma unroll
    for (int t = 0; t < 3; t++) dst[t] = *reinterpret_cast<const bf16x8*>(vr + t * TERM);
  };
  auto pv = [&](const uint16_t* Vc, const bf16x8& b0, const bf16x8& b1, const bf16x8& b2) {
    bf16x8 vt[2][3];
    if constexpr (TL_PF) vread(Vc, 0, vt[0]);
#pragma unroll
    for (int db = 0; db < NDB; db++) {
      if constexpr (TL_PF) {
        if (db + 1 < NDB) vread(Vc, db + 1, vt[(db + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
      } else {
        vread(Vc, db, vt[db & 1]);
      }
      const bf16x8 v0 = vt[db & 1][0], v1 = vt[db & 1][1], v2 = vt[db & 1][2];
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v2, b0, oacc[db], 0, 0, 0);
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v0, b2, oacc[db], 0, 0, 0);
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v1, b1, oacc[db], 0, 0, 0);
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v1, b0, oacc[db], 0, 0, 0);
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v0, b1, oacc[db], 0, 0, 0);
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v0, b0, oacc[db], 0, 0, 0);
    }
  };
  // softmax of tile tt's scores against the lazy offset: the new offset and
  // the scale alpha for what O and the sum held, this tile's probability
  // terms and their sum
  auto softmax = [&](int tt, const f32x4 (&sacc)[2], float& alpha, bool& moved, bf16x8& b0, bf16x8& b1,
                     bf16x8& b2) {
    float t[8];
    float tmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int j = tt * TL_KEYS + 16 * (e >> 2) + 4 * g + (e & 3);
      const bool ok = (unsigned)(j - klo) < (unsigned)(khi - klo);
      t[e] = ok ? sacc[e >> 2][e & 3] * p.scale : -INFINITY;
      tmax = fmaxf(tmax, t[e]);
    }
    tmax = rows4_max(tmax);
    const bool need = tmax > m_run + TL_TAU;
    moved = __any(need);
    const float mn = need ? tmax : m_run;
    alpha = exp_flush(m_run - mn);  // 1 where the offset stays, 0 for the first valid tile
    m_run = mn;
    uint32_t ph[8], pm[8], pl[8];
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float pv_ = exp_flush(t[e] - mn);  // masked keys: -inf, flushed to 0
      psum += pv_;
      const Split3 sp = split3(pv_);
      ph[e] = sp.h;
      pm[e] = sp.m;
      pl[e] = sp.l;
    }
    l_part = l_part * alpha + psum;
    b0 = as_bf16x8(u32x4{pack_hi16(ph[0], ph[1]), pack_hi16(ph[2], ph[3]), pack_hi16(ph[4], ph[5]),
                         pack_hi16(ph[6], ph[7])});
    b1 = as_bf16x8(u32x4{pack_hi16(pm[0], pm[1]), pack_hi16(pm[2], pm[3]), pack_hi16(pm[4], pm[5]),
                         pack_hi16(pm[6], pm[7])});
    b2 = as_bf16x8(u32x4{pack_hi16(pl[0], pl[1]), pack_hi16(pl[2], pl[3]), pack_hi16(pl[4], pl[5]),
                         pack_hi16(pl[6], pl[7])});
  };

  // Software pipeline, iteration tt: [barrier: K(tt), V(tt-1) landed; every
  // wave done with iteration tt-1] load V(tt); S(tt) = K(tt).Q^T; [barrier:
  // every wave done with the keys] load K(tt+1) (the last again past the
  // end); P.V of tile tt-1 with the softmax of tile tt written between its
  // blocks in four stages (each stage's results pinned where it is written,
  // so the VALU work sits among the MFMAs instead of after them), then O's
  // rescale, which must see tile tt-1's terms. Then P.V of the last tile. One key buffer and two
  // value buffers (144 KB).
  bf16x8 pb0, pb1, pb2;  // tile tt-1's probability terms
  // Tile tb + i's values go to Vs0 for even i, Vs1 for odd i: every LDS
  // access names its buffer statically (the compiler then keeps the other
  // buffer's loads in flight across the reads).
  // barrier, this tile's value loads into Vn, scores, barrier, the next
  // tile's key loads
  auto front = [&](int tt, uint16_t* Vn, f32x4 (&sacc)[2]) {
    dl_barrier<0x0F70>();  // vmcnt(0): K(tt), V(tt-1) landed (own loads, then everyone's)
    issue(img0 + tt * tstride + TL_IMG, Vn);
    qk(Ks, sacc);
    if constexpr (DS == 2) {
      Xs[(2 * wave) * 64 + lane] = sacc[0];
      Xs[(2 * wave + 1) * 64 + lane] = sacc[1];
    }
    dl_barrier<0xC07F>();  // every wave's key reads (and partial-score writes) done; no wait for the loads
    issue(img0 + min(tt + 1, te - 1) * tstride, Ks);
    if constexpr (DS == 2) {  // the partner's half (it writes again only after the next barrier)
      const int pw = wave ^ RB;
      sacc[0] = sacc[0] + Xs[(2 * pw) * 64 + lane];
      sacc[1] = sacc[1] + Xs[(2 * pw + 1) * 64 + lane];
    }
  };
  // P.V of tile tt-1 (terms pb*) with the softmax of tile tt (scores sacc)
  // written between its blocks of 16 dims, in four stages, so that the
  // VALU work sits among the MFMAs; the new terms replace pb* at the end
  auto pv_softmax = [&](const uint16_t* Vp, int tt, const f32x4 (&sacc)[2], float& alpha, bool& moved) {
    float t[8];
    float tmax = -INFINITY, mn = 0.f, psum = 0.f;
    uint32_t ph[8], pm[8], pl[8];
    constexpr int WPS = DS == 2 ? 2 : 1;  // weights per block in the last stage
    bf16x8 vt[2][3];
    if constexpr (TL_PF) vread(Vp, 0, vt[0]);
#pragma unroll
    for (int db = 0; db < NDB; db++) {
      if constexpr (TL_PF) {
        if (db + 1 < NDB) vread(Vp, db + 1, vt[(db + 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
      } else {
        vread(Vp, db, vt[db & 1]);
      }
      const bf16x8 v0 = vt[db & 1][0], v1 = vt[db & 1][1], v2 = vt[db & 1][2];
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v2, pb0, oacc[db], 0, 0, 0);
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v0, pb2, oacc[db], 0, 0, 0);
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v1, pb1, oacc[db], 0, 0, 0);
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v1, pb0, oacc[db], 0, 0, 0);
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v0, pb1, oacc[db], 0, 0, 0);
      oacc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v0, pb0, oacc[db], 0, 0, 0);
      if (db < 2) {  // scaled, masked scores (four per block) and the lane's maximum
#pragma unroll
        for (int e = 4 * db; e < 4 * db + 4; e++) {
          const int j = tt * TL_KEYS + 16 * (e >> 2) + 4 * g + (e & 3);
          const bool ok = (unsigned)(j - klo) < (unsigned)(khi - klo);
          t[e] = ok ? sacc[e >> 2][e & 3] * p.scale : -INFINITY;
          tmax = fmaxf(tmax, t[e]);
          asm volatile("" ::"v"(t[e]));  // computed here, not sunk to the use
        }
      } else if (db == 2) {  // the row's maximum
        tmax = rows4_max(tmax);
        asm volatile("" ::"v"(tmax));
      } else if (db == 3) {  // the offset
        const bool need = tmax > m_run + TL_TAU;
        moved = __any(need);
        mn = need ? tmax : m_run;
        alpha = exp_flush(m_run - mn);  // 1 where the offset stays, 0 for the first valid tile
        m_run = mn;
        asm volatile("" ::"v"(alpha), "v"(mn));
      } else if (db >= 4 && db < 4 + 8 / WPS) {  // WPS weights (masked keys: -inf, flushed to 0) and their exact bf16 terms
#pragma unroll
        for (int u = 0; u < WPS; u++) {
          const int e = (db - 4) * WPS + u;
          const float w = exp_flush(t[e] - mn);
          psum += w;
          const Split3 sp = split3(w);
          ph[e] = sp.h;
          pm[e] = sp.m;
          pl[e] = sp.l;
          asm volatile("" ::"v"(ph[e]), "v"(pm[e]), "v"(pl[e]), "v"(psum));
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    l_part = l_part * alpha + psum;
    pb0 = as_bf16x8(u32x4{pack_hi16(ph[0], ph[1]), pack_hi16(ph[2], ph[3]), pack_hi16(ph[4], ph[5]),
                          pack_hi16(ph[6], ph[7])});
    pb1 = as_bf16x8(u32x4{pack_hi16(pm[0], pm[1]), pack_hi16(pm[2], pm[3]), pack_hi16(pm[4], pm[5]),
                          pack_hi16(pm[6], pm[7])});
    pb2 = as_bf16x8(u32x4{pack_hi16(pl[0], pl[1]), pack_hi16(pl[2], pl[3]), pack_hi16(pl[4], pl[5]),
                          pack_hi16(pl[6], pl[7])});
  };
  auto iter = [&](int tt, uint16_t* Vn, const uint16_t* Vp) {
    f32x4 sacc[2];
    front(tt, Vn, sacc);
    float alpha;
    bool moved;
    pv_softmax(Vp, tt, sacc, alpha, moved);
    if (moved) {
#pragma unroll
      for (int db = 0; db < NDB; db++) oacc[db] *= alpha;
    }
  };
  if (tb < te) {
    {
      f32x4 sacc[2];
      front(tb, Vs0, sacc);
      float alpha;
      bool moved;
      softmax(tb, sacc, alpha, moved, pb0, pb1, pb2);  // O is still zero
    }
    int tt = tb + 1;
    for (; tt + 1 < te; tt += 2) {
      iter(tt, Vs1, Vs0);
      __builtin_amdgcn_sched_barrier(0);  // no code motion between the two halves (register pressure)
      iter(tt + 1, Vs0, Vs1);
    }
    if (tt < te) iter(tt, Vs1, Vs0);
    dl_barrier<0x0F70>();  // V(te-1) landed everywhere
    // the last tile's values: one P.V for either parity (no loads follow,
    // so the buffer need not be named statically here)
    pv(((te - 1 - tb) & 1) ? Vs1 : Vs0, pb0, pb1, pb2);
  } else {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the first image issued above
  }

  const float l_tot = rows4_sum(l_part);
  if (!qvalid) return;
  const int OW = p.H * HD;
  if (p.kparts > 1) {
    const int64_t arow = seq_row + tok;  // absolute packed row
    float* orow = p.part + ((int64_t)part * p.rows + arow) * OW + (int64_t)head * HD + 16 * NDB * hf + 4 * g;
#pragma unroll
    for (int db = 0; db < NDB; db++) *reinterpret_cast<f32x4*>(orow + 16 * db) = oacc[db];
    if (g == 0 && hf == 0) {
      float2* pml = reinterpret_cast<float2*>(p.part + (int64_t)p.kparts * p.rows * OW);
      pml[((int64_t)part * p.rows + arow) * p.H + head] = make_float2(m_run, l_tot);
    }
    return;
  }
  const float inv = 1.f / l_tot;
  float* orow = p.out + (start + tok) * OW + (int64_t)head * HD + 16 * NDB * hf + 4 * g;
#pragma unroll
  for (int db = 0; db < NDB; db++) *reinterpret_cast<f32x4*>(orow + 16 * db) = oacc[db] * inv;
}

// ---- dense attention on the MFMA (the tensor.AttentionScaled drop-in) ----------
// attention_dense_kernel<HD, DSPLIT> computes fa_attention's result for
// head_dim HD in {64, 128, 256, 512}: q [B,H,T,HD], k/v [B,H,S,HD] with
// arbitrary (16-byte multiple) batch and head strides (stride 0 for GQA's
// Expand) and rows of HD contiguous, and any additive mask tensor read
// through its broadcast strides. The reference's algebra
// (internal/blas/attention.go:105-122): raw scores s = q.k, with scale > 0
// row = s + mask/scale, weights exp(scale*row - scale*max(row)) with the
// flush below -87 (generic.go:278-307), so masked keys get weight exactly 0;
// with scale <= 0 the scores are scaled first and the mask added as is.
//
// Formulation as attention_varlen_kernel's (v_mfma_f32_16x16x4_f32): a wave
// owns 16 queries and HD/DSPLIT head dimensions, computes S^T = K.Q^T for a
// tile of 16 keys (lane l: query l%16 against keys 4(l/16)+r) and O += P.V
// with its probabilities as the A operand. DSPLIT = 1 (HD <= 256): four
// waves own 64 queries and the full head each, no exchange; DSPLIT = 2 (HD =
// 512): wave pairs split the head and add their partial scores through LDS.
// A work item is (batch, head, block of queries); K and V tiles are the
// contiguous 16*HD floats of 16 key rows, loaded straight into two LDS
// buffers (global_load_lds, 1 KB per wave instruction, 16-byte chunks
// XOR-swizzled by row), the next tile loading during the current one.
struct DenseParams {
  const float *q, *k, *v, *mask;
  float* out;
  int32_t H, T, S;
  int64_t q_sb, q_sh, k_sb, k_sh, v_sb, v_sh, m_sb, m_sh, m_sr, m_sc;
  float scale;
  int32_t qblocks;  // query blocks per (batch, head)
};

template <int HD, int DSPLIT>
__global__ __launch_bounds__(DL_NT) void attention_dense_kernel(DenseParams p) {
  constexpr int DW = HD / DSPLIT;  // head dimensions per wave
  constexpr int QB = 16 * (4 / DSPLIT);  // queries per item
  constexpr int ROWF = HD;
  constexpr int LOADS = KT * HD / 256 / 4;  // 1 KB loads per wave per K (or V) tile
  static_assert(HD >= 64 && LOADS >= 1, "head dimension");
  __shared__ __attribute__((aligned(16))) float K0[KT * ROWF];
  __shared__ __attribute__((aligned(16))) float V0[KT * ROWF];
  __shared__ __attribute__((aligned(16))) float K1[KT * ROWF];
  __shared__ __attribute__((aligned(16))) float V1[KT * ROWF];
  __shared__ __attribute__((aligned(16))) float Sx[DSPLIT == 2 ? 4 : 1][64 * 4];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int grp = wave / DSPLIT, half = wave % DSPLIT;
  const int g = lane >> 4;
  const int lq = lane & 15;

  const int bh = blockIdx.x / p.qblocks, qblk = blockIdx.x % p.qblocks;
  const int b = bh / p.H, h = bh % p.H;
  const int dofs = half * DW;
  const float* kbase = p.k + b * p.k_sb + h * p.k_sh;
  const float* vbase = p.v + b * p.v_sb + h * p.v_sh;
  const int S = p.S;

  const int qi = qblk * QB + grp * 16 + lq;
  const bool qvalid = qi < p.T;
  const int qc = qvalid ? qi : p.T - 1;
  f32x4 qreg[DW / 16];
  {
    const float* qr = p.q + b * p.q_sb + h * p.q_sh + (int64_t)qc * HD + dofs;
#pragma unroll
    for (int sg = 0; sg < DW / 16; sg++) qreg[sg] = *reinterpret_cast<const f32x4*>(qr + sg * 16 + g * 4);
  }
  const float* mrow = p.mask ? p.mask + b * p.m_sb + h * p.m_sh + (int64_t)qc * p.m_sr : nullptr;
  const bool pos = p.scale > 0.f;
  const float sa = pos ? p.scale : 1.f, inv_scale = pos ? 1.f / p.scale : 1.f;

  f32x4 oacc[DW / 16];
#pragma unroll
  for (int db = 0; db < DW / 16; db++) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegBig;
  float l_part = 0.f;

  // load j of wave w covers floats (4 LOADS w + j) * 256 .. +255 of the tile
  auto issue_tile = [&](int k0, float* Kb, float* Vb) {
#pragma unroll
    for (int j = 0; j < LOADS; j++) {
      const int f0 = (wave * LOADS + j) * 256;
      const int r = (f0 + lane * 4) / HD;              // tile row of this lane's chunk
      const int cpos = ((f0 + lane * 4) % HD) >> 2;    // its LDS chunk position in the row
      const int64_t key = min(k0 + r, S - 1);
      const int chunk = dl_pos(r, cpos);               // the global chunk that lands there
      __builtin_amdgcn_global_load_lds(kbase + key * HD + chunk * 4,
                                       (__attribute__((address_space(3))) void*)&Kb[f0], 16, 0, 0);
      __builtin_amdgcn_global_load_lds(vbase + key * HD + chunk * 4,
                                       (__attribute__((address_space(3))) void*)&Vb[f0], 16, 0, 0);
    }
  };
  issue_tile(0, K0, V0);

  auto step = [&](int k0, const float* Kc, const float* Vc, float* Kn, float* Vn) {
    dl_barrier<0x0070>();  // this tile landed everywhere; the other buffer is free
    if (k0 + KT < S) issue_tile(k0 + KT, Kn, Vn);
    f32x4 sacc = f32x4{0.f, 0.f, 0.f, 0.f};
    {
      const float* krow = &Kc[lq * ROWF];
      auto kfrag = [&](int sg) {
        return *reinterpret_cast<const f32x4*>(krow + dl_pos(lq, (dofs + sg * 16 + g * 4) >> 2) * 4);
      };
      f32x4 a = kfrag(0);
#pragma unroll
      for (int sg = 0; sg < DW / 16; sg++) {
        const f32x4 an = sg + 1 < DW / 16 ? kfrag(sg + 1) : a;
#pragma unroll
        for (int c = 0; c < 4; c++) sacc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c], qreg[sg][c], sacc, 0, 0, 0);
        a = an;
      }
    }
    if constexpr (DSPLIT == 2) {
      *reinterpret_cast<f32x4*>(&Sx[wave][lane * 4]) = sacc;
      dl_barrier<0xC07F>();  // lgkmcnt(0) only: the next tile's loads stay in flight
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
      valid[r] = j < S;
      float row = sacc[r];
      if (!pos) row = __fmul_rn(row, p.scale);
      if (mrow && valid[r]) row = __fadd_rn(__fmul_rn(inv_scale, mrow[(int64_t)j * p.m_sc]), row);
      const float t = sa * row;
      sacc[r] = t;
      if (valid[r]) tmax = fmaxf(tmax, t);
    }
    tmax = rows4_max(tmax);
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
      for (int db = 0; db < DW / 16; db++) oacc[db][r] *= ar;
    }
#pragma unroll
    for (int db = 0; db < DW / 16; db++) {
      const int f = dofs + db * 16 + lq;
      f32x4 bv;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const int row = 4 * g + c;
        bv[c] = Vc[row * ROWF + dl_pos(row, f >> 2) * 4 + (f & 3)];
      }
#pragma unroll
      for (int c = 0; c < 4; c++) oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(sacc[c], bv[c], oacc[db], 0, 0, 0);
    }
  };
  for (int k0 = 0; k0 < S; k0 += 2 * KT) {
    step(k0, K0, V0, K1, V1);
    if (k0 + KT < S) step(k0 + KT, K1, V1, K0, V0);
  }

  const float l_tot = rows4_sum(l_part);
  float* obase = p.out + ((int64_t)bh * p.T + qblk * QB + grp * 16) * HD + dofs;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int qr = 4 * g + r;
    const float inv = 1.f / __shfl(l_tot, qr, 64);
    if (qblk * QB + grp * 16 + qr < p.T) {
      float* orow = obase + (int64_t)qr * HD;
#pragma unroll
      for (int db = 0; db < DW / 16; db++) orow[db * 16 + lq] = oacc[db][r] * inv;
    }
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
  if (!a.item_ext) return set_error(ctx, FA_ERR_ARG, "attention: no item extents");
  p.qkv = a.qkv; p.out = a.out; p.items = d_items; p.ext = a.item_ext; p.row0 = a.row0;
  p.H = a.H; p.Hkv = a.Hkv; p.window = a.window; p.scale = a.scale;
  p.kparts = a.kparts; p.rows = a.rows; p.part = a.part;
  const dim3 grid((unsigned)((int64_t)n_items * a.kparts));
  if (a.D == 256)
    hipLaunchKernelGGL(attention_varlen_kernel<256>, grid, dim3(DL_NT), 0, s, p);
  else
    hipLaunchKernelGGL(attention_varlen_kernel<512>, grid, dim3(DL_NT), 0, s, p);
  if (a.kparts > 1) {
    // one (row, head) per wave; a short batch (C1: 384) one wave per
    // workgroup, spread over more CUs
    const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    const int per = a.rows * a.H <= 4LL * cus ? 1 : 4;
    const dim3 g2((unsigned)((a.rows * a.H + per - 1) / per)), b2(64 * per);
    if (a.D == 256)
      hipLaunchKernelGGL(attention_combine_kernel<256>, g2, b2, 0, s, a.part, a.kparts, a.rows, (int64_t)0, a.rows,
                         a.H, a.out);
    else
      hipLaunchKernelGGL(attention_combine_kernel<512>, g2, b2, 0, s, a.part, a.kparts, a.rows, (int64_t)0, a.rows,
                         a.H, a.out);
  }
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

// 64-row items on eight waves in dim-split pairs (attention_tiles_kernel<8,
// 2>) instead of four waves; FA_ATTN_PAIRS=0 selects the four-wave kernel.
static bool tiles_pairs() {
  static const bool on = [] {
    const char* e = std::getenv("FA_ATTN_PAIRS");
    return !(e && e[0] == '0');
  }();
  return on;
}

int launch_attention_tiles(fa_ctx* ctx, const AttnTilesArgs& a, const int32_t* d_items, int32_t n_items,
                           hipStream_t s) {
  if (a.Hkv <= 0 || a.H % a.Hkv != 0)
    return set_error(ctx, FA_ERR_ARG, "attention: %d query heads not a multiple of %d kv heads", a.H, a.Hkv);
  if (a.waves != 4 && a.waves != 8) return set_error(ctx, FA_ERR_ARG, "attention: %d waves per item (4 or 8)", a.waves);
  if (n_items == 0) return FA_OK;
  if (a.kparts < 1 || a.kparts > kMaxKeyParts || (a.kparts > 1 && (!a.part || a.rows <= 0 || a.nrows <= 0)))
    return set_error(ctx, FA_ERR_ARG, "attention: %d key parts (1..%d, > 1 needs a partial buffer)", a.kparts,
                     kMaxKeyParts);
  if (!a.item_ext) return set_error(ctx, FA_ERR_ARG, "attention: no item extents");
  TilesParams p;
  p.qkv = a.qkv; p.img = a.img; p.out = a.out; p.items = d_items; p.ext = a.item_ext;
  p.H = a.H; p.Hkv = a.Hkv; p.window = a.window; p.scale = a.scale; p.row0 = a.row0;
  p.kparts = a.kparts; p.rows = a.rows; p.part = a.part;
  p.gq = a.gq; p.cs = a.cos_t; p.sn = a.sin_t; p.eps = a.eps;
  const dim3 grid((unsigned)((int64_t)n_items * a.kparts));
  if (a.waves == 4 && tiles_pairs())
    hipLaunchKernelGGL((attention_tiles_kernel<8, 2>), grid, dim3(64 * 8), 0, s, p);
  else if (a.waves == 4)
    hipLaunchKernelGGL((attention_tiles_kernel<4, 1>), grid, dim3(64 * 4), 0, s, p);
  else
    hipLaunchKernelGGL((attention_tiles_kernel<8, 1>), grid, dim3(64 * 8), 0, s, p);
  if (a.kparts > 1)
    hipLaunchKernelGGL(attention_combine_kernel<256>, dim3((unsigned)((a.nrows * a.H + 3) / 4)), dim3(256), 0, s,
                       a.part, a.kparts, a.rows, a.row0, a.nrows, a.H, a.out);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int attention_varlen_qblock() { return QBLK; }
int attention_tiles_rows(int waves) { return 16 * waves; }
int attention_tiles_keys() { return TL_KEYS; }

bool attention_dense_ok(const AttnGenericArgs& a) {
  static const bool off = [] {
    const char* e = std::getenv("FA_ATTN_DENSE");
    return e && e[0] == '0';
  }();
  auto al = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const int64_t qblocks = (a.T + 63) / 64;
  return !off && (a.D == 64 || a.D == 128 || a.D == 256 || a.D == 512) && a.T > 0 && a.S > 0 && al(a.q) &&
         al(a.k) && al(a.v) && a.q_sb % 4 == 0 && a.q_sh % 4 == 0 && a.k_sb % 4 == 0 && a.k_sh % 4 == 0 &&
         a.v_sb % 4 == 0 && a.v_sh % 4 == 0 && (int64_t)a.B * a.H * qblocks * 2 < INT32_MAX;
}

int launch_attention_dense(fa_ctx* ctx, const AttnGenericArgs& a, hipStream_t s) {
  if (!attention_dense_ok(a)) return set_error(ctx, FA_ERR_UNSUPPORTED, "Attention: no MFMA path for these operands");
  DenseParams p;
  p.q = a.q; p.k = a.k; p.v = a.v; p.mask = a.mask; p.out = a.out;
  p.H = a.H; p.T = a.T; p.S = a.S;
  p.q_sb = a.q_sb; p.q_sh = a.q_sh; p.k_sb = a.k_sb; p.k_sh = a.k_sh; p.v_sb = a.v_sb; p.v_sh = a.v_sh;
  p.m_sb = a.m_sb; p.m_sh = a.m_sh; p.m_sr = a.m_sr; p.m_sc = a.m_sc;
  p.scale = a.scale;
  const int qb = a.D >= 256 ? 32 : 64;  // DSPLIT = 2 from head_dim 256: wave pairs share 16 queries
  p.qblocks = (a.T + qb - 1) / qb;
  const dim3 grid((unsigned)((int64_t)a.B * a.H * p.qblocks)), block(DL_NT);
  switch (a.D) {
    case 64: hipLaunchKernelGGL((attention_dense_kernel<64, 1>), grid, block, 0, s, p); break;
    case 128: hipLaunchKernelGGL((attention_dense_kernel<128, 1>), grid, block, 0, s, p); break;
    case 256: hipLaunchKernelGGL((attention_dense_kernel<256, 2>), grid, block, 0, s, p); break;
    default: hipLaunchKernelGGL((attention_dense_kernel<512, 2>), grid, block, 0, s, p); break;
  }
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_attention_generic(fa_ctx* ctx, const AttnGenericArgs& a, hipStream_t s) {
  if (a.D > GMAXD) return set_error(ctx, FA_ERR_UNSUPPORTED, "Attention: head dimension %d > %d", a.D, GMAXD);
  const int64_t rows = (int64_t)a.B * a.H * a.T;
  if (rows == 0) return FA_OK;
  hipLaunchKernelGGL(attention_generic_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, a);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

}  // namespace fa
