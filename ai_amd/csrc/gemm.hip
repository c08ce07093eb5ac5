// MFMA GEMMs for gfx950 with fp32 results: C = epilogue(A . B).
//
// A: fp32 [m x k] row-major. B: logical [k x n], stored bf16 or fp32, either
// as [n x k] rows (checkpoint [out,in] weights, docs) or [k x n] rows.
//
// Two kernels:
//  - gemm_x3_kernel (bf16 [n x k] weights, the encoder's path): each fp32 A
//    value is split exactly into three bf16 terms and multiplied by the bf16
//    weight with v_mfma_f32_32x32x16_bf16, accumulating in fp32 (the products
//    are exact, so the result carries fp32 information at the bf16 MFMA rate
//    divided by three). Described at the kernel.
//  - gemm_kernel (every other operand combination, and fp32 weights): fp32
//    operands on v_mfma_f32_32x32x2_f32, described below.
//
// gemm_kernel: a workgroup computes a BM x BN tile of C with WM x WN waves;
// each wave owns a (BM/WM) x (BN/WN) sub-tile made of 32x32 blocks of
// v_mfma_f32_32x32x2_f32 (16 accumulators per lane per block). K advances in
// slabs of BK through two LDS buffers: the next slab's global loads are
// issued at the top of a slab, written to the other buffer before the slab's
// last MFMA step, and one barrier per slab separates the buffers. The first
// operand reads of the next slab are issued right after that barrier, so
// their latency overlaps the current slab's last MFMAs; within a slab the
// operands of step s+1 are read while the MFMAs of step s run. bf16 weights
// are widened to fp32 (exact) when written to LDS, so the MFMA operands are
// always fp32.
//
// MFMA operand layout (32x32x2, one block): lane l supplies A[row l%32][k]
// and B[k][col l%32] with k = l/32; the 16 results of lane l are C[row][col]
// with col = l%32 and row = 8*(r/4) + 4*(l/32) + r%4 for r = 0..15. A
// product does not depend on the order of its k terms, so each lane reads
// four consecutive k values with one 16-byte LDS read: lanes 0-31 take
// k = 8s..8s+3 and lanes 32-63 take k = 8s+4..8s+7, and MFMA number c (0..3)
// pairs k = 8s+c with 8s+4+c on both operands.
//
// Work distribution (both kernels): one workgroup per tile, XCD-aware tile
// order, tile shape chosen per call from the output's tile count. A
// stream-K distribution (equal shares of (tile, K-slab) units plus a fixup
// pass over split tiles) measured slower at these sizes: the fixup pass alone
// costs 45-60 us at the C2 shapes.
//
// Epilogues: None; Generic (bias, row scale, activation, element-wise
// multiply, residual: the reference's order, internal/blas/gemm.go:276-347);
// GeGLU (gate and up weights interleaved in 32-row groups, so a wave's column
// blocks 2p and 2p+1 hold gate and up of the same 32 features and the lane
// writes gelu_tanh(gate) * up, models/gemma/embed.go:226-227).

#include <cstdlib>
#include <algorithm>
#include <cstring>

#include "fa_internal.h"
#include "device_math.h"

namespace fa {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct Tile {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
  static constexpr int NT = WM * WN * 64;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 32, FN = TN / 32;
  static constexpr int LDSK = BK + 4;  // padded LDS row stride (floats): rows start 4 banks apart
  static constexpr int S = BK / 8;     // MFMA steps (of 4 MFMA k-pairs) per slab
  static constexpr int ACC = FM * FN * 16;  // accumulators per lane
  static_assert(TM % 32 == 0 && TN % 32 == 0 && BK % 8 == 0, "tile shape");
  static_assert((BM * BK / 4) % NT == 0 && (BN * BK / 8) % NT == 0 && (BN * BK / 4) % NT == 0, "loader shape");
  static_assert((BM * BK) % NT == 0 && (BN * BK) % NT == 0, "checked loader shape");
};

// Tile shapes compiled into the library.
using T128x128 = Tile<128, 128, 32, 2, 2>;  // 4 waves of 64x64
using T64x64 = Tile<64, 64, 32, 2, 2>;      // 4 waves of 32x32
using T128x64v = Tile<128, 64, 32, 4, 1>;   // 4 waves of 32x64 (column-block pairs for GeGLU)

struct GemmParams {
  int64_t m, n, k;
  const float* a;
  int64_t lda;
  const void* b;
  int64_t ldb;
  float* c;
  int64_t ldc;
  const float* bias;
  const float* row_scale;
  const float* mul;
  int64_t ldm;
  const float* residual;
  int64_t ldr;
  int act;
  int tiles_m, tiles_n;
  int nk;  // K slabs per tile
  // split-bf16 kernel: K split into ksplit equal ranges (grid.y); range s
  // writes its partial product to c + s * c_split (epilogue None)
  int ksplit;
  int64_t c_split;
  // split-bf16 kernel with BT = 3: B is three bf16 planes (hi, mid, lo of
  // fp32 weights) b_plane elements apart
  int64_t b_plane;
  // batched products (grid.z = batch entries, BT = 3 only): entry z reads A
  // at a + z * a_bs, B at b + z * b_bs (bf16 elements) and writes c + z * c_bs
  int64_t a_bs, b_bs, c_bs;
  int nbatch;
};

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Tile index of this workgroup. Workgroup ids are dealt to the 8 XCDs
// round-robin; each XCD gets a contiguous run of tiles (row-major over n) so
// the tiles sharing A rows and B columns share that XCD's L2.
__device__ __forceinline__ int xcd_tile(const GemmParams& p) {
  constexpr int kXcd = 8;
  const int total = p.tiles_m * p.tiles_n;
  int tile = blockIdx.x;
  const int per = total / kXcd;
  if (per > 0 && tile < per * kXcd) tile = (tile % kXcd) * per + tile / kXcd;
  return tile;
}

// The Generic epilogue of one element (the reference's order,
// internal/blas/gemm.go:276-347); None returns v.
template <Epi EPI>
__device__ __forceinline__ float epi_value(const GemmParams& p, float v, int64_t row, int64_t col) {
  if constexpr (EPI == Epi::Generic) {
    if (p.bias) v = v + p.bias[col];
    if (p.row_scale) v = v * p.row_scale[row];
    if (p.act == FA_ACT_RELU) v = fmaxf(v, 0.f);
    else if (p.act == FA_ACT_GELU) v = gelu_tanh_ref(v);
    else if (p.act == FA_ACT_TANH) v = tanh_ref(v);
    if (p.mul) v = v * p.mul[row * p.ldm + col];
    if (p.residual) v = v + p.residual[row * p.ldr + col];
  }
  return v;
}

// Writes a wave's accumulators (FM x FN blocks of 32x32 in the MFMA C
// layout) through the epilogue. Shared by the fp32 and split-bf16 kernels,
// whose 32x32 MFMAs have the same C layout. Lane l holds rows
// 8*(r/4) + 4*(l/32) + r%4 of column l%32 of each block. A wave whose
// sub-tile lies inside C (every wave of an interior tile) stores without
// per-element bounds tests, from one base address and 16 precomputed row
// offsets; the tests made each of the lane's values a branch region.
template <class TL, Epi EPI>
__device__ __forceinline__ void store_c(const GemmParams& p, const f32x16 (&acc)[TL::FM][TL::FN], int64_t m0,
                                        int64_t n0, int wm, int wn, int lane) {
  constexpr int FM = TL::FM, FN = TL::FN;
  const int64_t M = p.m, N = p.n;
  const int lcol = lane & 31;
  const int lrow4 = (lane >> 5) * 4;
  const int64_t r0 = m0 + wm * TL::TM, c0 = n0 + wn * TL::TN;
  const bool inside = r0 + TL::TM <= M && c0 + TL::TN <= N;
  int roff[16];  // element offsets of the lane's 16 rows in a block (ldc < 2^26: launch_gemm)
#pragma unroll
  for (int r = 0; r < 16; r++) roff[r] = EPI == Epi::Generic ? 0 : ((r >> 2) * 8 + lrow4 + (r & 3)) * (int)p.ldc;
  if constexpr (EPI == Epi::GeGLU) {
    static_assert(FN % 2 == 0, "GeGLU pairs column blocks");
    const int64_t F = N / 2;
#pragma unroll
    for (int pj = 0; pj < FN / 2; pj++) {
      const int64_t fcol = c0 / 2 + pj * 32 + lcol;
#pragma unroll
      for (int i = 0; i < FM; i++) {
        float* base = p.c + (r0 + i * 32) * p.ldc + fcol;
        if (inside) {
#pragma unroll
          for (int r = 0; r < 16; r++) base[roff[r]] = gelu_tanh_ref(acc[i][2 * pj][r]) * acc[i][2 * pj + 1][r];
        } else {
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const int64_t row = r0 + i * 32 + (r >> 2) * 8 + lrow4 + (r & 3);
            if (row < M && fcol < F) base[roff[r]] = gelu_tanh_ref(acc[i][2 * pj][r]) * acc[i][2 * pj + 1][r];
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < FM; i++) {
#pragma unroll
      for (int j = 0; j < FN; j++) {
        const int64_t col = c0 + j * 32 + lcol;
        if constexpr (EPI == Epi::None) {
          float* base = p.c + (r0 + i * 32) * p.ldc + col;
          if (inside) {
#pragma unroll
            for (int r = 0; r < 16; r++) base[roff[r]] = acc[i][j][r];
            continue;
          }
        }
        // (the Generic epilogue keeps one checked path: its optional operands
        // already hold many registers)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int64_t row = r0 + i * 32 + (r >> 2) * 8 + lrow4 + (r & 3);
          if (row < M && col < N) p.c[row * p.ldc + col] = epi_value<EPI>(p, acc[i][j][r], row, col);
        }
      }
    }
  }
}

template <class TL, bool BBF16, bool BNK, bool FAST, Epi EPI>
__global__ __launch_bounds__(TL::NT) void gemm_kernel(GemmParams p) {
  constexpr int BM = TL::BM, BN = TL::BN, BK = TL::BK, NT = TL::NT, LDSK = TL::LDSK;
  constexpr int FM = TL::FM, FN = TL::FN, S = TL::S;
  __shared__ __attribute__((aligned(16))) float As[2][BM * LDSK];
  __shared__ __attribute__((aligned(16))) float Bs[2][BN * LDSK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / TL::WN, wn = wave % TL::WN;
  const int64_t M = p.m, N = p.n, K = p.k;
  const float* __restrict__ A = p.a;

  int64_t m0 = 0, n0 = 0;  // current tile origin

  // ---- global -> register staging ----
  constexpr int NA = BM * BK / 4 / NT;   // float4 of A per thread
  constexpr int NBH = BN * BK / 8 / NT;  // 8 x bf16 of B per thread
  constexpr int NBF = BN * BK / 4 / NT;  // float4 of fp32 B per thread
  constexpr int NCA = BM * BK / NT;      // checked path: elements per thread
  constexpr int NCB = BN * BK / NT;
  f32x4 ra[FAST ? NA : 1];
  uint4 rbh[(FAST && BBF16) ? NBH : 1];
  f32x4 rbf[(FAST && !BBF16) ? NBF : 1];
  float rs_a[FAST ? 1 : NCA], rs_b[FAST ? 1 : NCB];

  auto load_global = [&](int64_t k0) {
    if constexpr (FAST) {
#pragma unroll
      for (int i = 0; i < NA; i++) {
        const int idx = tid + NT * i;
        const int row = idx / (BK / 4), col = (idx % (BK / 4)) * 4;
        const int64_t gr = min(m0 + row, M - 1);
        ra[i] = *reinterpret_cast<const f32x4*>(A + gr * p.lda + k0 + col);
      }
      if constexpr (BBF16) {
        const uint16_t* B = static_cast<const uint16_t*>(p.b);
#pragma unroll
        for (int i = 0; i < NBH; i++) {
          const int idx = tid + NT * i;
          const int row = idx / (BK / 8), col = (idx % (BK / 8)) * 8;
          const int64_t gn = min(n0 + row, N - 1);
          rbh[i] = *reinterpret_cast<const uint4*>(B + gn * p.ldb + k0 + col);
        }
      } else {
        const float* B = static_cast<const float*>(p.b);
#pragma unroll
        for (int i = 0; i < NBF; i++) {
          const int idx = tid + NT * i;
          const int row = idx / (BK / 4), col = (idx % (BK / 4)) * 4;
          const int64_t gn = min(n0 + row, N - 1);
          rbf[i] = *reinterpret_cast<const f32x4*>(B + gn * p.ldb + k0 + col);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < NCA; i++) {
        const int idx = tid + NT * i;
        const int row = idx / BK, col = idx % BK;
        const int64_t gr = m0 + row, gk = k0 + col;
        rs_a[i] = (gr < M && gk < K) ? A[gr * p.lda + gk] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < NCB; i++) {
        const int idx = tid + NT * i;
        int nn, kk;
        if constexpr (BNK) {
          nn = idx / BK; kk = idx % BK;
        } else {
          nn = idx % BN; kk = idx / BN;
        }
        const int64_t gn = n0 + nn, gk = k0 + kk;
        float v = 0.f;
        if (gn < N && gk < K) {
          const int64_t off = BNK ? gn * p.ldb + gk : gk * p.ldb + gn;
          if constexpr (BBF16) v = bf16_to_f32(static_cast<const uint16_t*>(p.b)[off]);
          else v = static_cast<const float*>(p.b)[off];
        }
        rs_b[i] = v;
      }
    }
  };

  auto store_lds = [&](int buf) {
    if constexpr (FAST) {
#pragma unroll
      for (int i = 0; i < NA; i++) {
        const int idx = tid + NT * i;
        const int row = idx / (BK / 4), col = (idx % (BK / 4)) * 4;
        *reinterpret_cast<f32x4*>(&As[buf][row * LDSK + col]) = ra[i];
      }
      if constexpr (BBF16) {
#pragma unroll
        for (int i = 0; i < NBH; i++) {
          const int idx = tid + NT * i;
          const int row = idx / (BK / 8), col = (idx % (BK / 8)) * 8;
          f32x4 lo, hi;
          lo.x = __uint_as_float(rbh[i].x << 16); lo.y = __uint_as_float(rbh[i].x & 0xFFFF0000u);
          lo.z = __uint_as_float(rbh[i].y << 16); lo.w = __uint_as_float(rbh[i].y & 0xFFFF0000u);
          hi.x = __uint_as_float(rbh[i].z << 16); hi.y = __uint_as_float(rbh[i].z & 0xFFFF0000u);
          hi.z = __uint_as_float(rbh[i].w << 16); hi.w = __uint_as_float(rbh[i].w & 0xFFFF0000u);
          *reinterpret_cast<f32x4*>(&Bs[buf][row * LDSK + col]) = lo;
          *reinterpret_cast<f32x4*>(&Bs[buf][row * LDSK + col + 4]) = hi;
        }
      } else {
#pragma unroll
        for (int i = 0; i < NBF; i++) {
          const int idx = tid + NT * i;
          const int row = idx / (BK / 4), col = (idx % (BK / 4)) * 4;
          *reinterpret_cast<f32x4*>(&Bs[buf][row * LDSK + col]) = rbf[i];
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < NCA; i++) {
        const int idx = tid + NT * i;
        As[buf][(idx / BK) * LDSK + (idx % BK)] = rs_a[i];
      }
#pragma unroll
      for (int i = 0; i < NCB; i++) {
        const int idx = tid + NT * i;
        int nn, kk;
        if constexpr (BNK) {
          nn = idx / BK; kk = idx % BK;
        } else {
          nn = idx % BN; kk = idx / BN;
        }
        Bs[buf][nn * LDSK + kk] = rs_b[i];
      }
    }
  };

  const int arow = wm * TL::TM + (lane & 31);
  const int brow = wn * TL::TN + (lane & 31);
  const int kofs = (lane >> 5) * 4;
  auto read_ops = [&](int buf, int s, f32x4 (&oa)[FM], f32x4 (&ob)[FN]) {
#pragma unroll
    for (int i = 0; i < FM; i++)
      oa[i] = *reinterpret_cast<const f32x4*>(&As[buf][(arow + 32 * i) * LDSK + s * 8 + kofs]);
#pragma unroll
    for (int j = 0; j < FN; j++)
      ob[j] = *reinterpret_cast<const f32x4*>(&Bs[buf][(brow + 32 * j) * LDSK + s * 8 + kofs]);
  };

  f32x16 acc[FM][FN];

  // acc = A[m0:m0+BM, slabs kb..ke) . B[slabs kb..ke), n0:n0+BN]
  auto mainloop = [&](int kb, int ke) {
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
      for (int j = 0; j < FN; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;
    if (ke <= kb) return;
    f32x4 ca[FM], cb[FN];  // operands of the current step
    __syncthreads();       // the LDS buffers may still be read by a previous tile
    load_global((int64_t)kb * BK);
    store_lds(0);
    __syncthreads();
    read_ops(0, 0, ca, cb);
    for (int kt = kb; kt < ke; kt++) {
      const int buf = (kt - kb) & 1;
      const bool more = kt + 1 < ke;
      if (more) load_global((int64_t)(kt + 1) * BK);
#pragma unroll
      for (int s = 0; s < S; s++) {
        f32x4 na[FM], nb[FN];
        if (s + 1 < S) {
          read_ops(buf, s + 1, na, nb);
        } else if (more) {
          store_lds(buf ^ 1);
          __syncthreads();
          read_ops(buf ^ 1, 0, na, nb);
        }
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
          for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ca[i][c], cb[j][c], acc[i][j], 0, 0, 0);
        if (s + 1 < S || more) {
#pragma unroll
          for (int i = 0; i < FM; i++) ca[i] = na[i];
#pragma unroll
          for (int j = 0; j < FN; j++) cb[j] = nb[j];
        }
      }
    }
  };

  const int tile = xcd_tile(p);
  m0 = (int64_t)(tile / p.tiles_n) * BM;
  n0 = (int64_t)(tile % p.tiles_n) * BN;
  mainloop(0, p.nk);
  store_c<TL, EPI>(p, acc, m0, n0, wm, wn, lane);
}

template <class TL, bool BBF16, bool BNK, bool FAST, Epi EPI>
void launch_dp(GemmParams p, hipStream_t s) {
  p.tiles_m = (int)((p.m + TL::BM - 1) / TL::BM);
  p.tiles_n = (int)((p.n + TL::BN - 1) / TL::BN);
  p.nk = (int)((p.k + TL::BK - 1) / TL::BK);
  dim3 grid(p.tiles_m * p.tiles_n), block(TL::NT);
  hipLaunchKernelGGL((gemm_kernel<TL, BBF16, BNK, FAST, EPI>), grid, block, 0, s, p);
}

// ---------------------------------------------------------------------------
// Split-bf16 kernel for bf16 weights: C = A . B with A fp32, B bf16 [n x k].
//
// Each fp32 value a of A is written to LDS as three bf16 terms with
// a = hi + mid + lo exactly: hi keeps the top 8 significant bits of a
// (truncation), mid the top 8 of the remainder a - hi (exact in fp32), lo
// the rest (at most 8 significant bits, so exact in bf16). Products of a
// bf16 term and a bf16 weight are exact in fp32, and the three
// v_mfma_f32_32x32x16_bf16 per operand pair accumulate them in fp32, so C
// carries the same information as an fp32 product of A and the
// (bf16-exact) weights; only the summation order differs. Non-finite A
// values give NaN (inf - inf in the split).
//
// Operand layout (32x32x16): lane l supplies A[row l%32][8 k values] and
// B[8 k values][col l%32]; the k assignment is any bijection shared by both
// operands, here k = 8*(l/32) .. +7 of each 16-wide step, one 16-byte LDS
// read per operand. C has the 32x32x2 layout (store_c).
//
// Pipeline: slab kt is in LDS buffer kt&1 while registers hold the global
// values of slab kt+1 (split and written to the other buffer during slab kt's
// MFMAs) and receive slab kt+2; one barrier per slab. The loop body has no
// branches (the last loads are clamped, redundant), so the compiler
// interleaves the split's VALU work and the LDS traffic with the MFMAs.
template <int BM_, int BN_, int WM_, int WN_>
struct XTile {
  static constexpr int BM = BM_, BN = BN_, BK = 32, WM = WM_, WN = WN_;
  static constexpr int NT = WM * WN * 64;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 32, FN = TN / 32;
  static constexpr int S = BK / 16;   // MFMA k-steps per slab
  // waves per SIMD the register allocation must allow: two eight-wave
  // workgroups per CU need four (at most 128 VGPRs). The 128x256 tile
  // compiled to 136-152 VGPRs ran one workgroup per CU; capped (a 28-32 byte
  // spill) the C2 gate|up launch takes 65.9 instead of 71.7 us, 32 768 rows
  // 376.7 instead of 393.4 us.
  static constexpr int MINW = (WM * WN == 8 && BN == 256) ? 4 : 1;
  static_assert(TM % 32 == 0 && TN % 32 == 0, "tile shape");
};

using X128x64v = XTile<128, 64, 4, 1>;   // 4 waves of 32x64 (column-block pairs for GeGLU)
using X64x128 = XTile<64, 128, 2, 2>;    // 4 waves of 32x64
using X64x64 = XTile<64, 64, 2, 2>;      // 4 waves of 32x32
using X128x128w8 = XTile<128, 128, 4, 2>;  // 8 waves of 32x64
using X128x256w8 = XTile<128, 256, 4, 2>;  // 8 waves of 32x128 (80 KB of LDS: two workgroups per CU)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// A slab of the split kernel (ROWS rows of 32 bf16: four 16-byte chunks per
// row) is held chunk-major in LDS: chunk c of row r at 16-byte slot
// c * ROWS + (r ^ 2c). gfx950's LDS serves 16-byte reads 16 lanes at a time
// over 64 banks and 16-byte writes 8 lanes at a time over 32 banks (measured
// with SQ_LDS_BANK_CONFLICT on single-pattern probes). The operand reads
// (16 consecutive rows of one chunk per 16 lanes) then cover 16 distinct
// slots mod 16, and the staging writes (lanes 4j..4j+3 write the four chunks
// of one row, so 8 lanes hold two rows: r ^ 2c takes 8 distinct values mod 8)
// are conflict-free too. Row-major rows with the chunks swizzled per row
// measured 2-way conflicts on the reads (8 instead of 4 clocks per wave read).
template <int ROWS>
__device__ __forceinline__ int lds_chunk(int r, int c) { return (c * ROWS + (r ^ (2 * c))) * 8; }


// Staging registers hold vector types (HIP's struct uint4 in an array was
// placed in scratch memory by the compiler).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// BT = 3 (fp32 weights that are not bf16-exact, and fp32 B operands): B
// arrives as three bf16 planes hi + mid + lo (split like A), and each operand
// pair takes the six term products with i + j <= 2; the three dropped ones
// are below 2^-21 of |a| |w| (truncation splits: |mid| < 2^-7 |x|, |lo| <
// 2^-14 |x|).
template <class TL, Epi EPI, int BT = 1>
__global__ __launch_bounds__(TL::NT, TL::MINW) void gemm_x3_kernel(GemmParams p) {
  constexpr int BM = TL::BM, BN = TL::BN, BK = TL::BK, NT = TL::NT;
  constexpr int FM = TL::FM, FN = TL::FN;
  static_assert(TL::S == 2 && BK == 32, "two MFMA k-steps per 32-wide slab");
  static_assert(BT == 1 || BT == 3, "one or three B planes");
  __shared__ __attribute__((aligned(16))) uint16_t As[2][3][BM * BK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BT][BN * BK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / TL::WN, wn = wave % TL::WN;
  const int64_t M = p.m, N = p.n;
  if constexpr (BT == 3) {  // batch entry blockIdx.z (0 and zero strides when not batched)
    p.a += blockIdx.z * p.a_bs;
    p.b = static_cast<const uint16_t*>(p.b) + blockIdx.z * p.b_bs;
    p.c += blockIdx.z * p.c_bs;
  }
  const float* __restrict__ A = p.a;
  const uint16_t* __restrict__ B = static_cast<const uint16_t*>(p.b);

  const int tile = xcd_tile(p);
  const int64_t m0 = (int64_t)(tile / p.tiles_n) * BM;
  const int64_t n0 = (int64_t)(tile % p.tiles_n) * BN;
  const int nk = p.nk / p.ksplit;                      // slabs of this K range
  const int64_t k_off = (int64_t)blockIdx.y * nk * BK;  // its first k

  // Staging chunks: 8 consecutive k of one row (two float4 of A, one 16-byte
  // vector of B). A slab row is 4 chunks.
  constexpr int NA = BM * 4 / NT;  // A chunks per thread
  constexpr int NB = BN * 4 / NT;  // B chunks per thread
  static_assert(NA * NT == BM * 4 && NB * NT == BN * 4, "loader shape");

  int64_t ga[NA];  // element offsets of the A chunks (slab 0)
  const uint16_t* gb[NB];
  int la[NA], lb[NB];  // LDS element offsets of the chunks
#pragma unroll
  for (int i = 0; i < NA; i++) {
    const int idx = tid + NT * i, row = idx >> 2, c = idx & 3;
    ga[i] = min(m0 + row, M - 1) * p.lda + k_off + c * 8;
    la[i] = lds_chunk<BM>(row, c);
  }
#pragma unroll
  for (int i = 0; i < NB; i++) {
    const int idx = tid + NT * i, row = idx >> 2, c = idx & 3;
    gb[i] = B + min(n0 + row, N - 1) * p.ldb + k_off + c * 8;
    lb[i] = lds_chunk<BN>(row, c);
  }
  auto load_global = [&](f32x4 (&ra)[2 * NA], u32x4 (&rb)[BT * NB], int kt) {
#pragma unroll
    for (int i = 0; i < NA; i++) {
      const int64_t off = ga[i] + (int64_t)kt * BK;
      ra[2 * i] = *reinterpret_cast<const f32x4*>(A + off);
      ra[2 * i + 1] = *reinterpret_cast<const f32x4*>(A + off + 4);
    }
#pragma unroll
    for (int t = 0; t < BT; t++)
#pragma unroll
      for (int i = 0; i < NB; i++)
        rb[t * NB + i] = *reinterpret_cast<const u32x4*>(gb[i] + t * p.b_plane + (int64_t)kt * BK);
  };

  // hi + mid + lo = a exactly (split3, device_math.h), two bf16 per dword.
  auto split_store = [&](const f32x4 (&ra)[2 * NA], const u32x4 (&rb)[BT * NB], int buf) {
#pragma unroll
    for (int i = 0; i < NA; i++) {
      uint32_t h[8], m[8], l[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const Split3 sp = split3(ra[2 * i + (e >> 2)][e & 3]);
        h[e] = sp.h;
        m[e] = sp.m;
        l[e] = sp.l;
      }
      *reinterpret_cast<uint4*>(&As[buf][0][la[i]]) =
          make_uint4(pack_hi16(h[0], h[1]), pack_hi16(h[2], h[3]), pack_hi16(h[4], h[5]), pack_hi16(h[6], h[7]));
      *reinterpret_cast<uint4*>(&As[buf][1][la[i]]) =
          make_uint4(pack_hi16(m[0], m[1]), pack_hi16(m[2], m[3]), pack_hi16(m[4], m[5]), pack_hi16(m[6], m[7]));
      *reinterpret_cast<uint4*>(&As[buf][2][la[i]]) =
          make_uint4(pack_hi16(l[0], l[1]), pack_hi16(l[2], l[3]), pack_hi16(l[4], l[5]), pack_hi16(l[6], l[7]));
    }
#pragma unroll
    for (int t = 0; t < BT; t++)
#pragma unroll
      for (int i = 0; i < NB; i++) *reinterpret_cast<u32x4*>(&Bs[buf][t][lb[i]]) = rb[t * NB + i];
  };

  // Operand reads: lane half h takes chunk 2s+h of its row (32 consecutive
  // rows of one chunk per half-wave; 32 rows further is 32 slots further).
  const int arow = wm * TL::TM + (lane & 31);
  const int brow = wn * TL::TN + (lane & 31);
  const int h = lane >> 5;
  auto read_ops = [&](int buf, int s, bf16x8 (&oa)[3][FM], bf16x8 (&ob)[BT][FN]) {
    const int ca = lds_chunk<BM>(arow, 2 * s + h), cb = lds_chunk<BN>(brow, 2 * s + h);
#pragma unroll
    for (int t = 0; t < 3; t++)
#pragma unroll
      for (int i = 0; i < FM; i++) oa[t][i] = *reinterpret_cast<const bf16x8*>(&As[buf][t][ca + 32 * 8 * i]);
#pragma unroll
    for (int t = 0; t < BT; t++)
#pragma unroll
      for (int j = 0; j < FN; j++) ob[t][j] = *reinterpret_cast<const bf16x8*>(&Bs[buf][t][cb + 32 * 8 * j]);
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; i++)
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  auto mfma_step = [&](const bf16x8 (&oa)[3][FM], const bf16x8 (&ob)[BT][FN]) {
    // smallest terms first: (t, u) pairs by decreasing t + u, u <= t + u <= 2
#pragma unroll
    for (int sum = 2; sum >= 0; sum--)
#pragma unroll
      for (int u = 0; u < BT; u++) {
        const int t = sum - u;
        if (t < 0 || (BT == 1 && u > 0)) continue;
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
          for (int j = 0; j < FN; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(oa[t][i], ob[u][j], acc[i][j], 0, 0, 0);
      }
  };

  // Slab kt is in LDS buffer kt&1; `use` holds the global values of slab
  // kt+1 and `fill` receives slab kt+2 (clamped to the last slab: a
  // redundant load keeps the body free of branches, so the split's VALU work
  // and the LDS traffic interleave with the MFMAs).
  auto body = [&](int kt, const f32x4 (&ra_use)[2 * NA], const u32x4 (&rb_use)[BT * NB], f32x4 (&ra_fill)[2 * NA],
                  u32x4 (&rb_fill)[BT * NB]) {
    const int buf = kt & 1;
    load_global(ra_fill, rb_fill, min(kt + 2, nk - 1));
    bf16x8 a0[3][FM], b0[BT][FN], a1[3][FM], b1[BT][FN];
    read_ops(buf, 0, a0, b0);
    read_ops(buf, 1, a1, b1);
    mfma_step(a0, b0);
    split_store(ra_use, rb_use, buf ^ 1);
    mfma_step(a1, b1);
    __syncthreads();
  };

  f32x4 raA[2 * NA], raB[2 * NA];
  u32x4 rbA[BT * NB], rbB[BT * NB];
  load_global(raA, rbA, 0);
  split_store(raA, rbA, 0);
  load_global(raA, rbA, min(1, nk - 1));
  __syncthreads();
  int kt = 0;
  for (; kt + 2 < nk; kt += 2) {
    body(kt, raA, rbA, raB, rbB);
    body(kt + 1, raB, rbB, raA, rbA);
  }
  if (kt + 1 < nk) {
    body(kt, raA, rbA, raB, rbB);
    kt++;
  }
  {
    const int buf = kt & 1;
    bf16x8 a0[3][FM], b0[BT][FN], a1[3][FM], b1[BT][FN];
    read_ops(buf, 0, a0, b0);
    read_ops(buf, 1, a1, b1);
    mfma_step(a0, b0);
    mfma_step(a1, b1);
  }
  if (p.ksplit > 1) {  // this K range's partial product, no epilogue
    GemmParams q = p;
    q.c = p.c + blockIdx.y * p.c_split;
    store_c<TL, Epi::None>(q, acc, m0, n0, wm, wn, lane);
  } else {
    store_c<TL, EPI>(p, acc, m0, n0, wm, wn, lane);
  }
}

template <class TL, Epi EPI, int BT = 1>
void launch_x3(GemmParams p, hipStream_t s) {
  p.tiles_m = (int)((p.m + TL::BM - 1) / TL::BM);
  p.tiles_n = (int)((p.n + TL::BN - 1) / TL::BN);
  p.nk = (int)(p.k / TL::BK);
  if (p.ksplit < 1) p.ksplit = 1;
  if (p.nbatch < 1 || BT != 3) p.nbatch = 1;
  dim3 grid(p.tiles_m * p.tiles_n, p.ksplit, p.nbatch), block(TL::NT);
  hipLaunchKernelGGL((gemm_x3_kernel<TL, EPI, BT>), grid, block, 0, s, p);
}

// ---------------------------------------------------------------------------
// Split-bf16 kernel for few rows (a batch of short sentences, the pooled
// head): the same products as gemm_x3_kernel, organised for latency instead
// of operand reuse. A workgroup of NW waves computes one 32 x 64 tile of C
// (two 32x32 column blocks); wave w takes the w-th of NW equal runs of the
// tile's 32-wide K slabs and reads its operands from global memory straight
// into MFMA operand registers (no operand is shared between waves, so no LDS
// staging), splitting A into hi + mid + lo as it goes, with the next slab's
// loads in flight during the current slab's MFMAs (a ring of four slabs in
// flight measured slower). The NW partial tiles are
// added through LDS in wave order (a fixed order: the result does not depend
// on timing) and the workgroup's threads apply the epilogue. With K split
// across grid.y (p.ksplit > 1) each part writes its partial product to
// c + part * c_split without epilogue, as gemm_x3_kernel does.
// NB = 1 (GeGLU only): a 32 x 32 tile holding 16 features, its columns
// 0-15 the gate and 16-31 the up rows of those features (the weight's
// 32-row gate and up groups, read half a group at a time): twice the
// workgroups of the 32 x 64 tile, each loading half the weight columns.
constexpr int kSmallNW = 8;

template <int NW, Epi EPI, int NB = 2>
__global__ __launch_bounds__(NW * 64) void gemm_x3_small_kernel(GemmParams p) {
  static_assert(NB == 2 || (NB == 1 && EPI == Epi::GeGLU), "narrow tiles: GeGLU only");
  __shared__ __attribute__((aligned(16))) float red[NW][NB][16][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t M = p.m, N = p.n;
  const float* __restrict__ A = p.a;
  const uint16_t* __restrict__ B = static_cast<const uint16_t*>(p.b);
  const int64_t m0 = (int64_t)(blockIdx.x / p.tiles_n) * 32;
  const int64_t n0 = (int64_t)(blockIdx.x % p.tiles_n) * 32 * NB;
  const int nk = p.nk / p.ksplit;  // slabs of this K part
  const int s0 = (int)((int64_t)wave * nk / NW), s1 = (int)((int64_t)(wave + 1) * nk / NW);
  const int64_t k_off = (int64_t)blockIdx.y * nk * 32 + (lane >> 5) * 8;

  // lane l supplies row l%32 of A and column l%32 of each B block, k values
  // 8*(l/32) .. +7 of each 16-wide step (the bijection of gemm_x3_kernel)
  const float* arow = A + min(m0 + (lane & 31), M - 1) * p.lda + k_off;
  // NB = 1: features f0 .. f0 + 15 (f0 = n0 / 2), gate rows in lanes 0-15,
  // up rows (32 further) in lanes 16-31
  const int64_t brow_n = NB == 2 ? n0 + (lane & 31)
                                 : (n0 / 64) * 64 + (n0 / 2) % 32 + (lane & 15) + ((lane & 16) ? 32 : 0);
  const uint16_t* brow0 = B + min(brow_n, N - 1) * p.ldb + k_off;
  const uint16_t* brow1 = B + min(n0 + 32 + (lane & 31), N - 1) * p.ldb + k_off;

  f32x16 acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[j][r] = 0.f;

  // one slab: two k-steps of 16; per step two float4 of A and one 16-byte
  // vector of each B block
  struct Regs {
    f32x4 a[4];
    u32x4 b[2 * NB];
  };
  auto load = [&](Regs& g, int kt) {
    const int64_t o = (int64_t)kt * 32;
#pragma unroll
    for (int st = 0; st < 2; st++) {
      g.a[2 * st] = *reinterpret_cast<const f32x4*>(arow + o + 16 * st);
      g.a[2 * st + 1] = *reinterpret_cast<const f32x4*>(arow + o + 16 * st + 4);
      g.b[NB * st] = *reinterpret_cast<const u32x4*>(brow0 + o + 16 * st);
      if constexpr (NB == 2) g.b[2 * st + 1] = *reinterpret_cast<const u32x4*>(brow1 + o + 16 * st);
    }
  };
  auto compute = [&](const Regs& g) {
#pragma unroll
    for (int st = 0; st < 2; st++) {
      uint32_t h[8], m[8], l[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const Split3 sp = split3(g.a[2 * st + (e >> 2)][e & 3]);
        h[e] = sp.h;
        m[e] = sp.m;
        l[e] = sp.l;
      }
      bf16x8 oa[3];
      oa[0] = __builtin_bit_cast(bf16x8, (u32x4){pack_hi16(h[0], h[1]), pack_hi16(h[2], h[3]),
                                                 pack_hi16(h[4], h[5]), pack_hi16(h[6], h[7])});
      oa[1] = __builtin_bit_cast(bf16x8, (u32x4){pack_hi16(m[0], m[1]), pack_hi16(m[2], m[3]),
                                                 pack_hi16(m[4], m[5]), pack_hi16(m[6], m[7])});
      oa[2] = __builtin_bit_cast(bf16x8, (u32x4){pack_hi16(l[0], l[1]), pack_hi16(l[2], l[3]),
                                                 pack_hi16(l[4], l[5]), pack_hi16(l[6], l[7])});
      // smallest terms first, as gemm_x3_kernel
#pragma unroll
      for (int t = 2; t >= 0; t--) {
#pragma unroll
        for (int j = 0; j < NB; j++)
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(oa[t], __builtin_bit_cast(bf16x8, g.b[NB * st + j]),
                                                           acc[j], 0, 0, 0);
      }
    }
  };
  if (s0 < s1) {
    Regs ra, rb;
    load(ra, s0);
    int kt = s0;
    // the next slab's loads are issued before the current slab's MFMAs
    for (; kt + 2 < s1; kt += 2) {
      load(rb, kt + 1);
      compute(ra);
      load(ra, kt + 2);
      compute(rb);
    }
    if (kt + 1 < s1) {
      load(rb, kt + 1);
      compute(ra);
      compute(rb);
    } else {
      compute(ra);
    }
  }
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int r = 0; r < 16; r++) red[wave][j][r][lane] = acc[j][r];
  __syncthreads();

  // C element (j, r, l): row 8*(r/4) + 4*(l/32) + r%4, column 32*j + l%32
  GemmParams q = p;
  if (p.ksplit > 1) q.c = p.c + blockIdx.y * p.c_split;
  if constexpr (EPI == Epi::GeGLU && NB == 1) {
    // gate in columns 0-15 (lanes l % 32 < 16), up 16 columns further
    const int64_t F = N / 2;
    for (int e = tid; e < 16 * 32; e += NW * 64) {
      const int r = e >> 5, lq = e & 31;
      const int l = (lq & 15) | ((lq & 16) << 1);
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int w = 0; w < NW; w++) {
        g += red[w][0][r][l];
        u += red[w][0][r][l + 16];
      }
      const int64_t row = m0 + (r >> 2) * 8 + (l >> 5) * 4 + (r & 3);
      const int64_t fcol = n0 / 2 + (l & 15);
      if (row < M && fcol < F) p.c[row * p.ldc + fcol] = gelu_tanh_ref(g) * u;
    }
    return;
  }
  if constexpr (EPI == Epi::GeGLU && NB == 2) {
    if (p.ksplit == 1) {
      // gate block 0 and up block 1 hold the same 32 features
      const int64_t F = N / 2;
      for (int e = tid; e < 16 * 64; e += NW * 64) {
        const int r = e >> 6, l = e & 63;
        float g = 0.f, u = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
          g += red[w][0][r][l];
          u += red[w][NB - 1][r][l];
        }
        const int64_t row = m0 + (r >> 2) * 8 + (l >> 5) * 4 + (r & 3);
        const int64_t fcol = n0 / 2 + (l & 31);
        if (row < M && fcol < F) p.c[row * p.ldc + fcol] = gelu_tanh_ref(g) * u;
      }
      return;
    }
  }
  for (int e = tid; e < NB * 16 * 64; e += NW * 64) {
    const int j = e >> 10, r = (e >> 6) & 15, l = e & 63;
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < NW; w++) v += red[w][j][r][l];
    const int64_t row = m0 + (r >> 2) * 8 + (l >> 5) * 4 + (r & 3);
    const int64_t col = n0 + 32 * j + (l & 31);
    if (row < M && col < N)
      q.c[row * q.ldc + col] = (EPI == Epi::Generic && p.ksplit == 1) ? epi_value<Epi::Generic>(q, v, row, col) : v;
  }
}

// Narrow GeGLU tiles (16 features) while they fit one per CU
// (FA_SMALL_NARROW=0 turns them off): gate|up at 64 rows (144 narrow
// tiles), 11.4 -> 9.7 us per launch, 1.17 -> 1.12 ms per forward on
// MI355X; at 128 rows (288 narrow tiles, a second round on some CUs)
// 11.3 -> 13.6 us, so the 32 x 64 tiles stay there.
static bool small_narrow(const GemmParams& p, int cus) {
  static const bool on = [] {
    const char* e = std::getenv("FA_SMALL_NARROW");
    return !(e && e[0] == '0');
  }();
  return on && p.ksplit == 1 && p.n % 64 == 0 && ((p.m + 31) / 32) * (p.n / 32) <= cus;
}

template <Epi EPI>
void launch_x3_small(GemmParams p, hipStream_t s, int cus = 256) {
  p.tiles_m = (int)((p.m + 31) / 32);
  p.nk = (int)(p.k / 32);
  if (p.ksplit < 1) p.ksplit = 1;
  if constexpr (EPI == Epi::GeGLU) {
    if (small_narrow(p, cus)) {
      p.tiles_n = (int)(p.n / 32);
      dim3 grid(p.tiles_m * p.tiles_n, 1), block(kSmallNW * 64);
      hipLaunchKernelGGL((gemm_x3_small_kernel<kSmallNW, EPI, 1>), grid, block, 0, s, p);
      return;
    }
  }
  p.tiles_n = (int)((p.n + 63) / 64);
  dim3 grid(p.tiles_m * p.tiles_n, p.ksplit), block(kSmallNW * 64);
  hipLaunchKernelGGL((gemm_x3_small_kernel<kSmallNW, EPI>), grid, block, 0, s, p);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

enum class TileId { k128x128 = 0, k64x64, k128x64v, kCount };
const char* const kTileNames[] = {"128x128", "64x64", "128x64v"};

// FA_GEMM_TILE=<name> forces a tile shape on the fast path (tuning).
int forced_tile() {
  static int v = [] {
    const char* e = std::getenv("FA_GEMM_TILE");
    if (!e) return -1;
    for (int i = 0; i < (int)TileId::kCount; i++)
      if (std::strcmp(e, kTileNames[i]) == 0) return i;
    return -1;
  }();
  return v;
}

// Tile choice, from measurements on MI355X (M in 128..32768, N in
// 768..3072, K in 768..3072): while the 128x128 tiles would give fewer than
// six per CU, smaller tiles win (more resident workgroups per CU and a finer
// split over the CUs; 1.5x on the N=768 products at M=5517, 3x at M=128);
// beyond that the 128x128 tile's operand reuse wins. GeGLU needs an even
// number of 32-column blocks per wave: 128x64 with four waves stacked in M.
TileId pick_tile(int64_t m, int64_t n, Epi epi, int cus) {
  const int64_t tiles128 = ((m + 127) / 128) * ((n + 127) / 128);
  if (tiles128 >= 6LL * cus) return TileId::k128x128;
  return epi == Epi::GeGLU ? TileId::k128x64v : TileId::k64x64;
}

template <class TL, bool BBF16>
void dispatch_fast(const GemmParams& p, Epi epi, hipStream_t s) {
  switch (epi) {
    case Epi::None: launch_dp<TL, BBF16, true, true, Epi::None>(p, s); break;
    case Epi::Generic: launch_dp<TL, BBF16, true, true, Epi::Generic>(p, s); break;
    case Epi::GeGLU:
      if constexpr (TL::FN % 2 == 0) launch_dp<TL, BBF16, true, true, Epi::GeGLU>(p, s);
      break;
  }
}

template <bool BBF16>
void dispatch_tile(TileId t, const GemmParams& p, Epi epi, hipStream_t s) {
  switch (t) {
    case TileId::k64x64: dispatch_fast<T64x64, BBF16>(p, epi, s); break;
    case TileId::k128x64v: dispatch_fast<T128x64v, BBF16>(p, epi, s); break;
    default: dispatch_fast<T128x128, BBF16>(p, epi, s); break;
  }
}

enum class XTileId { x128x64v = 0, x64x128, x64x64, x128x128w8, x128x256w8, small, kCount };
const char* const kXTileNames[] = {"128x64v", "64x128", "64x64", "128x128w8", "128x256w8", "small"};

// FA_GEMM_XTILE=<name> forces a split-bf16 tile shape; FA_GEMM_MFMA=f32 runs
// bf16 weights through the fp32 MFMA kernel instead (tuning, comparison).
int forced_xtile() {
  static int v = [] {
    const char* e = std::getenv("FA_GEMM_XTILE");
    if (!e) return -1;
    for (int i = 0; i < (int)XTileId::kCount; i++)
      if (std::strcmp(e, kXTileNames[i]) == 0) return i;
    return -1;
  }();
  return v;
}

bool use_f32_mfma() {
  static bool v = [] {
    const char* e = std::getenv("FA_GEMM_MFMA");
    return e && std::strcmp(e, "f32") == 0;
  }();
  return v;
}

// Split-bf16 tile choice, from measurements on MI355X (M 5517 and 32768,
// N 768..2304, K 768 and 1152): the 128x128 tile of eight 32x64 waves (two
// workgroups per CU) is the fastest or within 4 % of the fastest at every
// measured shape once it gives the CUs half a tile each, except where its
// tiles (K-split parts included) fill just over one round of the CUs' two
// slots: there the 64x128 tile of four 32x64 waves (four workgroups per CU)
// halves the last round (the encoder's o and down products at 5 517 rows:
// 0.79 -> 0.76 and 1.06 -> 1.01 ms per forward). Below half a tile per CU,
// 64x64 tiles (128x64 for GeGLU, which needs column-block pairs) spread the
// work. From 1.5 128x256 tiles per CU on, and with at least 24 K slabs per
// tile, the 128x256 tile of eight 32x128 waves wins: it splits each A
// element for twice the columns (gate|up at 5 517 x 2304 x 768: 75 vs 81 us;
// 32 768 rows: 6-7 % faster), while below that its fewer tiles leave CUs
// idle (qkv at 1 840 rows: 31 vs 21 us) and with 16 slabs its longer
// prologue and epilogue lose (EmbeddingGemma 2's K = 512 products at 5 517
// rows: 84 vs 79 us for gate|up).
//
// Few rows: while its 32x64 tiles (K parts included) fit one per CU, the
// small-M kernel (eight waves splitting each tile's K) wins on latency: at
// 128 rows and K = 768, 8.4-8.8 vs 10.8-11.2 us per launch for N = 768,
// 1280, 2304; one pooled row against K = 3072, 15.9 vs 33.7 us; 512 x 768
// x 1152, 12.3 vs 15.2 us. With more tiles it loses (256 x 2304 x 768: 14.7
// vs 11.2 us): every tile re-splits its A rows and re-reads its B columns.
//
// A launch that shares the GPU with other streams' kernels (shared) takes
// the 128x256 tile from 0.75 tiles per CU on: the other streams fill the
// CUs it leaves idle, and it splits each A element half as often (per
// forward: C5's micro-batch qkv products at about 6 000 rows, 13.36 ->
// 13.17 ms; C4's gate|up at about 2 900 rows, 11.49 -> 11.37 ms; C3's o
// and down products unchanged); at 0.3-0.5 tiles per CU (C2's
// micro-batches, 1 840 rows) its longer per-tile chain loses (qkv: 5.10 ->
// 5.40 ms, gate|up 5.10 -> 5.15). Below half a 128x128 tile per CU a
// shared launch takes 64x128 tiles rather than 64x64: EmbeddingGemma 2's
// micro-batch products of N = 512 (K split in two), 4.28 -> 4.15 ms per
// forward on one box, 4.19 -> 4.17 on another.
XTileId pick_xtile(int64_t m, int64_t n, int64_t k, int ksplit, Epi epi, int cus, bool shared) {
  if (((m + 31) / 32) * ((n + 63) / 64) * ksplit <= cus) return XTileId::small;
  const int64_t tiles256 = ((m + 127) / 128) * ((n + 255) / 256) * ksplit;
  const int64_t need = shared ? 3LL * cus : 6LL * cus;  // 4 x (0.75 or 1.5 tiles per CU)
  if (4 * tiles256 >= need && k / (32LL * ksplit) >= 24) return XTileId::x128x256w8;
  const int64_t tiles128 = ((m + 127) / 128) * ((n + 127) / 128) * ksplit;
  if (2 * tiles128 < cus) return epi == Epi::GeGLU ? XTileId::x128x64v : shared ? XTileId::x64x128 : XTileId::x64x64;
  if (tiles128 > 2 * cus && 4 * tiles128 <= 5 * 2 * cus) return XTileId::x64x128;
  return XTileId::x128x128w8;
}

template <class TL>
void dispatch_x3_epi(const GemmParams& p, Epi epi, hipStream_t s) {
  switch (epi) {
    case Epi::None: launch_x3<TL, Epi::None>(p, s); break;
    case Epi::Generic: launch_x3<TL, Epi::Generic>(p, s); break;
    case Epi::GeGLU:
      if constexpr (TL::FN % 2 == 0) launch_x3<TL, Epi::GeGLU>(p, s);
      break;
  }
}

void dispatch_x3(XTileId t, const GemmParams& p, Epi epi, hipStream_t s, int cus = 256) {
  switch (t) {
    case XTileId::small:
      switch (epi) {
        case Epi::None: launch_x3_small<Epi::None>(p, s, cus); break;
        case Epi::Generic: launch_x3_small<Epi::Generic>(p, s, cus); break;
        case Epi::GeGLU: launch_x3_small<Epi::GeGLU>(p, s, cus); break;
      }
      break;
    case XTileId::x128x64v: dispatch_x3_epi<X128x64v>(p, epi, s); break;
    case XTileId::x64x128: dispatch_x3_epi<X64x128>(p, epi, s); break;
    case XTileId::x64x64: dispatch_x3_epi<X64x64>(p, epi, s); break;
    case XTileId::x128x256w8: dispatch_x3_epi<X128x256w8>(p, epi, s); break;
    default: dispatch_x3_epi<X128x128w8>(p, epi, s); break;
  }
}

// B as three bf16 planes (BT = 3): 128x128 tiles of eight 32x64 waves (96 KB
// of LDS: one workgroup per CU) once they give every CU half a tile, else
// 64x64 tiles (128x64 for GeGLU) of four waves.
void dispatch_x3_bt3(const GemmParams& p, Epi epi, int cus, hipStream_t s) {
  const int64_t tiles128 =
      ((p.m + 127) / 128) * ((p.n + 127) / 128) * std::max(p.ksplit, 1) * std::max(p.nbatch, 1);
  const bool big = 2 * tiles128 >= cus;
  switch (epi) {
    case Epi::None:
      if (big) launch_x3<X128x128w8, Epi::None, 3>(p, s); else launch_x3<X64x64, Epi::None, 3>(p, s);
      break;
    case Epi::Generic:
      if (big) launch_x3<X128x128w8, Epi::Generic, 3>(p, s); else launch_x3<X64x64, Epi::Generic, 3>(p, s);
      break;
    case Epi::GeGLU:
      if (big) launch_x3<X128x128w8, Epi::GeGLU, 3>(p, s); else launch_x3<X128x64v, Epi::GeGLU, 3>(p, s);
      break;
  }
}

// fp32 B [k x n] (FA_B_KN, rows of n) or [n x k] (FA_B_NK) -> three bf16
// planes [3][n][k] (hi, mid, lo: split3). One thread per (column, 8 k
// values); consecutive threads take consecutive columns of one 8-row band
// (KN: coalesced reads of each k row) or consecutive chunks of one column
// (NK: contiguous reads and writes).
// A bf16 source (bf16 != 0) is transposed only: one plane, its values as they are.
__global__ __launch_bounds__(256) void split_b_kernel(const void* __restrict__ bsrc, int64_t ldb, int kn, int bf16,
                                                      int64_t n, int64_t k, uint16_t* __restrict__ planes) {
  const float* b = static_cast<const float*>(bsrc);
  const uint16_t* b16 = static_cast<const uint16_t*>(bsrc);
  const int64_t kc_n = k / 8;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (gid >= n * kc_n) return;
  int64_t col, kc;
  if (kn) {
    kc = gid / n;
    col = gid - kc * n;
  } else {
    col = gid / kc_n;
    kc = gid - col * kc_n;
  }
  uint32_t h[8], m[8], l[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const int64_t at = kn ? (kc * 8 + e) * ldb + col : col * ldb + kc * 8 + e;
    const float x = bf16 ? __uint_as_float((uint32_t)b16[at] << 16) : b[at];
    const Split3 sp = split3(x);
    h[e] = sp.h;
    m[e] = sp.m;
    l[e] = sp.l;
  }
  const int64_t o = col * k + kc * 8, plane = n * k;
  if (bf16) {
    *reinterpret_cast<uint4*>(planes + o) =
        make_uint4(pack_hi16(h[0], h[1]), pack_hi16(h[2], h[3]), pack_hi16(h[4], h[5]), pack_hi16(h[6], h[7]));
    return;
  }
  *reinterpret_cast<uint4*>(planes + o) =
      make_uint4(pack_hi16(h[0], h[1]), pack_hi16(h[2], h[3]), pack_hi16(h[4], h[5]), pack_hi16(h[6], h[7]));
  *reinterpret_cast<uint4*>(planes + plane + o) =
      make_uint4(pack_hi16(m[0], m[1]), pack_hi16(m[2], m[3]), pack_hi16(m[4], m[5]), pack_hi16(m[6], m[7]));
  *reinterpret_cast<uint4*>(planes + 2 * plane + o) =
      make_uint4(pack_hi16(l[0], l[1]), pack_hi16(l[2], l[3]), pack_hi16(l[4], l[5]), pack_hi16(l[6], l[7]));
}

bool x3_has_geglu(XTileId t) { return t != XTileId::x64x64; }

// ---- strided and batched operands (tensor.MatMul's views) ---------------------
// Element offset of batch entry z (row-major over the batch dimensions) in a
// strided operand; 32-bit index arithmetic (entries < 2^31).
__device__ __forceinline__ int64_t batch_offset(const BatchMap& bm, int z) {
  int64_t off = 0;
  for (int d = bm.nd - 1; d >= 0; d--) {
    const int q = z / bm.dim[d];
    off += (int64_t)(z - q * bm.dim[d]) * bm.stride[d];
    z = q;
  }
  return off;
}

// A view [nb][m][k] with element (z, i, p) at src[off(z) + i*rs + p*cs] ->
// contiguous [nb][m][kp], columns k..kp-1 zero. One thread per 4 columns.
__global__ __launch_bounds__(256) void pack_a_kernel(const float* __restrict__ src, BatchMap bm, int z0, int64_t rs,
                                                     int64_t cs, int64_t m, int64_t k, int64_t kp, int64_t total,
                                                     float* __restrict__ dst) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= total) return;
  const int64_t kq = kp / 4;
  const int64_t row = t / kq;  // z * m + i
  const int64_t p0 = (t - row * kq) * 4;
  const int z = (int)(row / m);
  const float* s = src + batch_offset(bm, z0 + z) + (row - (int64_t)z * m) * rs;
  f32x4 v;
#pragma unroll
  for (int e = 0; e < 4; e++) v[e] = p0 + e < k ? s[(p0 + e) * cs] : 0.f;
  *reinterpret_cast<f32x4*>(dst + row * kp + p0) = v;
}

// B view, logical [k x n] per entry with element (z, p, j) at src[off(z) +
// p*rs + j*cs] -> three bf16 planes hi, mid, lo of [n][kp] per entry
// (planes + (3 z + term) * n * kp), columns k..kp-1 zero. One thread per
// (entry, column, 8 k values); consecutive threads take consecutive 8-value
// chunks of one column when p is the unit-stride index (k_major), else
// consecutive columns of one chunk.
__global__ __launch_bounds__(256) void split_b_view_kernel(const float* __restrict__ src, BatchMap bm, int z0, int64_t rs,
                                                           int64_t cs, int64_t n, int64_t k, int64_t kp, int k_major,
                                                           int64_t total, uint16_t* __restrict__ planes) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= total) return;
  const int64_t kc_n = kp / 8, per = n * kc_n;
  const int z = (int)(t / per);
  const int64_t r = t - (int64_t)z * per;
  int64_t col, kc;
  if (k_major) {
    col = r / kc_n;
    kc = r - col * kc_n;
  } else {
    kc = r / n;
    col = r - kc * n;
  }
  const float* s = src + batch_offset(bm, z0 + z) + col * cs;
  uint32_t h[8], md[8], l[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const int64_t p = kc * 8 + e;
    const Split3 sp = split3(p < k ? s[p * rs] : 0.f);
    h[e] = sp.h;
    md[e] = sp.m;
    l[e] = sp.l;
  }
  const int64_t plane = n * kp;
  uint16_t* o = planes + (int64_t)z * 3 * plane + col * kp + kc * 8;
  *reinterpret_cast<uint4*>(o) =
      make_uint4(pack_hi16(h[0], h[1]), pack_hi16(h[2], h[3]), pack_hi16(h[4], h[5]), pack_hi16(h[6], h[7]));
  *reinterpret_cast<uint4*>(o + plane) =
      make_uint4(pack_hi16(md[0], md[1]), pack_hi16(md[2], md[3]), pack_hi16(md[4], md[5]), pack_hi16(md[6], md[7]));
  *reinterpret_cast<uint4*>(o + 2 * plane) =
      make_uint4(pack_hi16(l[0], l[1]), pack_hi16(l[2], l[3]), pack_hi16(l[4], l[5]), pack_hi16(l[6], l[7]));
}

}  // namespace

int launch_pack_a(fa_ctx* ctx, const float* src, const BatchMap& bm, int z0, int64_t rs, int64_t cs, int64_t nb,
                  int64_t m, int64_t k, int64_t kp, float* dst, hipStream_t s) {
  if (kp % 4 != 0 || kp < k) return set_error(ctx, FA_ERR_ARG, "MatMul: packed width %lld", (long long)kp);
  const int64_t total = nb * m * (kp / 4);
  if (total == 0) return FA_OK;
  hipLaunchKernelGGL(pack_a_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src, bm, z0, rs, cs, m,
                     k, kp, total, dst);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_split_b_view(fa_ctx* ctx, const float* src, const BatchMap& bm, int z0, int64_t rs, int64_t cs,
                        int64_t nb, int64_t n, int64_t k, int64_t kp, uint16_t* planes, hipStream_t s) {
  if (kp % 8 != 0 || kp < k) return set_error(ctx, FA_ERR_ARG, "MatMul: packed width %lld", (long long)kp);
  const int64_t total = nb * n * (kp / 8);
  if (total == 0) return FA_OK;
  const int k_major = (rs == 1 && cs != 1) ? 1 : 0;
  hipLaunchKernelGGL(split_b_view_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, src, bm, z0, rs, cs,
                     n, k, kp, k_major, total, planes);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

bool gemm_f32_mfma_forced() { return use_f32_mfma(); }

int gemm_ksplit() {
  static const int v = [] {
    if (use_f32_mfma()) return 1;  // the fp32-MFMA kernel computes whole K ranges only
    const char* e = std::getenv("FA_GEMM_KSPLIT");
    return (e && std::strcmp(e, "1") == 0) ? 1 : 2;
  }();
  return v;
}

int launch_split_b(fa_ctx* ctx, const void* b, int b_dtype, int64_t ldb, int layout, int64_t n, int64_t k,
                   uint16_t* planes, hipStream_t s) {
  if (n <= 0 || k <= 0) return FA_OK;
  if (k % 8 != 0) return set_error(ctx, FA_ERR_ARG, "MatMul: split of B needs k %% 8 == 0, got %lld", (long long)k);
  const int64_t threads = n * (k / 8);
  hipLaunchKernelGGL(split_b_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, b, ldb,
                     layout == FA_B_KN ? 1 : 0, b_dtype == FA_DT_BF16 ? 1 : 0, n, k, planes);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int launch_gemm(fa_ctx* ctx, const GemmArgs& g, hipStream_t s) {
  if (g.m < 0 || g.n < 0 || g.k < 0)
    return set_error(ctx, FA_ERR_ARG, "MatMul: negative size m=%lld n=%lld k=%lld", (long long)g.m,
                     (long long)g.n, (long long)g.k);
  if (g.m == 0 || g.n == 0) return FA_OK;
  if (g.epi == Epi::GeGLU && (g.n % 64 != 0))
    return set_error(ctx, FA_ERR_ARG, "GeGLU product needs n (2F) divisible by 64, got %lld", (long long)g.n);
  // the epilogue addresses a 32-row block with 32-bit offsets
  if (g.ldc >= (1LL << 26))
    return set_error(ctx, FA_ERR_ARG, "MatMul: ldc %lld above 2^26 elements", (long long)g.ldc);
  GemmParams p;
  std::memset(&p, 0, sizeof p);
  p.m = g.m; p.n = g.n; p.k = g.k;
  p.a = g.a; p.lda = g.lda; p.b = g.b; p.ldb = g.ldb; p.c = g.c; p.ldc = g.ldc;
  p.bias = g.bias; p.row_scale = g.row_scale; p.mul = g.mul; p.ldm = g.ldm;
  p.residual = g.residual; p.ldr = g.ldr; p.act = g.act;
  p.ksplit = 1;
  p.b_plane = g.b_plane;
  p.nbatch = 1;
  if (g.b_terms != 1 && g.b_terms != 3) return set_error(ctx, FA_ERR_ARG, "MatMul: %d B planes", g.b_terms);
  if (g.nbatch > 1) {
    // batch entries on grid.z: the three-plane kernel only, one K range
    if (g.b_terms != 3 || g.ksplit > 1 || g.nbatch > kMaxGridZ)
      return set_error(ctx, FA_ERR_ARG, "MatMul: a batch of %lld needs three B planes, no K split and <= %d entries",
                       (long long)g.nbatch, kMaxGridZ);
    p.nbatch = (int)g.nbatch;
    p.a_bs = g.a_bs;
    p.b_bs = g.b_bs;
    p.c_bs = g.c_bs;
  }
  if (((g.m + 63) / 64) * ((g.n + 63) / 64) > INT32_MAX / 4) return set_error(ctx, FA_ERR_ARG, "MatMul: too many tiles");
  const bool bf16 = g.b_dtype == FA_DT_BF16;
  const bool nk = g.b_layout == FA_B_NK;
  if (g.ksplit > 1) {
    // K split into equal ranges of whole slabs, partial products to c + s*c_split
    if (!(bf16 && nk && g.epi == Epi::None && g.k % (32 * g.ksplit) == 0 && g.c_split >= g.m * g.ldc &&
          !use_f32_mfma()))
      return set_error(ctx, FA_ERR_ARG, "MatMul: K split needs bf16 [n x k] weights, no epilogue, k %% (32*%d) == 0 "
                       "and disjoint partial outputs", g.ksplit);
    p.ksplit = g.ksplit;
    p.c_split = g.c_split;
  }
  // The fast loaders read 16-byte vectors: every row start must be 16-byte
  // aligned and k a whole number of 32-wide slabs.
  const bool fast = nk && g.k > 0 && g.k % 32 == 0 && aligned16(g.a) && aligned16(g.b) && g.lda % 4 == 0 &&
                    (bf16 ? g.ldb % 8 == 0 : g.ldb % 4 == 0);
  if (p.ksplit > 1 && !fast) return set_error(ctx, FA_ERR_ARG, "MatMul: K split needs 16-byte aligned rows");
  if (g.b_terms == 3) {
    if (!(fast && bf16))
      return set_error(ctx, FA_ERR_ARG, "MatMul: three B planes need bf16 [n x k] planes, k %% 32 == 0 and 16-byte "
                       "aligned rows");
    dispatch_x3_bt3(p, g.epi, ctx->cu_count > 0 ? ctx->cu_count : 256, s);
  } else if (fast && bf16 && !use_f32_mfma()) {
    const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
    XTileId t = (XTileId)forced_xtile();
    if ((int)t < 0 || (g.epi == Epi::GeGLU && !x3_has_geglu(t))) t = pick_xtile(g.m, g.n, g.k, p.ksplit, g.epi, cus, g.shared);
    dispatch_x3(t, p, g.epi, s, cus);
  } else if (fast) {
    TileId t = (TileId)forced_tile();
    if ((int)t < 0 || (g.epi == Epi::GeGLU && t == TileId::k64x64))
      t = pick_tile(g.m, g.n, g.epi, ctx->cu_count > 0 ? ctx->cu_count : 256);
    if (bf16) dispatch_tile<true>(t, p, g.epi, s);
    else dispatch_tile<false>(t, p, g.epi, s);
  } else {
    using TC = T128x128;
#define FA_DISPATCH_EPI(BB, NK)                                                      \
  switch (g.epi) {                                                                   \
    case Epi::None: launch_dp<TC, BB, NK, false, Epi::None>(p, s); break;           \
    case Epi::Generic: launch_dp<TC, BB, NK, false, Epi::Generic>(p, s); break;     \
    case Epi::GeGLU: launch_dp<TC, BB, NK, false, Epi::GeGLU>(p, s); break;         \
  }
    if (bf16) {
      if (nk) { FA_DISPATCH_EPI(true, true) }
      else { FA_DISPATCH_EPI(true, false) }
    } else {
      if (nk) { FA_DISPATCH_EPI(false, true) }
      else { FA_DISPATCH_EPI(false, false) }
    }
#undef FA_DISPATCH_EPI
  }
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

}  // namespace fa
