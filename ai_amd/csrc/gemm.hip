// fp32-accumulate MFMA GEMM for gfx950: C = epilogue(A . B).
//
// A: fp32 [m x k] row-major. B: logical [k x n], stored bf16 or fp32, either
// as [n x k] rows (checkpoint [out,in] weights, docs) or [k x n] rows. The
// workgroup computes a 128x128 tile of C with four waves (2x2), each wave a
// 64x64 sub-tile as 2x2 blocks of v_mfma_f32_32x32x2_f32 (16 accumulators
// per lane per block). K advances in slabs of 32 through two LDS buffers:
// the next slab's global loads are issued before the current slab's MFMAs
// and written to the other buffer afterwards, so one barrier per slab
// suffices. bf16 weights are widened to fp32 (exact) when they are written
// to LDS, so the MFMA operands are always fp32.
//
// MFMA operand layout (32x32x2, one block): lane l supplies A[row l%32][k]
// and B[k][col l%32] with k = l/32; the 16 results of lane l are C[row][col]
// with col = l%32 and row = 8*(r/4) + 4*(l/32) + r%4 for r = 0..15. A
// product does not depend on the order of its k terms, so each lane reads
// four consecutive k values with one 16-byte LDS read: lanes 0-31 take
// k = 8s..8s+3 and lanes 32-63 take k = 8s+4..8s+7, and MFMA number c (0..3)
// pairs k = 8s+c with 8s+4+c on both operands.
//
// Epilogues: None; Generic (bias, row scale, activation, element-wise
// multiply, residual: the reference's order, internal/blas/gemm.go:276-347);
// GeGLU (the gate and up weights interleaved in 32-row groups, so each wave's
// two column blocks hold gate and up of the same 32 features and the lane
// writes gelu_tanh(gate) * up, models/gemma/embed.go:226-227).

#include "fa_internal.h"
#include "device_math.h"

namespace fa {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int LDSK = BK + 4;  // padded LDS row stride (floats): rows start 4 banks apart
constexpr int NTHREADS = 256;

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
};

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

template <bool BBF16, bool BNK, bool FAST, Epi EPI>
__global__ __launch_bounds__(NTHREADS) void gemm_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) float As[2][BM * LDSK];
  __shared__ __attribute__((aligned(16))) float Bs[2][BN * LDSK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  const int total = p.tiles_m * p.tiles_n;
  int tile = blockIdx.x;
  {
    // XCD-aware: give each XCD a contiguous run of tiles (row-major over n).
    constexpr int kXcd = 8;
    int per = total / kXcd;
    if (per > 0 && tile < per * kXcd) tile = (tile % kXcd) * per + tile / kXcd;
  }
  const int tm = tile / p.tiles_n, tn = tile % p.tiles_n;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t M = p.m, N = p.n, K = p.k;
  const float* __restrict__ A = p.a;

  // ---- global -> register staging ----
  f32x4 ra[4];
  uint32_t rbh[2][4];  // bf16 pairs (FAST bf16 path)
  f32x4 rbf[4];        // fp32 B (FAST f32 path)
  float rs_a[16], rs_b[16];  // checked path

  auto load_global = [&](int64_t k0) {
    if constexpr (FAST) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        int row = (tid >> 3) + 32 * i, col = (tid & 7) * 4;
        int64_t gr = min(m0 + row, M - 1);
        ra[i] = *reinterpret_cast<const f32x4*>(A + gr * p.lda + k0 + col);
      }
      if constexpr (BBF16) {
        const uint16_t* B = static_cast<const uint16_t*>(p.b);
#pragma unroll
        for (int i = 0; i < 2; i++) {
          int row = (tid >> 2) + 64 * i, col = (tid & 3) * 8;
          int64_t gn = min(n0 + row, N - 1);
          uint4 v = *reinterpret_cast<const uint4*>(B + gn * p.ldb + k0 + col);
          rbh[i][0] = v.x; rbh[i][1] = v.y; rbh[i][2] = v.z; rbh[i][3] = v.w;
        }
      } else {
        const float* B = static_cast<const float*>(p.b);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          int row = (tid >> 3) + 32 * i, col = (tid & 7) * 4;
          int64_t gn = min(n0 + row, N - 1);
          rbf[i] = *reinterpret_cast<const f32x4*>(B + gn * p.ldb + k0 + col);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        int idx = tid + NTHREADS * i;
        int row = idx >> 5, col = idx & 31;
        int64_t gr = m0 + row, gk = k0 + col;
        rs_a[i] = (gr < M && gk < K) ? A[gr * p.lda + gk] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < 16; i++) {
        int idx = tid + NTHREADS * i;
        int nn, kk;
        if constexpr (BNK) {
          nn = idx >> 5; kk = idx & 31;
        } else {
          nn = idx & 127; kk = idx >> 7;
        }
        int64_t gn = n0 + nn, gk = k0 + kk;
        float v = 0.f;
        if (gn < N && gk < K) {
          int64_t off = BNK ? gn * p.ldb + gk : gk * p.ldb + gn;
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
      for (int i = 0; i < 4; i++) {
        int row = (tid >> 3) + 32 * i, col = (tid & 7) * 4;
        *reinterpret_cast<f32x4*>(&As[buf][row * LDSK + col]) = ra[i];
      }
      if constexpr (BBF16) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
          int row = (tid >> 2) + 64 * i, col = (tid & 3) * 8;
          f32x4 lo, hi;
          lo.x = __uint_as_float(rbh[i][0] << 16); lo.y = __uint_as_float(rbh[i][0] & 0xFFFF0000u);
          lo.z = __uint_as_float(rbh[i][1] << 16); lo.w = __uint_as_float(rbh[i][1] & 0xFFFF0000u);
          hi.x = __uint_as_float(rbh[i][2] << 16); hi.y = __uint_as_float(rbh[i][2] & 0xFFFF0000u);
          hi.z = __uint_as_float(rbh[i][3] << 16); hi.w = __uint_as_float(rbh[i][3] & 0xFFFF0000u);
          *reinterpret_cast<f32x4*>(&Bs[buf][row * LDSK + col]) = lo;
          *reinterpret_cast<f32x4*>(&Bs[buf][row * LDSK + col + 4]) = hi;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          int row = (tid >> 3) + 32 * i, col = (tid & 7) * 4;
          *reinterpret_cast<f32x4*>(&Bs[buf][row * LDSK + col]) = rbf[i];
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; i++) {
        int idx = tid + NTHREADS * i;
        As[buf][(idx >> 5) * LDSK + (idx & 31)] = rs_a[i];
      }
#pragma unroll
      for (int i = 0; i < 16; i++) {
        int idx = tid + NTHREADS * i;
        int nn, kk;
        if constexpr (BNK) {
          nn = idx >> 5; kk = idx & 31;
        } else {
          nn = idx & 127; kk = idx >> 7;
        }
        Bs[buf][nn * LDSK + kk] = rs_b[i];
      }
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  const int nk = (int)((K + BK - 1) / BK);
  load_global(0);
  store_lds(0);
  __syncthreads();

  const int arow = wm * 64 + (lane & 31);
  const int brow = wn * 64 + (lane & 31);
  const int kofs = (lane >> 5) * 4;

  for (int kt = 0; kt < nk; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_global((int64_t)(kt + 1) * BK);
    const float* as = As[buf];
    const float* bs = Bs[buf];
#pragma unroll
    for (int s = 0; s < BK / 8; s++) {
      f32x4 a0 = *reinterpret_cast<const f32x4*>(&as[arow * LDSK + s * 8 + kofs]);
      f32x4 a1 = *reinterpret_cast<const f32x4*>(&as[(arow + 32) * LDSK + s * 8 + kofs]);
      f32x4 b0 = *reinterpret_cast<const f32x4*>(&bs[brow * LDSK + s * 8 + kofs]);
      f32x4 b1 = *reinterpret_cast<const f32x4*>(&bs[(brow + 32) * LDSK + s * 8 + kofs]);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[c], b0[c], acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[c], b1[c], acc[0][1], 0, 0, 0);
        acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[c], b0[c], acc[1][0], 0, 0, 0);
        acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[c], b1[c], acc[1][1], 0, 0, 0);
      }
    }
    if (kt + 1 < nk) store_lds(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue ----
  const int lcol = lane & 31;
  const int lrow4 = (lane >> 5) * 4;
  if constexpr (EPI == Epi::GeGLU) {
    // wave's block 0 = gate features, block 1 = up features (same 32 features)
    const int64_t fcol = n0 / 2 + wn * 32 + lcol;
    const int64_t F = N / 2;
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        int64_t row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + lrow4 + (r & 3);
        if (row < M && fcol < F) {
          float g = acc[i][0][r], u = acc[i][1][r];
          p.c[row * p.ldc + fcol] = gelu_tanh_ref(g) * u;
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int64_t col = n0 + wn * 64 + j * 32 + lcol;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          int64_t row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + lrow4 + (r & 3);
          if (row < M && col < N) {
            float v = acc[i][j][r];
            if constexpr (EPI == Epi::Generic) {
              if (p.bias) v = v + p.bias[col];
              if (p.row_scale) v = v * p.row_scale[row];
              if (p.act == FA_ACT_RELU) v = fmaxf(v, 0.f);
              else if (p.act == FA_ACT_GELU) v = gelu_tanh_ref(v);
              if (p.mul) v = v * p.mul[row * p.ldm + col];
              if (p.residual) v = v + p.residual[row * p.ldr + col];
            }
            p.c[row * p.ldc + col] = v;
          }
        }
      }
    }
  }
}

template <bool BBF16, bool BNK, bool FAST, Epi EPI>
void launch_t(const GemmParams& p, hipStream_t s) {
  dim3 grid(p.tiles_m * p.tiles_n), block(NTHREADS);
  hipLaunchKernelGGL((gemm_kernel<BBF16, BNK, FAST, EPI>), grid, block, 0, s, p);
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

int launch_gemm(fa_ctx* ctx, const GemmArgs& g, hipStream_t s) {
  if (g.m < 0 || g.n < 0 || g.k < 0)
    return set_error(ctx, FA_ERR_ARG, "MatMul: negative size m=%lld n=%lld k=%lld", (long long)g.m,
                     (long long)g.n, (long long)g.k);
  if (g.m == 0 || g.n == 0) return FA_OK;
  if (g.epi == Epi::GeGLU && (g.n % 64 != 0))
    return set_error(ctx, FA_ERR_ARG, "GeGLU product needs n (2F) divisible by 64, got %lld", (long long)g.n);
  GemmParams p;
  p.m = g.m; p.n = g.n; p.k = g.k;
  p.a = g.a; p.lda = g.lda; p.b = g.b; p.ldb = g.ldb; p.c = g.c; p.ldc = g.ldc;
  p.bias = g.bias; p.row_scale = g.row_scale; p.mul = g.mul; p.ldm = g.ldm;
  p.residual = g.residual; p.ldr = g.ldr; p.act = g.act;
  int64_t tm = (g.m + BM - 1) / BM, tn = (g.n + BN - 1) / BN;
  if (tm * tn > INT32_MAX) return set_error(ctx, FA_ERR_ARG, "MatMul: too many tiles");
  p.tiles_m = (int)tm; p.tiles_n = (int)tn;
  const bool bf16 = g.b_dtype == FA_DT_BF16;
  const bool nk = g.b_layout == FA_B_NK;
  // The fast loaders read 16-byte vectors: every row start must be 16-byte
  // aligned and k a whole number of slabs.
  const bool fast = nk && g.k > 0 && g.k % BK == 0 && aligned16(g.a) && aligned16(g.b) && g.lda % 4 == 0 &&
                    (bf16 ? g.ldb % 8 == 0 : g.ldb % 4 == 0);
  if (g.k == 0) {
    // empty inner dimension: the product is zero; the epilogue still applies
  }
#define FA_DISPATCH_EPI(BB, NK, FT)                                            \
  switch (g.epi) {                                                           \
    case Epi::None: launch_t<BB, NK, FT, Epi::None>(p, s); break;            \
    case Epi::Generic: launch_t<BB, NK, FT, Epi::Generic>(p, s); break;      \
    case Epi::GeGLU: launch_t<BB, NK, FT, Epi::GeGLU>(p, s); break;          \
  }
  if (fast) {
    if (bf16) { FA_DISPATCH_EPI(true, true, true) }
    else { FA_DISPATCH_EPI(false, true, true) }
  } else {
    if (bf16) {
      if (nk) { FA_DISPATCH_EPI(true, true, false) }
      else { FA_DISPATCH_EPI(true, false, false) }
    } else {
      if (nk) { FA_DISPATCH_EPI(false, true, false) }
      else { FA_DISPATCH_EPI(false, false, false) }
    }
  }
#undef FA_DISPATCH_EPI
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

}  // namespace fa
