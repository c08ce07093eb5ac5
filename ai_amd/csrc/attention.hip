// Bidirectional attention for gfx950.
//
// attention_varlen_kernel (the model path): packed variable-length
// sequences, grouped-query heads (every query head h reads key/value head
// h / (H/Hkv)), head_dim 256, optional sliding window |i-j| < window, padding
// implied by the packing (a sequence's keys are exactly its valid tokens).
// Computes softmax(scale * q.k^T) . v with an online softmax over key tiles,
// never materialising scores or masks. Masked keys get weight exactly 0, and
// so does any weight whose exponent is below -87 (the reference's flush,
// internal/kernel/generic.go:278-307), as in tensor.AttentionScaled
// (tensor/attention.go:67-83) + blas.AttentionBlock (internal/blas/
// attention.go:61-136) with PaddingMask + WindowMask (attention.go:33-42,
// 97-107; models/gemma/embed.go:168-186).
//
// MFMA formulation (v_mfma_f32_16x16x4_f32; lane l of a 16x16 result holds
// column l%16 and rows 4*(l/16)+r, r=0..3): each wave owns 16 queries of one
// head and computes the TRANSPOSED products
//     S^T[key, query] = K . Q^T        (A = K tile from LDS, B = Q in VGPRs)
//     O^T[d, query]  += V^T . P^T      (A = V^T tile from LDS, B = P in VGPRs)
// so that every lane's accumulators belong to a single query (column l%16):
// the probabilities computed from S^T are already in the B-operand layout of
// the second product, and the online-softmax rescale of O^T is a per-lane
// scalar. Within a 16-wide k step each lane group g = l/16 takes 4
// consecutive k values (one 16-byte LDS read); MFMA c (0..3) pairs them, which
// is a permutation of the k sum.
//
// attention_generic_kernel (the tensor.AttentionScaled drop-in): arbitrary
// B, H, T, S, D <= 512, strides and an additive mask tensor, one wavefront
// per query row, the reference's algebra: raw scores, + mask/scale, max,
// exp(scale*row - scale*max) with the flush, P.V, times 1/sum.

#include "fa_internal.h"
#include "device_math.h"

namespace fa {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int AD = 256;        // head_dim
constexpr int QW = 16;         // queries per wave
constexpr int NWAVE = 4;       // waves per workgroup
constexpr int QBLK = QW * NWAVE;
constexpr int KT = 32;         // keys per LDS tile
constexpr int KLD = AD + 4;    // padded K row stride (floats)
constexpr int VLD = KT + 4;    // padded V^T row stride (floats)
constexpr float kNegBig = -1e30f;

struct VarlenParams {
  const float* qkv;
  float* out;
  const int32_t* cu;
  const int32_t* items;  // pairs (seq, q0)
  int32_t H, Hkv;
  int32_t window;
  float scale;
};

__global__ __launch_bounds__(256, 2) void attention_varlen_kernel(VarlenParams p) {
  __shared__ __attribute__((aligned(16))) float Ks[KT * KLD];
  __shared__ __attribute__((aligned(16))) float Vt[AD * VLD];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int g = lane >> 4;   // lane group: k sub-range / result row group
  const int lq = lane & 15;  // the lane's query column

  const int seq = p.items[2 * blockIdx.x];
  const int q0 = p.items[2 * blockIdx.x + 1];
  const int h = blockIdx.y;
  const int hk = h / (p.H / p.Hkv);
  const int start = p.cu[seq];
  const int L = p.cu[seq + 1] - start;
  const int W = (p.H + 2 * p.Hkv) * AD;
  const float* qbase = p.qkv + (int64_t)start * W + (int64_t)h * AD;
  const float* kbase = p.qkv + (int64_t)start * W + (int64_t)(p.H + hk) * AD;
  const float* vbase = p.qkv + (int64_t)start * W + (int64_t)(p.H + p.Hkv + hk) * AD;

  const int qi = q0 + wave * QW + lq;  // this lane's query
  const bool qvalid = qi < L;

  // Q in VGPRs, B-operand layout: qreg[sg] = Q[qi][16*sg + 4*g .. +4]
  f32x4 qreg[AD / 16];
  {
    const float* qr = qbase + (int64_t)(qvalid ? qi : 0) * W;
#pragma unroll
    for (int sg = 0; sg < AD / 16; sg++) {
      f32x4 v = *reinterpret_cast<const f32x4*>(qr + sg * 16 + g * 4);
      qreg[sg] = qvalid ? v : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  f32x4 oacc[AD / 16];
#pragma unroll
  for (int db = 0; db < AD / 16; db++) oacc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegBig;  // running max of scaled scores of this lane's query
  float l_part = 0.f;     // this lane's share of the running sum

  // keys this workgroup needs
  const int qlast = min(q0 + QBLK, L) - 1;
  int kbeg = 0, kend = L;
  if (p.window > 0) {
    kbeg = max(0, q0 - p.window + 1);
    kend = min(L, qlast + p.window);
  }

  for (int k0 = kbeg; k0 < kend; k0 += KT) {
    __syncthreads();  // previous tile fully consumed
    // K tile: rows k0..k0+31 -> Ks[row][d]
#pragma unroll
    for (int i = 0; i < (KT * AD / 4) / 256; i++) {
      const int idx = tid + 256 * i;
      const int row = idx >> 6, c4 = idx & 63;
      f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
      if (k0 + row < kend) v = *reinterpret_cast<const f32x4*>(kbase + (int64_t)(k0 + row) * W + c4 * 4);
      *reinterpret_cast<f32x4*>(&Ks[row * KLD + c4 * 4]) = v;
    }
    // V tile transposed: Vt[d][key]
#pragma unroll
    for (int i = 0; i < (KT * AD / 4) / 256; i++) {
      const int idx = tid + 256 * i;
      const int row = idx & (KT - 1), c4 = idx / KT;
      f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
      if (k0 + row < kend) v = *reinterpret_cast<const f32x4*>(vbase + (int64_t)(k0 + row) * W + c4 * 4);
      Vt[(c4 * 4 + 0) * VLD + row] = v.x;
      Vt[(c4 * 4 + 1) * VLD + row] = v.y;
      Vt[(c4 * 4 + 2) * VLD + row] = v.z;
      Vt[(c4 * 4 + 3) * VLD + row] = v.w;
    }
    __syncthreads();

    // S^T for two 16-key sub-blocks
    f32x4 sacc[KT / 16];
#pragma unroll
    for (int kb = 0; kb < KT / 16; kb++) {
      sacc[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      const float* krow = &Ks[(kb * 16 + lq) * KLD + g * 4];
#pragma unroll
      for (int sg = 0; sg < AD / 16; sg++) {
        f32x4 a = *reinterpret_cast<const f32x4*>(krow + sg * 16);
#pragma unroll
        for (int c = 0; c < 4; c++)
          sacc[kb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c], qreg[sg][c], sacc[kb], 0, 0, 0);
      }
    }

    // mask, scale, tile max over this query's keys (spread over the 4 lane groups)
    float tmax = kNegBig;
    bool valid[KT / 16][4];
#pragma unroll
    for (int kb = 0; kb < KT / 16; kb++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int j = k0 + kb * 16 + g * 4 + r;
        bool ok = qvalid && j < kend;
        if (p.window > 0) ok = ok && (qi - j < p.window) && (j - qi < p.window);
        valid[kb][r] = ok;
        const float t = sacc[kb][r] * p.scale;
        sacc[kb][r] = t;
        if (ok) tmax = fmaxf(tmax, t);
      }
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = exp_flush(m_run - m_new);  // 0 when m_run is the sentinel
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int kb = 0; kb < KT / 16; kb++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const float pv = valid[kb][r] ? exp_flush(sacc[kb][r] - m_new) : 0.f;
        sacc[kb][r] = pv;
        psum += pv;
      }
    }
    l_part = l_part * alpha + psum;
#pragma unroll
    for (int db = 0; db < AD / 16; db++) oacc[db] *= alpha;

    // O^T += V^T . P^T
#pragma unroll
    for (int kb = 0; kb < KT / 16; kb++) {
#pragma unroll
      for (int db = 0; db < AD / 16; db++) {
        f32x4 a = *reinterpret_cast<const f32x4*>(&Vt[(db * 16 + lq) * VLD + kb * 16 + g * 4]);
#pragma unroll
        for (int c = 0; c < 4; c++)
          oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c], sacc[kb][c], oacc[db], 0, 0, 0);
      }
    }
  }

  float l_tot = l_part + __shfl_xor(l_part, 16, 64);
  l_tot += __shfl_xor(l_tot, 32, 64);
  if (!qvalid) return;
  const float inv = 1.f / l_tot;
  float* orow = p.out + (int64_t)(start + qi) * (p.H * AD) + (int64_t)h * AD;
#pragma unroll
  for (int db = 0; db < AD / 16; db++) {
    f32x4 o = oacc[db] * inv;
    *reinterpret_cast<f32x4*>(orow + db * 16 + g * 4) = o;
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
  if (a.D != AD) return set_error(ctx, FA_ERR_UNSUPPORTED, "attention: head_dim %d != 256", a.D);
  if (a.Hkv <= 0 || a.H % a.Hkv != 0)
    return set_error(ctx, FA_ERR_ARG, "attention: %d query heads not a multiple of %d kv heads", a.H, a.Hkv);
  if (n_items == 0) return FA_OK;
  VarlenParams p;
  p.qkv = a.qkv; p.out = a.out; p.cu = a.cu_seqlens; p.items = d_items;
  p.H = a.H; p.Hkv = a.Hkv; p.window = a.window; p.scale = a.scale;
  dim3 grid((unsigned)n_items, (unsigned)a.H), block(256);
  hipLaunchKernelGGL(attention_varlen_kernel, grid, block, 0, s, p);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

int attention_varlen_qblock() { return QBLK; }

int launch_attention_generic(fa_ctx* ctx, const AttnGenericArgs& a, hipStream_t s) {
  if (a.D > GMAXD) return set_error(ctx, FA_ERR_UNSUPPORTED, "Attention: head dimension %d > %d", a.D, GMAXD);
  const int64_t rows = (int64_t)a.B * a.H * a.T;
  if (rows == 0) return FA_OK;
  hipLaunchKernelGGL(attention_generic_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, a);
  FA_CHECK_LAUNCH(ctx);
  return FA_OK;
}

}  // namespace fa
