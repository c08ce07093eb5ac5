// fa_oracle.cpp — TEST INFRASTRUCTURE, NOT PRODUCT CODE.
//
// A CPU restatement of fiber/ai's EmbeddingGemma-300M encoder forward pass
// (models/gemma, tensor, internal/blas, internal/kernel), written from the
// reference's Go source text. It is the parity checker for the HIP path and
// the timed CPU baseline ("port"). Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load it; the product library never does.
//
// Every function names the reference lines it follows. All arithmetic is
// float32 in the reference's operation order where that order is visible
// at the Go level (RMSNorm's sequential sum, the epilogue order, the
// softmax algebra, GELU's composed steps, pooling); float64 only where the
// reference uses it (RoPE tables, the 1/sqrt of RMSNorm and rmsScale).
// The GEMM accumulation order inside a product is the one place that is
// not the reference's (its 14x32 AVX-512 micro-kernel over KC=512 blocks);
// the reference's own tests bound that freedom at 1e-4*(1+|w|)
// (internal/blas/gemm_test.go:39-56).
//
// Parity status of each function, and the test that pins it, is listed in
// the header comment of tests/test_oracle.py.
//
// Build: oracle/Makefile (g++ -O3 -march=native -fopenmp).

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>
#include <omp.h>

#define ORC_API extern "C" __attribute__((visibility("default")))

typedef int64_t i64;

// ---------------------------------------------------------------------------
// Element-wise math (internal/kernel/generic.go, internal/kernel/math.go)
// ---------------------------------------------------------------------------

// Cephes-style expf with the reference's flush: inputs below -87 give
// exactly 0 (generic.go:278-307; constants generic.go:239-255).
static inline float orc_expf(float v) {
  const float expLog2e = 1.44269504088896341f;
  const float expMagic = 12582912.0f;
  const float expLn2Hi = 0.693359375f;
  const float expLn2Lo = -2.12194440e-4f;
  const float expHi = 88.3762626647949f;
  const float expLo = -87.0f;
  const float c0 = 1.9875691500e-4f, c1 = 1.3981999507e-3f, c2 = 8.3334519073e-3f;
  const float c3 = 4.1665795894e-2f, c4 = 1.6666665459e-1f, c5 = 5.0000001201e-1f;
  if (v < expLo) return 0.0f;
  v = std::min(v, expHi);
  float t = v * expLog2e + expMagic;
  float nf = t - expMagic;
  float r = v - nf * expLn2Hi;
  r -= nf * expLn2Lo;
  float p = c0;
  p = p * r + c1;
  p = p * r + c2;
  p = p * r + c3;
  p = p * r + c4;
  p = p * r + c5;
  p = p * r * r + r + 1.0f;
  int32_t tb, pb;
  std::memcpy(&tb, &t, 4);
  std::memcpy(&pb, &p, 4);
  int32_t e = tb - 0x4B400000;
  uint32_t outb = (uint32_t)pb + ((uint32_t)e << 23);
  float out;
  std::memcpy(&out, &outb, 4);
  return out;
}

// Eigen's float tanh as the reference states it (generic.go:313-359).
static inline float orc_tanhf(float v) {
  const float clamp = 7.99881172180175781f, tiny = 0.0004f;
  const float a1 = 4.89352455891786e-03f, a3 = 6.37261928875436e-04f, a5 = 1.48572235717979e-05f;
  const float a7 = 5.12229709037114e-08f, a9 = -8.60467152213735e-11f, a11 = 2.00018790482477e-13f;
  const float a13 = -2.76076847742355e-16f;
  const float b0 = 4.89352518554385e-03f, b2 = 2.26843463243900e-03f, b4 = 1.18534705686654e-04f;
  const float b6 = 1.19825839466702e-06f;
  if (v > -tiny && v < tiny) return v;
  if (v >= 9) return 1.0f;
  if (v <= -9) return -1.0f;
  v = std::min(std::max(v, -clamp), clamp);
  float v2 = v * v;
  float p = a13;
  p = p * v2 + a11;
  p = p * v2 + a9;
  p = p * v2 + a7;
  p = p * v2 + a5;
  p = p * v2 + a3;
  p = p * v2 + a1;
  p *= v;
  float q = b6;
  q = q * v2 + b4;
  q = q * v2 + b2;
  q = q * v2 + b0;
  return p / q;
}

// tanh-GELU as the reference composes it from vector kernels
// (math.go:117-143): u = c*((x*x*x)*0.044715 + x); 0.5*x*(1+tanh(u)) in
// the order Mul, Mul, Scale, Axpy, Scale, Tanh, AddScalar, Mul, Scale.
static inline float orc_geluf(float x) {
  const float geluC = 0.7978845608028654f;
  float z = x * x;
  z = z * x;
  z = z * 0.044715f;
  z = 1.0f * x + z;
  z = z * geluC;
  z = orc_tanhf(z);
  z = z + 1.0f;
  z = z * x;
  z = z * 0.5f;
  return z;
}

// generic Dot: four interleaved partial sums (generic.go:146-161).
static inline float orc_dotf(const float* x, const float* y, i64 n) {
  float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  i64 i = 0;
  for (; i + 4 <= n; i += 4) {
    s0 += x[i] * y[i];
    s1 += x[i + 1] * y[i + 1];
    s2 += x[i + 2] * y[i + 2];
    s3 += x[i + 3] * y[i + 3];
  }
  for (; i < n; i++) s0 += x[i] * y[i];
  return (s0 + s1) + (s2 + s3);
}

// generic Sum: four interleaved partial sums (generic.go:163-176).
static inline float orc_sumf(const float* x, i64 n) {
  float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
  i64 i = 0;
  for (; i + 4 <= n; i += 4) {
    s0 += x[i];
    s1 += x[i + 1];
    s2 += x[i + 2];
    s3 += x[i + 3];
  }
  for (; i < n; i++) s0 += x[i];
  return (s0 + s1) + (s2 + s3);
}

ORC_API void orc_exp(const float* x, float* z, i64 n) {
  for (i64 i = 0; i < n; i++) z[i] = orc_expf(x[i]);
}
ORC_API void orc_tanh(const float* x, float* z, i64 n) {
  for (i64 i = 0; i < n; i++) z[i] = orc_tanhf(x[i]);
}
ORC_API void orc_gelu(const float* x, float* z, i64 n) {
  for (i64 i = 0; i < n; i++) z[i] = orc_geluf(x[i]);
}

// ---------------------------------------------------------------------------
// Row statistics and normalisation
// ---------------------------------------------------------------------------

// RowSumSquares: Dot(row,row) per row (tensor/matmul_fused.go:125-143).
ORC_API void orc_row_sum_squares(const float* x, i64 m, i64 n, i64 ldx, float* out) {
#pragma omp parallel for schedule(static)
  for (i64 i = 0; i < m; i++) out[i] = orc_dotf(x + i * ldx, x + i * ldx, n);
}

// rmsScale: float32(1/sqrt(float64(ss/float32(n)+eps))) (models/gemma/embed.go:432-438).
static inline float orc_rms_inv(float ss, int n, float eps) {
  float t = ss / (float)n + eps;
  return (float)(1.0 / std::sqrt((double)t));
}
ORC_API void orc_rms_scale(const float* ss, i64 m, int n, float eps, float* out) {
  for (i64 i = 0; i < m; i++) out[i] = orc_rms_inv(ss[i], n, eps);
}

// rmsNormFused: sequential float32 sum of squares, inv as above, then
// dst = v*inv*g (tensor/attention.go:312-337). g is used as given (the
// model passes 1+w, models/gemma/model.go:131-140).
ORC_API void orc_rmsnorm(const float* x, const float* g, float eps, i64 rows, i64 n, float* out) {
#pragma omp parallel for schedule(static)
  for (i64 r = 0; r < rows; r++) {
    const float* row = x + r * n;
    float ss = 0;
    for (i64 i = 0; i < n; i++) ss += row[i] * row[i];
    float inv = orc_rms_inv(ss, (int)n, eps);
    float* dst = out + r * n;
    for (i64 i = 0; i < n; i++) dst[i] = row[i] * inv * g[i];
  }
}

// ---------------------------------------------------------------------------
// RoPE (tensor/rope.go:20-87): rotate-half, float64 angle tables rounded to
// float32, row r of a [.., T, D] tensor at position positions[r % T].
// ---------------------------------------------------------------------------
static void rope_tables(double base, const int32_t* positions, int T, int D, std::vector<float>& cs,
                        std::vector<float>& sn) {
  int half = D / 2;
  std::vector<double> invFreq(half);
  for (int i = 0; i < half; i++) invFreq[i] = std::pow(base, -(double)(2 * i) / (double)D);
  cs.assign((size_t)T * half, 0.f);
  sn.assign((size_t)T * half, 0.f);
  for (int t = 0; t < T; t++) {
    double p = (double)positions[t];
    for (int i = 0; i < half; i++) {
      double a = p * invFreq[i];
      cs[(size_t)t * half + i] = (float)std::cos(a);
      sn[(size_t)t * half + i] = (float)std::sin(a);
    }
  }
}

static inline void rope_row(const float* so, float* dst, const float* c, const float* s, int D) {
  int half = D / 2;
  for (int i = 0; i < half; i++) {
    float x1 = so[i], x2 = so[i + half];
    dst[i] = x1 * c[i] - x2 * s[i];
    dst[i + half] = x1 * s[i] + x2 * c[i];
  }
}

// x is [rows, D] where row r has position positions[r % T] (the
// reference's contiguous [.., T, D] case).
ORC_API int orc_rope(const float* x, double base, const int32_t* positions, i64 rows, int T, int D, float* out) {
  if (D % 2 != 0 || T <= 0) return -1;
  std::vector<float> cs, sn;
  rope_tables(base, positions, T, D, cs, sn);
  int half = D / 2;
#pragma omp parallel for schedule(static)
  for (i64 r = 0; r < rows; r++) {
    int t = (int)(r % T);
    rope_row(x + r * D, out + r * D, &cs[(size_t)t * half], &sn[(size_t)t * half], D);
  }
  return 0;
}

// ---------------------------------------------------------------------------
// Masks (tensor/attention.go:17-42,97-107): additive -1e9.
// ---------------------------------------------------------------------------
static const float kMaskNeg = -1e9f;

ORC_API void orc_padding_mask(const int32_t* lengths, int b, int n, float* out) {
  for (int i = 0; i < b; i++)
    for (int j = 0; j < n; j++) out[(i64)i * n + j] = (j >= std::max(0, (int)lengths[i])) ? kMaskNeg : 0.f;
}
ORC_API void orc_window_mask(int n, int w, float* out) {
  for (int i = 0; i < n; i++)
    for (int j = 0; j < n; j++) out[(i64)i * n + j] = (j - i >= w || i - j >= w) ? kMaskNeg : 0.f;
}
ORC_API void orc_causal_mask(int n, float* out) {
  for (int i = 0; i < n; i++)
    for (int j = 0; j < n; j++) out[(i64)i * n + j] = (j > i) ? kMaskNeg : 0.f;
}

// ---------------------------------------------------------------------------
// GEMM with the blas epilogue (internal/blas/gemm.go:276-347).
// C[m x n] = epilogue(A[m x k] . B[k x n]); A, B, C row-major with leading
// dimensions. Epilogue order: Bias -> RowScale -> Act -> Mul -> Residual.
// ---------------------------------------------------------------------------
enum { ORC_ACT_NONE = 0, ORC_ACT_RELU = 1, ORC_ACT_GELU = 2 };

#if defined(__AVX512F__)
#define ORC_VW 16
#define ORC_MR 4
#else
#define ORC_VW 8
#define ORC_MR 3
#endif
#define ORC_NV 4
#define ORC_NRW (ORC_VW * ORC_NV)
#define ORC_KC 256
#define ORC_MC 96

typedef float vf __attribute__((vector_size(ORC_VW * 4)));
typedef float vfu __attribute__((vector_size(ORC_VW * 4), aligned(4)));

// Micro-kernel: MR rows x NRW cols over kc, B packed [kc][NRW].
static inline void micro(int kc, const float* const* arow, const float* bp, float* c, i64 ldc, bool first,
                         int rows_valid, int cols_valid) {
  vf acc[ORC_MR][ORC_NV];
  for (int r = 0; r < ORC_MR; r++)
    for (int v = 0; v < ORC_NV; v++) acc[r][v] = (vf){0};
  for (int p = 0; p < kc; p++) {
    vf b[ORC_NV];
    for (int v = 0; v < ORC_NV; v++) b[v] = *(const vfu*)(bp + (i64)p * ORC_NRW + v * ORC_VW);
    for (int r = 0; r < ORC_MR; r++) {
      vf a = (vf){0} + arow[r][p];
      for (int v = 0; v < ORC_NV; v++) acc[r][v] += a * b[v];
    }
  }
  for (int r = 0; r < rows_valid; r++) {
    float* cr = c + (i64)r * ldc;
    if (cols_valid == ORC_NRW) {
      for (int v = 0; v < ORC_NV; v++) {
        vf cur = first ? (vf){0} : *(vfu*)(cr + v * ORC_VW);
        *(vfu*)(cr + v * ORC_VW) = cur + acc[r][v];
      }
    } else {
      float tmp[ORC_NRW];
      for (int v = 0; v < ORC_NV; v++) *(vfu*)(tmp + v * ORC_VW) = acc[r][v];
      for (int j = 0; j < cols_valid; j++) cr[j] = (first ? 0.f : cr[j]) + tmp[j];
    }
  }
}

static void apply_epilogue_row(float* row, i64 i, i64 c0, i64 c1, const float* bias, const float* rowscale, int act,
                               const float* mul, i64 ldm, const float* residual, i64 ldr) {
  for (i64 j = c0; j < c1; j++) {
    float v = row[j];
    if (bias) v = v + bias[j];
    if (rowscale) v = v * rowscale[i];
    if (act == ORC_ACT_RELU) v = std::max(v, 0.f);
    else if (act == ORC_ACT_GELU) v = orc_geluf(v);
    if (mul) v = v * mul[i * ldm + j];
    if (residual) v = v + residual[i * ldr + j];
    row[j] = v;
  }
}

ORC_API int orc_gemm(i64 m, i64 n, i64 k, const float* A, i64 lda, const float* B, i64 ldb, float* C, i64 ldc,
                     const float* bias, const float* rowscale, int act, const float* mul, i64 ldm,
                     const float* residual, i64 ldr) {
  if (m < 0 || n < 0 || k < 0) return -1;
  if (m == 0 || n == 0) return 0;
  i64 nmb = (m + ORC_MC - 1) / ORC_MC;
  i64 nnb = (n + ORC_NRW - 1) / ORC_NRW;
#pragma omp parallel
  {
    std::vector<float> bp((size_t)ORC_KC * ORC_NRW);
#pragma omp for schedule(dynamic, 1) collapse(2)
    for (i64 ib = 0; ib < nmb; ib++) {
      for (i64 jb = 0; jb < nnb; jb++) {
        i64 i0 = ib * ORC_MC, i1 = std::min(m, i0 + ORC_MC);
        i64 j0 = jb * ORC_NRW;
        int cols = (int)std::min<i64>(ORC_NRW, n - j0);
        if (k == 0) {
          for (i64 i = i0; i < i1; i++)
            for (int j = 0; j < cols; j++) C[i * ldc + j0 + j] = 0.f;
        }
        for (i64 p0 = 0; p0 < k; p0 += ORC_KC) {
          int kc = (int)std::min<i64>(ORC_KC, k - p0);
          for (int p = 0; p < kc; p++) {
            const float* src = B + (p0 + p) * ldb + j0;
            float* dst = &bp[(size_t)p * ORC_NRW];
            int j = 0;
            for (; j < cols; j++) dst[j] = src[j];
            for (; j < ORC_NRW; j++) dst[j] = 0.f;
          }
          for (i64 i = i0; i < i1; i += ORC_MR) {
            int rv = (int)std::min<i64>(ORC_MR, i1 - i);
            const float* ar[ORC_MR];
            for (int r = 0; r < ORC_MR; r++) ar[r] = A + std::min(i + r, i1 - 1) * lda + p0;
            micro(kc, ar, bp.data(), C + i * ldc + j0, ldc, p0 == 0, rv, cols);
          }
        }
        if (bias || rowscale || act || mul || residual)
          for (i64 i = i0; i < i1; i++)
            apply_epilogue_row(C + i * ldc, i, j0, j0 + cols, bias, rowscale, act, mul, ldm, residual, ldr);
      }
    }
  }
  return 0;
}

// ---------------------------------------------------------------------------
// Attention (tensor/attention.go:67-83,130-287; internal/blas/attention.go:61-136)
// Per (batch, head): scores row = q.k for every key; the mask joins the raw
// scores as mask*invScale (attention.go:185-192); max; ExpSum with
// a = scale, b = -scale*max (generic.go:264-276, flush below -87); the
// unnormalised probabilities times V; the row scaled by 1/sum.
// Lead dims are (B, H) with element strides; GQA is a zero head stride on
// k and v (the reference's Expand). The mask has strides (mb, mh, mrow,
// mcol) over [B, H, T, S]; pass mask == nullptr for none.
// ---------------------------------------------------------------------------
ORC_API int orc_attention(const float* q, const float* k, const float* v, int B, int H, int T, int S, int D,
                          i64 qsb, i64 qsh, i64 ksb, i64 ksh, i64 vsb, i64 vsh, const float* mask, i64 msb,
                          i64 msh, i64 msr, i64 msc, float scale, float* out) {
  if (B < 0 || H < 0 || T < 0 || S <= 0 || D <= 0) return -1;
  // out is [B, H, T, D] contiguous, like the reference's result.
  const i64 rows_total = (i64)B * H * T;
#pragma omp parallel
  {
    std::vector<float> row(S);
    std::vector<float> acc(D);
#pragma omp for schedule(static)
    for (i64 idx = 0; idx < rows_total; idx++) {
      int b = (int)(idx / ((i64)H * T));
      int h = (int)((idx / T) % H);
      int i = (int)(idx % T);
      const float* qi = q + b * qsb + h * qsh + (i64)i * D;
      const float* kb = k + b * ksb + h * ksh;
      const float* vb = v + b * vsb + h * vsh;
      // raw scores (the GEMM of q-panel x K-panels, attention.go:102-104)
      for (int j = 0; j < S; j++) {
        const float* kj = kb + (i64)j * D;
        float s = 0;
        for (int c = 0; c < D; c++) s += qi[c] * kj[c];
        row[j] = s;
      }
      float a = scale, invScale = 1.f;
      if (scale > 0) {
        invScale = 1.f / scale;
      } else {
        for (int j = 0; j < S; j++) row[j] = row[j] * scale;
        a = 1.f;
      }
      if (mask) {
        const float* mr = mask + b * msb + h * msh + (i64)i * msr;
        for (int j = 0; j < S; j++) row[j] = invScale * mr[j * msc] + row[j];
      }
      float mx = row[0];
      for (int j = 1; j < S; j++) mx = std::max(mx, row[j]);
      float bsh = -a * mx, sum = 0;
      for (int j = 0; j < S; j++) {
        row[j] = orc_expf(a * row[j] + bsh);
      }
      for (int j = 0; j < S; j++) sum += row[j];
      float inv = 1.f / sum;
      for (int c = 0; c < D; c++) acc[c] = 0.f;
      for (int j = 0; j < S; j++) {
        float p = row[j];
        if (p == 0.f) continue;  // exact zero weight adds exactly 0
        const float* vj = vb + (i64)j * D;
        for (int c = 0; c < D; c++) acc[c] += p * vj[c];
      }
      float* o = out + idx * D;
      for (int c = 0; c < D; c++) o[c] = acc[c] * inv;
    }
  }
  return 0;
}

// ---------------------------------------------------------------------------
// Similarities + top-k (cluster/cluster.go:185-190; ties -> lower index as
// tensor/reduce.go:286-289's first-max rule). NaN scores rank below every
// number (a NaN never compares greater in the reference's Argmax loop; the
// loop only returns a NaN when it is the row's first element, an artifact
// this build does not follow); slots past a row's non-NaN scores hold index
// -1 and value NaN.
// ---------------------------------------------------------------------------
ORC_API int orc_similarities_topk(const float* Q, i64 nq, const float* Dm, i64 nd, int d, int topk, int32_t* idx,
                                  float* val) {
  if (topk <= 0 || topk > nd) return -1;
#pragma omp parallel
  {
    std::vector<float> sc(nd);
    std::vector<int32_t> order(nd);
#pragma omp for schedule(dynamic, 1)
    for (i64 qi = 0; qi < nq; qi++) {
      const float* qr = Q + qi * d;
      for (i64 j = 0; j < nd; j++) {
        const float* dr = Dm + j * d;
        float s = 0;
        for (int c = 0; c < d; c++) s += qr[c] * dr[c];
        sc[j] = s;
      }
      for (i64 j = 0; j < nd; j++) order[j] = (int32_t)j;
      std::partial_sort(order.begin(), order.begin() + topk, order.end(), [&](int32_t a, int32_t b) {
        const bool na = std::isnan(sc[a]), nb = std::isnan(sc[b]);
        if (na != nb) return nb;
        if (!na && sc[a] != sc[b]) return sc[a] > sc[b];
        return a < b;
      });
      for (int t = 0; t < topk; t++) {
        const bool nan = std::isnan(sc[order[t]]);
        idx[qi * topk + t] = nan ? -1 : order[t];
        if (val) val[qi * topk + t] = sc[order[t]];
      }
    }
  }
  return 0;
}

// ---------------------------------------------------------------------------
// The encoder model (models/gemma: config.go, model.go, embed.go)
// ---------------------------------------------------------------------------
struct OrcConfig {
  int hidden, layers, heads, kv_heads, head_dim, ffn, vocab;
  int sliding_window, bidirectional, pattern;
  double rope_local, rope_theta, qpas;
  float eps;
  int n_dense;
  int dense_out[4];
  int dense_tanh[4];  // Dense layer followed by Tanh (model.go:296-301)
};

struct OrcLayer {
  std::vector<float> wq, wk, wv, wo, wgate, wup, wdown;  // [in, out], pre-norms folded into q,k,v,gate,up
  std::vector<float> inputNorm, postAttnNorm, preFFNNorm, postFFNNorm, qNorm, kNorm;  // 1+w
  std::vector<float> raw_wq, raw_wk, raw_wv, raw_wgate, raw_wup;  // before folding
};

struct OrcModel {
  OrcConfig cfg;
  std::vector<float> embed;  // [vocab, hidden]
  std::vector<OrcLayer> layers;
  std::vector<float> norm;                 // 1+w
  std::vector<std::vector<float>> dense;   // [in, out]
  std::vector<int> dense_in, dense_out;
  bool finalized = false;
  std::map<std::string, int> seen;
};

// Config.window (config.go:331-339) for Variant 0.
static int cfg_window(const OrcConfig& c) {
  if (c.bidirectional) return c.sliding_window / 2 + 1;
  return c.sliding_window;
}
// isSliding via default layer types (config.go:213-225, 342).
static bool cfg_sliding(const OrcConfig& c, int l) { return (l + 1) % c.pattern != 0; }
// ropeBase (config.go:346-362).
static double cfg_rope_base(const OrcConfig& c, int l) {
  if (cfg_sliding(c, l)) return c.rope_local != 0 ? c.rope_local : 10000.0;
  return c.rope_theta != 0 ? c.rope_theta : 10000.0;
}

ORC_API void* orc_model_create(int hidden, int layers, int heads, int kv_heads, int head_dim, int ffn, int vocab,
                               int sliding_window, int bidirectional, int pattern, double rope_local,
                               double rope_theta, double qpas, float eps, int n_dense, const int* dense_out) {
  if (n_dense < 0 || n_dense > 4) return nullptr;
  OrcModel* m = new OrcModel();
  OrcConfig& c = m->cfg;
  c.hidden = hidden; c.layers = layers; c.heads = heads; c.kv_heads = kv_heads; c.head_dim = head_dim;
  c.ffn = ffn; c.vocab = vocab; c.sliding_window = sliding_window; c.bidirectional = bidirectional;
  c.pattern = pattern > 0 ? pattern : 6; c.rope_local = rope_local; c.rope_theta = rope_theta; c.qpas = qpas;
  c.eps = eps; c.n_dense = n_dense;
  for (int i = 0; i < n_dense; i++) {
    c.dense_out[i] = dense_out[i];
    c.dense_tanh[i] = 0;
  }
  m->layers.resize(layers);
  m->dense.resize(n_dense);
  m->dense_in.resize(n_dense);
  m->dense_out.resize(n_dense);
  int in = hidden;
  for (int i = 0; i < n_dense; i++) {
    m->dense_in[i] = in;
    m->dense_out[i] = dense_out[i];
    in = dense_out[i];
  }
  return m;
}

ORC_API void orc_model_destroy(void* p) { delete (OrcModel*)p; }

// Dense layer i of the head followed by Tanh (torch.nn.modules.activation.Tanh,
// model.go:296-301; applied after the product, embed.go:415-418).
ORC_API int orc_model_set_dense_tanh(void* p, int i, int on) {
  OrcModel* m = (OrcModel*)p;
  if (i < 0 || i >= m->cfg.n_dense) return -3;
  m->cfg.dense_tanh[i] = on != 0;
  return 0;
}

// transpose [out, in] -> [in, out] (model.go:121-127)
static std::vector<float> transpose_w(const float* w, int out, int in) {
  std::vector<float> t((size_t)in * out);
#pragma omp parallel for schedule(static)
  for (int i = 0; i < in; i++)
    for (int o = 0; o < out; o++) t[(size_t)i * out + o] = w[(size_t)o * in + i];
  return t;
}
// norm: w + 1 (model.go:131-140)
static std::vector<float> plus_one(const float* w, int n) {
  std::vector<float> t(n);
  for (int i = 0; i < n; i++) t[i] = w[i] + 1.0f;
  return t;
}

// Set one checkpoint tensor by its Hugging Face name (model.go:142-191;
// head modules "dense.<i>.linear.weight", model.go:277-304). Matrices are
// [out, in] float32 as stored.
ORC_API int orc_model_set(void* p, const char* name, const float* data, i64 numel) {
  OrcModel* m = (OrcModel*)p;
  const OrcConfig& c = m->cfg;
  std::string s(name);
  int H = c.heads, Hkv = c.kv_heads, D = c.head_dim, d = c.hidden, F = c.ffn;
  auto expect = [&](i64 n) { return numel == n; };
  if (s == "embed_tokens.weight") {
    if (!expect((i64)c.vocab * d)) return -2;
    m->embed.assign(data, data + numel);
  } else if (s == "norm.weight") {
    if (!expect(d)) return -2;
    m->norm = plus_one(data, d);
  } else if (s.rfind("dense.", 0) == 0) {
    int i = std::atoi(s.c_str() + 6);
    if (i < 0 || i >= c.n_dense) return -3;
    if (!expect((i64)m->dense_in[i] * m->dense_out[i])) return -2;
    m->dense[i] = transpose_w(data, m->dense_out[i], m->dense_in[i]);
  } else if (s.rfind("layers.", 0) == 0) {
    int l = std::atoi(s.c_str() + 7);
    if (l < 0 || l >= c.layers) return -3;
    std::string rest = s.substr(s.find('.', 7) + 1);
    OrcLayer& L = m->layers[l];
    if (rest == "input_layernorm.weight") { if (!expect(d)) return -2; L.inputNorm = plus_one(data, d); }
    else if (rest == "post_attention_layernorm.weight") { if (!expect(d)) return -2; L.postAttnNorm = plus_one(data, d); }
    else if (rest == "pre_feedforward_layernorm.weight") { if (!expect(d)) return -2; L.preFFNNorm = plus_one(data, d); }
    else if (rest == "post_feedforward_layernorm.weight") { if (!expect(d)) return -2; L.postFFNNorm = plus_one(data, d); }
    else if (rest == "self_attn.q_norm.weight") { if (!expect(D)) return -2; L.qNorm = plus_one(data, D); }
    else if (rest == "self_attn.k_norm.weight") { if (!expect(D)) return -2; L.kNorm = plus_one(data, D); }
    else if (rest == "self_attn.q_proj.weight") { if (!expect((i64)H * D * d)) return -2; L.raw_wq = transpose_w(data, H * D, d); }
    else if (rest == "self_attn.k_proj.weight") { if (!expect((i64)Hkv * D * d)) return -2; L.raw_wk = transpose_w(data, Hkv * D, d); }
    else if (rest == "self_attn.v_proj.weight") { if (!expect((i64)Hkv * D * d)) return -2; L.raw_wv = transpose_w(data, Hkv * D, d); }
    else if (rest == "self_attn.o_proj.weight") { if (!expect((i64)d * H * D)) return -2; L.wo = transpose_w(data, d, H * D); }
    else if (rest == "mlp.gate_proj.weight") { if (!expect((i64)F * d)) return -2; L.raw_wgate = transpose_w(data, F, d); }
    else if (rest == "mlp.up_proj.weight") { if (!expect((i64)F * d)) return -2; L.raw_wup = transpose_w(data, F, d); }
    else if (rest == "mlp.down_proj.weight") { if (!expect((i64)d * F)) return -2; L.wdown = transpose_w(data, d, F); }
    else return -3;
  } else {
    return -3;
  }
  m->seen[s]++;
  return 0;
}

// Fold the pre-norms into the weights they feed: W' = diag(1+g)*W with W
// [in, out] (model.go:210-222).
static std::vector<float> fold(const std::vector<float>& w, const std::vector<float>& g, int in, int out) {
  std::vector<float> r((size_t)in * out);
#pragma omp parallel for schedule(static)
  for (int i = 0; i < in; i++)
    for (int o = 0; o < out; o++) r[(size_t)i * out + o] = w[(size_t)i * out + o] * g[i];
  return r;
}

ORC_API int orc_model_finalize(void* p) {
  OrcModel* m = (OrcModel*)p;
  const OrcConfig& c = m->cfg;
  int expected = 2 + c.n_dense + 13 * c.layers;
  if ((int)m->seen.size() != expected) return -4;
  int H = c.heads, Hkv = c.kv_heads, D = c.head_dim, d = c.hidden, F = c.ffn;
  for (auto& L : m->layers) {
    L.wq = fold(L.raw_wq, L.inputNorm, d, H * D);
    L.wk = fold(L.raw_wk, L.inputNorm, d, Hkv * D);
    L.wv = fold(L.raw_wv, L.inputNorm, d, Hkv * D);
    L.wgate = fold(L.raw_wgate, L.preFFNNorm, d, F);
    L.wup = fold(L.raw_wup, L.preFFNNorm, d, F);
    std::vector<float>().swap(L.raw_wq);
    std::vector<float>().swap(L.raw_wk);
    std::vector<float>().swap(L.raw_wv);
    std::vector<float>().swap(L.raw_wgate);
    std::vector<float>().swap(L.raw_wup);
  }
  m->finalized = true;
  return 0;
}

// Model.encode for Variant 0 (embed.go:160-240): h [B*T, d] = the final
// hidden states. ids is [B*T] right-padded with 0 (embed.go:122-138). For
// inspection, snapshot i (0 <= i < n_snap) copies the residual stream x after
// the first snap[i] layers (0 <= snap[i] <= layers; 0 is the scaled
// embedding gather) into snaps + i*B*T*d, or h itself when snap[i] < 0.
static int orc_encode(OrcModel* m, const int32_t* ids, const int32_t* lengths, int B, int T, const int* snap,
                      int n_snap, float* snaps, std::vector<float>& h) {
  if (!m->finalized) return -5;
  const OrcConfig& c = m->cfg;
  const int H = c.heads, Hkv = c.kv_heads, D = c.head_dim, d = c.hidden, F = c.ffn;
  const i64 M = (i64)B * T;
  const float eps = c.eps;
  const float scale = (float)(1.0 / std::sqrt(c.qpas));  // model.go:100
  for (i64 i = 0; i < M; i++)
    if (ids[i] < 0 || ids[i] >= c.vocab) return -7;
  for (int i = 0; i < n_snap; i++)
    if (snap[i] > c.layers) return -8;
  auto take = [&](int layers_done, const std::vector<float>& src) {
    for (int i = 0; i < n_snap; i++)
      if (snap[i] == layers_done) std::memcpy(snaps + (size_t)i * M * d, src.data(), sizeof(float) * M * d);
  };

  std::vector<int32_t> positions(T);
  for (int t = 0; t < T; t++) positions[t] = t;
  const int w = cfg_window(c);
  const bool use_window = c.sliding_window > 0 && T > w;  // embed.go:169-172

  // x = E.Rows(ids) * float32(sqrt(hidden)) (embed.go:175-176)
  const float sq = (float)std::sqrt((double)d);
  std::vector<float> x((size_t)M * d);
#pragma omp parallel for schedule(static)
  for (i64 r = 0; r < M; r++) {
    const float* e = &m->embed[(size_t)ids[r] * d];
    for (int i = 0; i < d; i++) x[(size_t)r * d + i] = e[i] * sq;
  }

  std::vector<float> ss(M), sc(M);
  std::vector<float> q0((size_t)M * H * D), k0((size_t)M * Hkv * D), v0((size_t)M * Hkv * D);
  std::vector<float> q((size_t)M * H * D), k((size_t)M * Hkv * D);
  std::vector<float> qr((size_t)M * H * D), kr((size_t)M * Hkv * D), vc((size_t)M * Hkv * D);
  std::vector<float> att((size_t)M * H * D), attc((size_t)M * H * D);
  std::vector<float> o0((size_t)M * d), o((size_t)M * d);
  std::vector<float> up((size_t)M * F), gu((size_t)M * F);
  // Additive mask [B, 1, T, T] for the layer: pad (+ window on sliding layers), embed.go:168-186.
  std::vector<float> padm((size_t)B * T), winm, mask_sl;
  orc_padding_mask(lengths, B, T, padm.data());
  if (use_window) {
    winm.resize((size_t)T * T);
    orc_window_mask(T, w, winm.data());
    mask_sl.resize((size_t)B * T * T);
    for (int b = 0; b < B; b++)
      for (int i = 0; i < T; i++)
        for (int j = 0; j < T; j++)
          mask_sl[((size_t)b * T + i) * T + j] = padm[(size_t)b * T + j] + winm[(size_t)i * T + j];
  }
  std::vector<float> cs, sn, tmp;
  take(0, x);

  for (int l = 0; l < c.layers; l++) {
    const OrcLayer& L = m->layers[l];
    // Attention block
    orc_row_sum_squares(x.data(), M, d, d, ss.data());
    orc_rms_scale(ss.data(), M, d, eps, sc.data());
    orc_gemm(M, H * D, d, x.data(), d, L.wq.data(), H * D, q0.data(), H * D, nullptr, sc.data(), 0, nullptr, 0, nullptr, 0);
    orc_gemm(M, Hkv * D, d, x.data(), d, L.wk.data(), Hkv * D, k0.data(), Hkv * D, nullptr, sc.data(), 0, nullptr, 0, nullptr, 0);
    orc_gemm(M, Hkv * D, d, x.data(), d, L.wv.data(), Hkv * D, v0.data(), Hkv * D, nullptr, sc.data(), 0, nullptr, 0, nullptr, 0);
    orc_rmsnorm(q0.data(), L.qNorm.data(), eps, M * H, D, q.data());
    orc_rmsnorm(k0.data(), L.kNorm.data(), eps, M * Hkv, D, k.data());
    // Permute [B,T,h,D] -> [B,h,T,D] and RoPE with positions 0..T-1 (embed.go:201-207, rope.go:20-87)
    double base = cfg_rope_base(c, l);
    rope_tables(base, positions.data(), T, D, cs, sn);
    const int half = D / 2;
#pragma omp parallel for schedule(static)
    for (i64 r = 0; r < M; r++) {
      int b = (int)(r / T), t = (int)(r % T);
      for (int h = 0; h < H; h++)
        rope_row(&q[((size_t)r * H + h) * D], &qr[(((size_t)b * H + h) * T + t) * D], &cs[(size_t)t * half],
                 &sn[(size_t)t * half], D);
      for (int h = 0; h < Hkv; h++) {
        rope_row(&k[((size_t)r * Hkv + h) * D], &kr[(((size_t)b * Hkv + h) * T + t) * D], &cs[(size_t)t * half],
                 &sn[(size_t)t * half], D);
        std::memcpy(&vc[(((size_t)b * Hkv + h) * T + t) * D], &v0[((size_t)r * Hkv + h) * D], sizeof(float) * D);
      }
    }
    // AttentionScaled(q, k.Expand, v.Expand, mask, scale) (embed.go:209); GQA: head h reads kv head h/(H/Hkv)
    const bool sl = use_window && cfg_sliding(c, l);
    const int grp = H / Hkv;
    const float* mk = sl ? mask_sl.data() : padm.data();
    const i64 msb = sl ? (i64)T * T : T, msr = sl ? T : 0;
    tmp.resize((size_t)B * grp * T * D);
    for (int hk = 0; hk < Hkv; hk++) {
      // query heads hk*grp .. hk*grp+grp-1 read kv head hk (stride 0 over them, the reference's Expand)
      orc_attention(&qr[(size_t)hk * grp * T * D], &kr[(size_t)hk * T * D], &vc[(size_t)hk * T * D], B, grp, T, T, D,
                    (i64)H * T * D, (i64)T * D, (i64)Hkv * T * D, 0, (i64)Hkv * T * D, 0, mk, msb, 0, msr, 1, scale,
                    tmp.data());
      for (int b = 0; b < B; b++)
        for (int g = 0; g < grp; g++)
          std::memcpy(&att[(((size_t)b * H + hk * grp + g) * T) * D], &tmp[(((size_t)b * grp + g) * T) * D],
                      sizeof(float) * T * D);
    }
    // Permute back [B,H,T,D] -> [B,T,H*D] (embed.go:212)
#pragma omp parallel for schedule(static)
    for (i64 r = 0; r < M; r++) {
      int b = (int)(r / T), t = (int)(r % T);
      for (int h = 0; h < H; h++)
        std::memcpy(&attc[((size_t)r * H + h) * D], &att[(((size_t)b * H + h) * T + t) * D], sizeof(float) * D);
    }
    orc_gemm(M, d, H * D, attc.data(), H * D, L.wo.data(), d, o0.data(), d, nullptr, nullptr, 0, nullptr, 0, nullptr, 0);
    orc_rmsnorm(o0.data(), L.postAttnNorm.data(), eps, M, d, o.data());
#pragma omp parallel for schedule(static)
    for (i64 i = 0; i < M * d; i++) x[i] = x[i] + o[i];
    // Feed-forward block (embed.go:224-235)
    orc_row_sum_squares(x.data(), M, d, d, ss.data());
    orc_rms_scale(ss.data(), M, d, eps, sc.data());
    orc_gemm(M, F, d, x.data(), d, L.wup.data(), F, up.data(), F, nullptr, sc.data(), 0, nullptr, 0, nullptr, 0);
    orc_gemm(M, F, d, x.data(), d, L.wgate.data(), F, gu.data(), F, nullptr, sc.data(), ORC_ACT_GELU, up.data(), F,
             nullptr, 0);
    orc_gemm(M, d, F, gu.data(), F, L.wdown.data(), d, o0.data(), d, nullptr, nullptr, 0, nullptr, 0, nullptr, 0);
    orc_rmsnorm(o0.data(), L.postFFNNorm.data(), eps, M, d, o.data());
#pragma omp parallel for schedule(static)
    for (i64 i = 0; i < M * d; i++) x[i] = x[i] + o[i];
    take(l + 1, x);
  }
  h.resize((size_t)M * d);
  orc_rmsnorm(x.data(), m->norm.data(), eps, M, d, h.data());
  for (int i = 0; i < n_snap; i++)
    if (snap[i] < 0) std::memcpy(snaps + (size_t)i * M * d, h.data(), sizeof(float) * M * d);
  return 0;
}

// The encoder's states for inspection (orc_encode's snapshots); snaps is
// [n_snap, B*T, d].
ORC_API int orc_model_encode(void* p, const int32_t* ids, const int32_t* lengths, int B, int T, const int* snap,
                             int n_snap, float* snaps) {
  std::vector<float> h;
  return orc_encode((OrcModel*)p, ids, lengths, B, T, snap, n_snap, snaps, h);
}

// Model.encode (orc_encode) followed by pool (embed.go:381-404), applyHead
// and l2normalize (embed.go:408-429,472-475). out is [B, dim].
ORC_API int orc_model_embed(void* p, const int32_t* ids, const int32_t* lengths, int B, int T, int dim, float* out) {
  OrcModel* m = (OrcModel*)p;
  if (!m->finalized) return -5;
  const OrcConfig& c = m->cfg;
  const int d = c.hidden;
  int full = d;
  if (c.n_dense > 0) full = m->dense_out[c.n_dense - 1];
  if (dim <= 0) dim = full;
  if (dim > full) return -6;
  std::vector<float> h;
  const int rc = orc_encode(m, ids, lengths, B, T, nullptr, 0, nullptr, h);
  if (rc) return rc;

  // pool: masked mean (embed.go:381-404)
  std::vector<float> pooled((size_t)B * d, 0.f);
  for (int b = 0; b < B; b++) {
    int n = lengths[b];
    if (n == 0) n = 1;
    float* dst = &pooled[(size_t)b * d];
    for (int t = 0; t < n; t++) {
      const float* row = &h[((size_t)b * T + t) * d];
      for (int i = 0; i < d; i++) dst[i] += row[i];
    }
    float inv = 1.f / (float)n;
    for (int i = 0; i < d; i++) dst[i] *= inv;
  }
  // applyHead: Dense layers, Narrow(dim) before L2, l2normalize (embed.go:408-429,472-475)
  std::vector<float> y = pooled, y2;
  int cur = d;
  for (int i = 0; i < c.n_dense; i++) {
    int no = m->dense_out[i];
    y2.assign((size_t)B * no, 0.f);
    orc_gemm(B, no, cur, y.data(), cur, m->dense[i].data(), no, y2.data(), no, nullptr, nullptr, 0, nullptr, 0, nullptr, 0);
    if (c.dense_tanh[i])  // (*Tensor).Tanh: kernel.Tanh, the rational of generic.go:313-359
      for (auto& v : y2) v = orc_tanhf(v);
    y.swap(y2);
    cur = no;
  }
  for (int b = 0; b < B; b++) {
    const float* yr = &y[(size_t)b * cur];
    std::vector<float> sq2(dim);
    for (int i = 0; i < dim; i++) sq2[i] = yr[i] * yr[i];
    float s = orc_sumf(sq2.data(), dim);
    float nrm = std::sqrt(s + 1e-12f);
    for (int i = 0; i < dim; i++) out[(size_t)b * dim + i] = yr[i] / nrm;
  }
  return 0;
}

ORC_API int orc_num_threads(void) { return omp_get_max_threads(); }

// ---------------------------------------------------------------------------
// cluster (cluster/cluster.go): Normalize, Nearest, KMeans with k-means++
// seeding from Go's math/rand/v2 PCG generator.
// ---------------------------------------------------------------------------

// Go standard library math/rand/v2 (Go >= 1.22; not part of the reference
// tree): PCG is O'Neill's 128-bit LCG with the pcg-cpp default multiplier
// and increment, state (hi, lo) = (seed1, seed2) as NewPCG sets it; Uint64
// advances the state and returns the DXSM ("double xorshift multiply")
// output of the new state.
struct OrcPCG {
  uint64_t hi, lo;
};

static uint64_t orc_pcg_next(OrcPCG& p) {
  typedef unsigned __int128 u128;
  const u128 mul = ((u128)2549297995355413924ULL << 64) | 4865540595714422341ULL;
  const u128 inc = ((u128)6364136223846793005ULL << 64) | 1442695040888963407ULL;
  const u128 s = (((u128)p.hi << 64) | p.lo) * mul + inc;
  p.hi = (uint64_t)(s >> 64);
  p.lo = (uint64_t)s;
  uint64_t h = p.hi;
  h ^= h >> 32;
  h *= 0xda942042e4dd58b5ULL;
  h ^= h >> 48;
  h *= (p.lo | 1);
  return h;
}

// Rand.IntN (uint64n on 64-bit hosts): a mask for powers of two, else
// Lemire's multiply-shift with rejection of the biased low products.
static uint64_t orc_pcg_uint64n(OrcPCG& p, uint64_t n) {
  typedef unsigned __int128 u128;
  if ((n & (n - 1)) == 0) return orc_pcg_next(p) & (n - 1);
  u128 m = (u128)orc_pcg_next(p) * n;
  if ((uint64_t)m < n) {
    const uint64_t thresh = (0 - n) % n;
    while ((uint64_t)m < thresh) m = (u128)orc_pcg_next(p) * n;
  }
  return (uint64_t)(m >> 64);
}

// Rand.Float64: 53 random bits / 2^53.
static double orc_pcg_float64(OrcPCG& p) { return (double)(orc_pcg_next(p) << 11 >> 11) / 9007199254740992.0; }

// state[2] = {hi, lo}; the draws advance it.
ORC_API void orc_pcg_uint64s(uint64_t* state, int64_t count, uint64_t* out) {
  OrcPCG p{state[0], state[1]};
  for (int64_t i = 0; i < count; i++) out[i] = orc_pcg_next(p);
  state[0] = p.hi;
  state[1] = p.lo;
}
ORC_API void orc_pcg_intns(uint64_t* state, uint64_t n, int64_t count, uint64_t* out) {
  OrcPCG p{state[0], state[1]};
  for (int64_t i = 0; i < count; i++) out[i] = orc_pcg_uint64n(p, n);
  state[0] = p.hi;
  state[1] = p.lo;
}
ORC_API void orc_pcg_float64s(uint64_t* state, int64_t count, double* out) {
  OrcPCG p{state[0], state[1]};
  for (int64_t i = 0; i < count; i++) out[i] = orc_pcg_float64(p);
  state[0] = p.hi;
  state[1] = p.lo;
}

// cluster.Normalize (cluster.go:17-28): row / sqrt(sum of squares), a zero
// norm replaced by 1 so zero rows stay zero. Sum(1) is one horizontal
// kernel.Sum per row (tensor/reduce.go:131-141).
static void orc_normalize_rows(const float* x, i64 n, int d, float* out) {
#pragma omp parallel for schedule(static)
  for (i64 i = 0; i < n; i++) {
    const float* r = x + i * d;
    std::vector<float> sq(d);
    for (int j = 0; j < d; j++) sq[j] = r[j] * r[j];
    float nrm = std::sqrt(orc_sumf(sq.data(), d));
    if (nrm == 0) nrm = 1;
    for (int j = 0; j < d; j++) out[i * d + j] = r[j] / nrm;
  }
}

ORC_API void orc_cluster_normalize(const float* x, i64 n, int d, float* out) { orc_normalize_rows(x, n, d, out); }

// sim[n x k] = x . c^T, then the first-max argmax of each row
// (tensor/reduce.go:269-297): the first index holding the row's maximum.
static void orc_sim_argmax(const float* x, i64 n, const float* c, i64 k, int d, float* sim, int32_t* idx) {
#pragma omp parallel for schedule(static)
  for (i64 i = 0; i < n; i++) {
    float* sr = sim + i * k;
    for (i64 j = 0; j < k; j++) sr[j] = orc_dotf(x + i * d, c + j * d, d);
    float best = sr[0];
    int32_t bi = 0;
    for (i64 j = 1; j < k; j++)
      if (sr[j] > best) {
        best = sr[j];
        bi = (int32_t)j;
      }
    idx[i] = bi;
  }
}

// cluster.Nearest (cluster.go:134-146).
ORC_API int orc_cluster_nearest(const float* x, i64 n, const float* c, i64 k, int d, int32_t* idx, float* sim_out) {
  if (k <= 0) return -1;
  std::vector<float> sim((size_t)(n * k));
  orc_sim_argmax(x, n, c, k, d, sim.data(), idx);
  for (i64 i = 0; i < n; i++) sim_out[i] = sim[(size_t)(i * k + idx[i])];
  return 0;
}

// cluster.KMeans (cluster.go:39-131). chosen[k] receives the seeding's row
// indices (test visibility).
ORC_API int orc_cluster_kmeans(const float* x, i64 n, int d, int k, int iters, uint64_t seed, float* centres_out,
                               int32_t* assign, float* similarity, int32_t* sizes, int* iterations,
                               int32_t* chosen) {
  if (k <= 0 || k > n) return -1;
  OrcPCG rng{seed, seed ^ 0x9e3779b97f4a7c15ULL};
  // k-means++ (cluster.go:51-85)
  std::vector<float> centres;
  centres.reserve((size_t)k * d);
  const i64 first = (i64)orc_pcg_uint64n(rng, (uint64_t)n);
  chosen[0] = (int32_t)first;
  centres.insert(centres.end(), x + first * d, x + (first + 1) * d);
  std::vector<float> best((size_t)n, -1.0f), sim1((size_t)n);
  std::vector<double> weights((size_t)n);
  for (int r = 1; r < k; r++) {
    const float* c = centres.data() + (size_t)(r - 1) * d;
#pragma omp parallel for schedule(static)
    for (i64 i = 0; i < n; i++) sim1[i] = orc_dotf(x + i * d, c, d);
    double total = 0;
    for (i64 i = 0; i < n; i++) {
      if (sim1[i] > best[i]) best[i] = sim1[i];
      const double w = (double)(1 - best[i]);
      weights[i] = w * w;
      total += weights[i];
    }
    double pick = orc_pcg_float64(rng) * total;
    i64 idx = n - 1;
    for (i64 i = 0; i < n; i++) {
      pick -= weights[i];
      if (pick <= 0) {
        idx = i;
        break;
      }
    }
    chosen[r] = (int32_t)idx;
    centres.insert(centres.end(), x + idx * d, x + (idx + 1) * d);
  }
  std::vector<float> cs((size_t)k * d);
  orc_normalize_rows(centres.data(), k, d, cs.data());

  // Lloyd rounds (cluster.go:86-129)
  for (i64 i = 0; i < n; i++) {
    assign[i] = 0;
    similarity[i] = 0;
  }
  for (int c = 0; c < k; c++) sizes[c] = 0;
  *iterations = 0;
  std::vector<float> sim((size_t)(n * k)), sums((size_t)k * d);
  std::vector<int32_t> na((size_t)n);
  for (int it = 1; it <= iters; it++) {
    *iterations = it;
    orc_sim_argmax(x, n, cs.data(), k, d, sim.data(), na.data());
    i64 changed = 0;
    for (i64 i = 0; i < n; i++) {
      similarity[i] = sim[(size_t)(i * k + na[i])];
      if (na[i] != assign[i]) changed++;
      assign[i] = na[i];
    }
    std::fill(sums.begin(), sums.end(), 0.0f);
    for (int c = 0; c < k; c++) sizes[c] = 0;
    for (i64 i = 0; i < n; i++) {
      const int a = assign[i];
      sizes[a]++;
      float* acc = sums.data() + (size_t)a * d;
      for (int j = 0; j < d; j++) acc[j] += x[i * d + j];
    }
    for (int c = 0; c < k; c++) {
      if (sizes[c] != 0) continue;
      i64 worst = 0;  // empty centre: restart on the worst-fitting row
      for (i64 i = 0; i < n; i++)
        if (similarity[i] < similarity[worst]) worst = i;
      std::memcpy(sums.data() + (size_t)c * d, x + worst * d, sizeof(float) * d);
      similarity[worst] = 1;
    }
    orc_normalize_rows(sums.data(), k, d, cs.data());
    if (changed == 0 && it > 1) break;
  }
  std::memcpy(centres_out, cs.data(), sizeof(float) * cs.size());
  return 0;
}

// ---------------------------------------------------------------------------
// EmbeddingGemma 2 text tower (models/gemma: config.go:247-362, model.go:
// 105-205, embed.go:247-377, 408-429).
// ---------------------------------------------------------------------------
struct Orc2Layer {
  int D = 0, Hkv = 0;
  bool sliding = true;
  float scalar = 1;
  std::vector<float> wq, wk, wv, wo, wgate, wup, wdown, pleGate, pleProj;  // [in, out]
  std::vector<float> inputNorm, postAttnNorm, preFFNNorm, postFFNNorm, qNorm, kNorm, plePostNorm;  // gains as is
  std::vector<float> raw_wq, raw_wk, raw_wv, raw_wgate, raw_wup;
};

struct OrcModel2 {
  int hidden = 0, layers = 0, heads = 0, ffn = 0, vocab = 0, radius = 0, P = 0, E = 0, n_dense = 0;
  double rope_local = 1e4, rope_theta = 1e6;
  float eps = 1e-6f;
  std::vector<Orc2Layer> L;
  std::vector<float> embed, norm, pleProj, pleNorm, embProj;  // pleProj [hidden, layers*P], embProj [hidden, E]
  std::vector<std::vector<float>> dense;
  std::vector<int> dense_in, dense_out;
  std::map<std::string, int> seen;
  bool finalized = false;
};

ORC_API void* orc_model2_create(int hidden, int layers, int heads, int ffn, int vocab, int radius, int ple_dim,
                                int embedding_dim, double rope_local, double rope_theta, float eps,
                                const int* layer_head_dim, const int* layer_kv_heads, const int* layer_sliding,
                                int n_dense, const int* dense_out) {
  if (n_dense < 0 || n_dense > 4 || layers <= 0) return nullptr;
  OrcModel2* m = new OrcModel2();
  m->hidden = hidden; m->layers = layers; m->heads = heads; m->ffn = ffn; m->vocab = vocab; m->radius = radius;
  m->P = ple_dim; m->E = embedding_dim; m->rope_local = rope_local; m->rope_theta = rope_theta; m->eps = eps;
  m->n_dense = n_dense;
  m->L.resize(layers);
  for (int l = 0; l < layers; l++) {
    m->L[l].D = layer_head_dim[l];
    m->L[l].Hkv = layer_kv_heads[l];
    m->L[l].sliding = layer_sliding[l] != 0;
  }
  int in = embedding_dim;
  m->dense.resize(n_dense);
  for (int i = 0; i < n_dense; i++) {
    m->dense_in.push_back(in);
    m->dense_out.push_back(dense_out[i]);
    in = dense_out[i];
  }
  return m;
}

ORC_API void orc_model2_destroy(void* p) { delete (OrcModel2*)p; }

// model.go:142-205 with Variant 2's loaders: norms keep their gains
// (model.go:128-140), per-layer geometry from the layer's head_dim and
// key/value heads, "layer_scalar" one value (model.go:183-190).
ORC_API int orc_model2_set(void* p, const char* name, const float* data, i64 numel) {
  OrcModel2* m = (OrcModel2*)p;
  const std::string s(name);
  const int d = m->hidden, H = m->heads, F = m->ffn, P = m->P;
  auto gain = [&](std::vector<float>& dst, i64 n) {
    if (numel != n) return -2;
    dst.assign(data, data + n);
    return 0;
  };
  auto mat = [&](std::vector<float>& dst, int out, int in) {
    if (numel != (i64)out * in) return -2;
    dst = transpose_w(data, out, in);
    return 0;
  };
  int rc = 0;
  if (s == "embed_tokens.weight") {
    if (numel != (i64)m->vocab * d) return -2;
    m->embed.assign(data, data + numel);
  } else if (s == "norm.weight") {
    rc = gain(m->norm, d);
  } else if (s == "ple.per_layer_model_projection.weight") {
    rc = mat(m->pleProj, m->layers * P, d);
  } else if (s == "ple.per_layer_projection_norm.weight") {
    rc = gain(m->pleNorm, P);
  } else if (s == "embedding_projection.weight") {
    rc = mat(m->embProj, m->E, d);
  } else if (s.rfind("dense.", 0) == 0) {
    int i = std::atoi(s.c_str() + 6);
    if (i < 0 || i >= m->n_dense) return -3;
    rc = mat(m->dense[i], m->dense_out[i], m->dense_in[i]);
  } else if (s.rfind("layers.", 0) == 0) {
    int l = std::atoi(s.c_str() + 7);
    if (l < 0 || l >= m->layers) return -3;
    const std::string rest = s.substr(s.find('.', 7) + 1);
    Orc2Layer& Y = m->L[l];
    const int D = Y.D, Hkv = Y.Hkv;
    if (rest == "input_layernorm.weight") rc = gain(Y.inputNorm, d);
    else if (rest == "post_attention_layernorm.weight") rc = gain(Y.postAttnNorm, d);
    else if (rest == "pre_feedforward_layernorm.weight") rc = gain(Y.preFFNNorm, d);
    else if (rest == "post_feedforward_layernorm.weight") rc = gain(Y.postFFNNorm, d);
    else if (rest == "self_attn.q_norm.weight") rc = gain(Y.qNorm, D);
    else if (rest == "self_attn.k_norm.weight") rc = gain(Y.kNorm, D);
    else if (rest == "self_attn.q_proj.weight") rc = mat(Y.raw_wq, H * D, d);
    else if (rest == "self_attn.k_proj.weight") rc = mat(Y.raw_wk, Hkv * D, d);
    else if (rest == "self_attn.v_proj.weight") rc = mat(Y.raw_wv, Hkv * D, d);
    else if (rest == "self_attn.o_proj.weight") rc = mat(Y.wo, d, H * D);
    else if (rest == "mlp.gate_proj.weight") rc = mat(Y.raw_wgate, F, d);
    else if (rest == "mlp.up_proj.weight") rc = mat(Y.raw_wup, F, d);
    else if (rest == "mlp.down_proj.weight") rc = mat(Y.wdown, d, F);
    else if (rest == "ple_block.per_layer_input_gate.weight") rc = mat(Y.pleGate, P, d);
    else if (rest == "ple_block.per_layer_projection.weight") rc = mat(Y.pleProj, d, P);
    else if (rest == "ple_block.post_per_layer_input_norm.weight") rc = gain(Y.plePostNorm, d);
    else if (rest == "layer_scalar") {
      if (numel != 1) return -2;
      Y.scalar = data[0];
    } else return -3;
  } else {
    return -3;
  }
  if (rc) return rc;
  m->seen[s]++;
  return 0;
}

// Pre-norm gains folded into the weights they feed (model.go:206-222).
ORC_API int orc_model2_finalize(void* p) {
  OrcModel2* m = (OrcModel2*)p;
  const int expected = 5 + m->n_dense + 17 * m->layers;
  if ((int)m->seen.size() != expected) return -4;
  const int d = m->hidden, H = m->heads, F = m->ffn;
  for (auto& Y : m->L) {
    Y.wq = fold(Y.raw_wq, Y.inputNorm, d, H * Y.D);
    Y.wk = fold(Y.raw_wk, Y.inputNorm, d, Y.Hkv * Y.D);
    Y.wv = fold(Y.raw_wv, Y.inputNorm, d, Y.Hkv * Y.D);
    Y.wgate = fold(Y.raw_wgate, Y.preFFNNorm, d, F);
    Y.wup = fold(Y.raw_wup, Y.preFFNNorm, d, F);
    std::vector<float>().swap(Y.raw_wq);
    std::vector<float>().swap(Y.raw_wk);
    std::vector<float>().swap(Y.raw_wv);
    std::vector<float>().swap(Y.raw_wgate);
    std::vector<float>().swap(Y.raw_wup);
  }
  m->finalized = true;
  return 0;
}

// encode2 + encode2From (embed.go:247-377), pool (embed.go:381-404) and
// applyHead with the embedding projection (embed.go:408-429). hidden_out
// (optional) receives the final normed hidden states [B, T, hidden].
ORC_API int orc_model2_embed(void* p, const int32_t* ids, const int32_t* lengths, int B, int T, int dim, float* out,
                             float* hidden_out) {
  OrcModel2* m = (OrcModel2*)p;
  if (!m->finalized) return -5;
  const int d = m->hidden, H = m->heads, F = m->ffn, P = m->P, NL = m->layers;
  const i64 M = (i64)B * T;
  const float eps = m->eps;
  int full = m->E;
  if (m->n_dense > 0) full = m->dense_out[m->n_dense - 1];
  if (dim <= 0) dim = full;
  if (dim > full) return -6;
  for (i64 i = 0; i < M; i++)
    if (ids[i] < 0 || ids[i] >= m->vocab) return -7;
  std::vector<int32_t> positions(T);
  for (int t = 0; t < T; t++) positions[t] = t;
  const int w = m->radius + 1;                       // config.go:331-335
  const bool use_window = m->radius > 0 && T > w;    // embed.go:268-271

  const float sq = (float)std::sqrt((double)d);
  std::vector<float> x((size_t)M * d);
#pragma omp parallel for schedule(static)
  for (i64 r = 0; r < M; r++) {
    const float* e = &m->embed[(size_t)ids[r] * d];
    for (int i = 0; i < d; i++) x[(size_t)r * d + i] = e[i] * sq;
  }
  // per-layer inputs (embed.go:274-279)
  std::vector<float> pl((size_t)M * NL * P), ple((size_t)M * NL * P);
  orc_gemm(M, NL * P, d, x.data(), d, m->pleProj.data(), NL * P, pl.data(), NL * P, nullptr, nullptr, 0, nullptr, 0,
           nullptr, 0);
  const float inv_sqrt_d = (float)(1 / std::sqrt((double)d));
#pragma omp parallel for schedule(static)
  for (i64 i = 0; i < M * NL * P; i++) pl[i] = pl[i] * inv_sqrt_d;
  orc_rmsnorm(pl.data(), m->pleNorm.data(), eps, M * NL, P, ple.data());

  std::vector<float> padm((size_t)B * T), winm, mask_sl;
  orc_padding_mask(lengths, B, T, padm.data());
  if (use_window) {
    winm.resize((size_t)T * T);
    orc_window_mask(T, w, winm.data());
    mask_sl.resize((size_t)B * T * T);
    for (int b = 0; b < B; b++)
      for (int i = 0; i < T; i++)
        for (int j = 0; j < T; j++)
          mask_sl[((size_t)b * T + i) * T + j] = padm[(size_t)b * T + j] + winm[(size_t)i * T + j];
  }
  std::vector<float> ss(M), sc(M), o0((size_t)M * d), o((size_t)M * d), up((size_t)M * F), gu((size_t)M * F);
  std::vector<float> pleL((size_t)M * P), g((size_t)M * P), cs, sn, tmp;
  for (int l = 0; l < NL; l++) {
    const Orc2Layer& Y = m->L[l];
    const int D = Y.D, Hkv = Y.Hkv, half = D / 2;
    std::vector<float> q0((size_t)M * H * D), k0((size_t)M * Hkv * D), v0((size_t)M * Hkv * D);
    std::vector<float> q((size_t)M * H * D), k((size_t)M * Hkv * D), v((size_t)M * Hkv * D);
    std::vector<float> qr((size_t)M * H * D), kr((size_t)M * Hkv * D), vc((size_t)M * Hkv * D);
    std::vector<float> att((size_t)M * H * D), attc((size_t)M * H * D), ones(D, 1.0f);
    orc_row_sum_squares(x.data(), M, d, d, ss.data());
    orc_rms_scale(ss.data(), M, d, eps, sc.data());
    orc_gemm(M, H * D, d, x.data(), d, Y.wq.data(), H * D, q0.data(), H * D, nullptr, sc.data(), 0, nullptr, 0, nullptr, 0);
    orc_gemm(M, Hkv * D, d, x.data(), d, Y.wk.data(), Hkv * D, k0.data(), Hkv * D, nullptr, sc.data(), 0, nullptr, 0, nullptr, 0);
    orc_gemm(M, Hkv * D, d, x.data(), d, Y.wv.data(), Hkv * D, v0.data(), Hkv * D, nullptr, sc.data(), 0, nullptr, 0, nullptr, 0);
    orc_rmsnorm(q0.data(), Y.qNorm.data(), eps, M * H, D, q.data());
    orc_rmsnorm(k0.data(), Y.kNorm.data(), eps, M * Hkv, D, k.data());
    orc_rmsnorm(v0.data(), ones.data(), eps, M * Hkv, D, v.data());  // v_norm: no weight (model.go:189)
    const double base = Y.sliding ? (m->rope_local != 0 ? m->rope_local : 10000.0)
                                  : (m->rope_theta != 0 ? m->rope_theta : 10000.0);  // config.go:346-351
    rope_tables(base, positions.data(), T, D, cs, sn);
#pragma omp parallel for schedule(static)
    for (i64 r = 0; r < M; r++) {
      const int b = (int)(r / T), t = (int)(r % T);
      for (int h = 0; h < H; h++)
        rope_row(&q[((size_t)r * H + h) * D], &qr[(((size_t)b * H + h) * T + t) * D], &cs[(size_t)t * half],
                 &sn[(size_t)t * half], D);
      for (int h = 0; h < Hkv; h++) {
        rope_row(&k[((size_t)r * Hkv + h) * D], &kr[(((size_t)b * Hkv + h) * T + t) * D], &cs[(size_t)t * half],
                 &sn[(size_t)t * half], D);
        std::memcpy(&vc[(((size_t)b * Hkv + h) * T + t) * D], &v[((size_t)r * Hkv + h) * D], sizeof(float) * D);
      }
    }
    // grouped-query attention, query head h reads key/value head h/rep,
    // score scale 1 (model.go:105-110)
    const bool sl = use_window && Y.sliding;
    const int grp = H / Hkv;
    const float* mk = sl ? mask_sl.data() : padm.data();
    const i64 msb = sl ? (i64)T * T : T, msr = sl ? T : 0;
    tmp.resize((size_t)B * grp * T * D);
    for (int hk = 0; hk < Hkv; hk++) {
      orc_attention(&qr[(size_t)hk * grp * T * D], &kr[(size_t)hk * T * D], &vc[(size_t)hk * T * D], B, grp, T, T, D,
                    (i64)H * T * D, (i64)T * D, (i64)Hkv * T * D, 0, (i64)Hkv * T * D, 0, mk, msb, 0, msr, 1, 1.0f,
                    tmp.data());
      for (int b = 0; b < B; b++)
        for (int gg = 0; gg < grp; gg++)
          std::memcpy(&att[(((size_t)b * H + hk * grp + gg) * T) * D], &tmp[(((size_t)b * grp + gg) * T) * D],
                      sizeof(float) * T * D);
    }
#pragma omp parallel for schedule(static)
    for (i64 r = 0; r < M; r++) {
      const int b = (int)(r / T), t = (int)(r % T);
      for (int h = 0; h < H; h++)
        std::memcpy(&attc[((size_t)r * H + h) * D], &att[(((size_t)b * H + h) * T + t) * D], sizeof(float) * D);
    }
    orc_gemm(M, d, H * D, attc.data(), H * D, Y.wo.data(), d, o0.data(), d, nullptr, nullptr, 0, nullptr, 0, nullptr, 0);
    orc_rmsnorm(o0.data(), Y.postAttnNorm.data(), eps, M, d, o.data());
#pragma omp parallel for schedule(static)
    for (i64 i = 0; i < M * d; i++) x[i] = x[i] + o[i];
    // feed-forward (embed.go:344-357)
    orc_row_sum_squares(x.data(), M, d, d, ss.data());
    orc_rms_scale(ss.data(), M, d, eps, sc.data());
    orc_gemm(M, F, d, x.data(), d, Y.wup.data(), F, up.data(), F, nullptr, sc.data(), 0, nullptr, 0, nullptr, 0);
    orc_gemm(M, F, d, x.data(), d, Y.wgate.data(), F, gu.data(), F, nullptr, sc.data(), ORC_ACT_GELU, up.data(), F,
             nullptr, 0);
    orc_gemm(M, d, F, gu.data(), F, Y.wdown.data(), d, o0.data(), d, nullptr, nullptr, 0, nullptr, 0, nullptr, 0);
    orc_rmsnorm(o0.data(), Y.postFFNNorm.data(), eps, M, d, o.data());
#pragma omp parallel for schedule(static)
    for (i64 i = 0; i < M * d; i++) x[i] = x[i] + o[i];
    // per-layer-input block and layer scalar (embed.go:359-371)
#pragma omp parallel for schedule(static)
    for (i64 r = 0; r < M; r++) std::memcpy(&pleL[(size_t)r * P], &ple[((size_t)r * NL + l) * P], sizeof(float) * P);
    orc_gemm(M, P, d, x.data(), d, Y.pleGate.data(), P, g.data(), P, nullptr, nullptr, ORC_ACT_GELU, pleL.data(), P,
             nullptr, 0);
    orc_gemm(M, d, P, g.data(), P, Y.pleProj.data(), d, o0.data(), d, nullptr, nullptr, 0, nullptr, 0, nullptr, 0);
    orc_rmsnorm(o0.data(), Y.plePostNorm.data(), eps, M, d, o.data());
#pragma omp parallel for schedule(static)
    for (i64 i = 0; i < M * d; i++) {
      const float x4 = x[i] + o[i];
      x[i] = x4 * Y.scalar;
    }
  }
  std::vector<float> h((size_t)M * d);
  orc_rmsnorm(x.data(), m->norm.data(), eps, M, d, h.data());
  if (hidden_out) std::memcpy(hidden_out, h.data(), sizeof(float) * h.size());
  std::vector<float> pooled((size_t)B * d, 0.f);
  for (int b = 0; b < B; b++) {
    int n = lengths[b];
    if (n == 0) n = 1;
    float* dst = &pooled[(size_t)b * d];
    for (int t = 0; t < n; t++) {
      const float* row = &h[((size_t)b * T + t) * d];
      for (int i = 0; i < d; i++) dst[i] += row[i];
    }
    const float inv = 1.f / (float)n;
    for (int i = 0; i < d; i++) dst[i] *= inv;
  }
  std::vector<float> y((size_t)B * m->E), y2;
  orc_gemm(B, m->E, d, pooled.data(), d, m->embProj.data(), m->E, y.data(), m->E, nullptr, nullptr, 0, nullptr, 0,
           nullptr, 0);
  int cur = m->E;
  for (int i = 0; i < m->n_dense; i++) {
    const int no = m->dense_out[i];
    y2.assign((size_t)B * no, 0.f);
    orc_gemm(B, no, cur, y.data(), cur, m->dense[i].data(), no, y2.data(), no, nullptr, nullptr, 0, nullptr, 0, nullptr,
             0);
    y.swap(y2);
    cur = no;
  }
  for (int b = 0; b < B; b++) {
    const float* yr = &y[(size_t)b * cur];
    std::vector<float> sq2(dim);
    for (int i = 0; i < dim; i++) sq2[i] = yr[i] * yr[i];
    const float s = orc_sumf(sq2.data(), dim);
    const float nrm = std::sqrt(s + 1e-12f);
    for (int i = 0; i < dim; i++) out[(size_t)b * dim + i] = yr[i] / nrm;
  }
  return 0;
}
