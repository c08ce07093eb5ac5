// tensor.MatMul on strided and batched operands (fa_matmul_strided[_dev]):
// the general case of the reference's MatMul (tensor/matmul.go:19-127) and
// of MatMulFused on strided views (tensor/matmul_fused.go:40-96).
//
// Route: the right operand is rewritten, per batch entry, into three bf16
// planes hi + mid + lo of [n][kp] (kp = k rounded up to 32, zero columns past
// k) read through its strides by split_b_view_kernel, which is what the
// reference's PackB does for its micro-kernel (internal/blas/gemm.go:395-416);
// the left operand is used in place when it is row-major with 16-byte aligned
// rows, k % 32 == 0 and equally spaced batch entries, else packed to
// [nb][m][kp] by pack_a_kernel (the reference's packA, gemm.go:815-850). The
// product is the six-term split-bf16 kernel with the batch entries on grid.z.
#include <algorithm>
#include <cstring>

#include "fa_internal.h"

using fa::set_error;

namespace fa {
namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// Largest element offset a view reaches (its extent - 1), or -1 when empty.
int64_t view_last(int nbatch, const int64_t* batch, const fa_matrix& v, int64_t rows, int64_t cols) {
  if (rows == 0 || cols == 0) return -1;
  int64_t last = (rows - 1) * v.rs + (cols - 1) * v.cs;
  for (int d = 0; d < nbatch; d++) {
    if (batch[d] == 0) return -1;
    last += (batch[d] - 1) * v.bstride[d];
  }
  return last;
}

// Whether the batch entries of v are equally spaced (entry z at z * *step),
// true for a single entry.
bool uniform_batch(int nbatch, const int64_t* batch, const fa_matrix& v, int64_t* step) {
  int64_t s = -1, span = 1;  // s: the step of the innermost dimension of size > 1
  for (int d = nbatch - 1; d >= 0; d--) {
    if (batch[d] == 1) continue;
    if (s < 0) s = v.bstride[d];
    else if (v.bstride[d] != s * span) return false;
    span *= batch[d];
  }
  *step = s < 0 ? 0 : s;
  return true;
}

BatchMap batch_map(int nbatch, const int64_t* batch, const fa_matrix& v) {
  BatchMap bm;
  bm.nd = nbatch;
  for (int d = 0; d < nbatch; d++) {
    bm.dim[d] = (int)batch[d];
    bm.stride[d] = v.bstride[d];
  }
  return bm;
}

int check_args(fa_ctx* ctx, int32_t nbatch, const int64_t* batch, int64_t m, int64_t n, int64_t k,
               const fa_matrix* a, const fa_matrix* b, const fa_epilogue* e, int64_t* nb) {
  const char* op = e ? "MatMulFused" : "MatMul";
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "%s: ctx is NULL", op);
  if (nbatch < 0 || nbatch > FA_MAX_BATCH_DIMS)
    return set_error(ctx, FA_ERR_ARG, "%s: %d batch dimensions (0..%d)", op, nbatch, FA_MAX_BATCH_DIMS);
  if (nbatch > 0 && !batch) return set_error(ctx, FA_ERR_ARG, "%s: batch shape is NULL", op);
  if (e && nbatch > 0) return set_error(ctx, FA_ERR_ARG, "MatMulFused: expected 2-D operands, got %d batch dimensions", nbatch);
  if (m < 0 || n < 0 || k < 0)
    return set_error(ctx, FA_ERR_ARG, "%s: negative size [%lld x %lld] . [%lld x %lld]", op, (long long)m,
                     (long long)k, (long long)k, (long long)n);
  if (!a || !b) return set_error(ctx, FA_ERR_ARG, "%s: operand is NULL", op);
  int64_t entries = 1;
  for (int d = 0; d < nbatch; d++) {
    if (batch[d] < 0) return set_error(ctx, FA_ERR_ARG, "%s: negative batch dimension %lld", op, (long long)batch[d]);
    if (batch[d] > INT32_MAX) return set_error(ctx, FA_ERR_ARG, "%s: batch dimension %lld", op, (long long)batch[d]);
    entries *= batch[d];
    if (entries > INT32_MAX) return set_error(ctx, FA_ERR_ARG, "%s: more than 2^31 batch entries", op);
  }
  for (const fa_matrix* v : {a, b}) {
    if (v->rs < 0 || v->cs < 0) return set_error(ctx, FA_ERR_ARG, "%s: negative stride", op);
    for (int d = 0; d < nbatch; d++)
      if (v->bstride[d] < 0) return set_error(ctx, FA_ERR_ARG, "%s: negative batch stride", op);
  }
  if (e) {
    if (e->act < FA_ACT_NONE || e->act > FA_ACT_TANH)
      return set_error(ctx, FA_ERR_ARG, "MatMulFused: unknown activation %d", e->act);
    if (e->mul && e->ldm < n) return set_error(ctx, FA_ERR_ARG, "MatMulFused: Mul leading dimension < n");
    if (e->residual && e->ldr < n) return set_error(ctx, FA_ERR_ARG, "MatMulFused: Residual leading dimension < n");
  }
  if (n >= (1LL << 26)) return set_error(ctx, FA_ERR_ARG, "%s: n %lld above 2^26", op, (long long)n);
  *nb = entries;
  return FA_OK;
}

// out = epilogue(A . B) for device operands, enqueued on ctx's stream.
int matmul_strided(fa_ctx* ctx, int32_t nbatch, const int64_t* batch, int64_t nb, int64_t m, int64_t n, int64_t k,
                   const fa_matrix& a, const fa_matrix& b, const fa_epilogue* e, float* out) {
  if (nb == 0 || m == 0 || n == 0) return FA_OK;
  const int64_t kp = std::max<int64_t>(32, (k + 31) / 32 * 32);
  int64_t astep = 0;
  const bool a_direct = k > 0 && k % 32 == 0 && (a.cs == 1 || k == 1) && (a.rs >= k || m == 1) &&
                        aligned16(a.data) && (m == 1 || a.rs % 4 == 0) &&
                        uniform_batch(nbatch, batch, a, &astep) && astep % 4 == 0;
  const BatchMap bma = batch_map(nbatch, batch, a), bmb = batch_map(nbatch, batch, b);
  // entries per pass: the planes (and a packed A) of a pass stay below 256 MiB
  const int64_t per = 6 * n * kp + (a_direct ? 0 : 4 * m * kp);
  const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>({(int64_t)kMaxGridZ, nb, (256LL << 20) / per}));
  DevBuf& planes = ctx->slot(slots::S_BPLANES);
  int rc;
  if ((rc = planes.ensure(ctx, (size_t)(chunk * 6 * n * kp)))) return rc;
  if (!a_direct && (rc = ctx->slot(slots::S_APACK).ensure(ctx, (size_t)(chunk * 4 * m * kp)))) return rc;
  for (int64_t z0 = 0; z0 < nb; z0 += chunk) {
    const int64_t cnt = std::min(chunk, nb - z0);
    GemmArgs g;
    g.m = m; g.n = n; g.k = kp;
    g.b = planes.ptr; g.ldb = kp; g.b_dtype = FA_DT_BF16; g.b_layout = FA_B_NK;
    g.b_terms = 3; g.b_plane = n * kp; g.b_bs = 3 * n * kp;
    g.c = out + z0 * m * n; g.ldc = n; g.c_bs = m * n;
    g.nbatch = cnt;
    if ((rc = launch_split_b_view(ctx, b.data, bmb, (int)z0, b.rs, b.cs, cnt, n, k, kp, planes.as<uint16_t>(),
                                  ctx->stream)))
      return rc;
    if (a_direct) {
      g.a = a.data + z0 * astep; g.lda = m == 1 ? kp : a.rs; g.a_bs = astep;
    } else {
      float* pa = ctx->slot(slots::S_APACK).as<float>();
      if ((rc = launch_pack_a(ctx, a.data, bma, (int)z0, a.rs, a.cs, cnt, m, k, kp, pa, ctx->stream))) return rc;
      g.a = pa; g.lda = kp; g.a_bs = m * kp;
    }
    if (e && (e->bias || e->row_scale || e->act != FA_ACT_NONE || e->mul || e->residual)) {
      g.epi = Epi::Generic;
      g.bias = e->bias; g.row_scale = e->row_scale; g.act = e->act;
      g.mul = e->mul; g.ldm = e->ldm; g.residual = e->residual; g.ldr = e->ldr;
    }
    if ((rc = launch_gemm(ctx, g, ctx->stream))) return rc;
  }
  return FA_OK;
}

}  // namespace
}  // namespace fa

using namespace fa::slots;

extern "C" {

int fa_matmul_strided_dev(fa_ctx* ctx, int32_t nbatch, const int64_t* batch, int64_t m, int64_t n, int64_t k,
                          const fa_matrix* a, const fa_matrix* b, const fa_epilogue* e, float* out) {
  int64_t nb = 0;
  int rc = fa::check_args(ctx, nbatch, batch, m, n, k, a, b, e, &nb);
  if (rc) return rc;
  if ((rc = fa::refuse_capture(ctx, ctx->stream, e ? "MatMulFused" : "MatMul"))) return rc;
  if (nb == 0 || m == 0 || n == 0) return FA_OK;
  if ((k > 0 && (!a->data || !b->data)) || !out) return set_error(ctx, FA_ERR_ARG, "MatMul: NULL data pointer");
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  return fa::matmul_strided(ctx, nbatch, batch, nb, m, n, k, *a, *b, e, out);
}

int fa_matmul_strided(fa_ctx* ctx, int32_t nbatch, const int64_t* batch, int64_t m, int64_t n, int64_t k,
                      const fa_matrix* a, const fa_matrix* b, const fa_epilogue* e, float* out) {
  int64_t nb = 0;
  int rc = fa::check_args(ctx, nbatch, batch, m, n, k, a, b, e, &nb);
  if (rc) return rc;
  if ((rc = fa::refuse_capture(ctx, ctx->stream, e ? "MatMulFused" : "MatMul"))) return rc;
  if (nb == 0 || m == 0 || n == 0) return FA_OK;
  if ((k > 0 && (!a->data || !b->data)) || !out) return set_error(ctx, FA_ERR_ARG, "MatMul: NULL data pointer");
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  // the host storage each view reaches, copied as it lies
  const int64_t alast = fa::view_last(nbatch, batch, *a, m, k), blast = fa::view_last(nbatch, batch, *b, k, n);
  void *da = nullptr, *db = nullptr, *p = nullptr;
  if ((rc = fa::stage_h2d(ctx, S_A, a->data, (size_t)(alast + 1) * 4, &da))) return rc;
  if ((rc = fa::stage_h2d(ctx, S_B, b->data, (size_t)(blast + 1) * 4, &db))) return rc;
  fa_matrix av = *a, bv = *b;
  av.data = (const float*)da;
  bv.data = (const float*)db;
  const size_t obytes = (size_t)(nb * m * n) * 4;
  if ((rc = ctx->slot(S_C).ensure(ctx, obytes))) return rc;
  fa_epilogue de{};
  if (e) {
    de = *e;
    if (e->bias) { if ((rc = fa::stage_h2d(ctx, S_BIAS, e->bias, (size_t)n * 4, &p))) return rc; de.bias = (const float*)p; }
    if (e->row_scale) { if ((rc = fa::stage_h2d(ctx, S_ROWSCALE, e->row_scale, (size_t)m * 4, &p))) return rc; de.row_scale = (const float*)p; }
    if (e->mul) { if ((rc = fa::stage_h2d(ctx, S_MUL, e->mul, (size_t)((m - 1) * e->ldm + n) * 4, &p))) return rc; de.mul = (const float*)p; }
    if (e->residual) { if ((rc = fa::stage_h2d(ctx, S_RES, e->residual, (size_t)((m - 1) * e->ldr + n) * 4, &p))) return rc; de.residual = (const float*)p; }
  }
  if ((rc = fa::matmul_strided(ctx, nbatch, batch, nb, m, n, k, av, bv, e ? &de : nullptr, ctx->slot(S_C).as<float>())))
    return rc;
  FA_HIP_CHECK(ctx, hipMemcpyAsync(out, ctx->slot(S_C).ptr, obytes, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

}  // extern "C"
