// Context, errors, device buffers and the tensor-level C-ABI entry points
// (host pointers in, host pointers out).
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "fa_internal.h"

namespace fa {

namespace {
thread_local std::string tls_error;

// Live handles. A process that exits with a context or model still open
// would otherwise leave streams, events, pinned host buffers and device
// memory to the HIP runtime's own teardown, which then aborts ("terminate
// called after throwing an instance of 'std::bad_variant_access'", seen with
// a model left open). close_at_exit() is registered with atexit() on the
// first fa_create, after the runtime has initialised (and registered its
// teardown), so it runs first and releases what is still open, models
// before contexts. The containers are never destroyed (no static destructor
// runs after the handler).
std::mutex g_reg_mu;
std::vector<fa_ctx*>* g_ctxs = new std::vector<fa_ctx*>();
std::vector<std::pair<fa_model*, fa_ctx*>>* g_models = new std::vector<std::pair<fa_model*, fa_ctx*>>();
bool g_exit_hook = false;

void ctx_release(fa_ctx* ctx) {
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  for (auto& b : ctx->scratch) b.release();
  (void)hipStreamDestroy(ctx->stream);
  noalloc_release(ctx);
  delete ctx;
}

void close_at_exit() {
  std::vector<std::pair<fa_model*, fa_ctx*>> models;
  std::vector<fa_ctx*> ctxs;
  {
    std::lock_guard<std::mutex> lk(g_reg_mu);
    models.swap(*g_models);
    ctxs.swap(*g_ctxs);
  }
  for (auto it = models.rbegin(); it != models.rend(); ++it) model_release(it->first);
  for (auto it = ctxs.rbegin(); it != ctxs.rend(); ++it) ctx_release(*it);
}

// Removes x from v; whether it was there.
template <class V, class F>
bool take(V& v, F match) {
  for (size_t i = 0; i < v.size(); i++)
    if (match(v[i])) {
      v.erase(v.begin() + (long)i);
      return true;
    }
  return false;
}
}  // namespace

void register_model(fa_model* m, fa_ctx* ctx) {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  g_models->push_back({m, ctx});
}

bool unregister_model(fa_model* m) {
  std::lock_guard<std::mutex> lk(g_reg_mu);
  return take(*g_models, [m](const std::pair<fa_model*, fa_ctx*>& e) { return e.first == m; });
}

int refuse_capture(fa_ctx* ctx, hipStream_t s, const char* op) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(s, &st);
  if (e != hipSuccess) return set_error(ctx, FA_ERR_HIP, "%s: hipStreamIsCapturing: %s", op, hipGetErrorString(e));
  if (st != hipStreamCaptureStatusNone)
    return set_error(ctx, FA_ERR_STATE,
                     "%s: the context's stream is being captured into a HIP graph; this entry point may allocate "
                     "and upload per-call data and cannot be captured (fa_similarities_topk_dev_noalloc can)",
                     op);
  return FA_OK;
}

int set_error(fa_ctx* ctx, int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) ctx->last_error = buf;
  tls_error = buf;
  return code;
}

int DevBuf::ensure(fa_ctx* ctx, size_t need) {
  if (need <= bytes && ptr) return FA_OK;
  if (ptr) {
    hipError_t e = hipStreamSynchronize(ctx->stream);  // in-flight work may still read it
    if (e != hipSuccess) return set_error(ctx, FA_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
    (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
  size_t sz = need < 256 ? 256 : need;
  sz = (sz + 255) & ~size_t(255);
  hipError_t e = hipMalloc(&ptr, sz);
  if (e != hipSuccess) {
    ptr = nullptr;
    return set_error(ctx, FA_ERR_OOM, "hipMalloc(%zu): %s", sz, hipGetErrorString(e));
  }
  bytes = sz;
  return FA_OK;
}

void DevBuf::release() {
  if (ptr) (void)hipFree(ptr);
  ptr = nullptr;
  bytes = 0;
}

int stage_h2d(fa_ctx* ctx, size_t slot, const void* src, size_t bytes, void** out) {
  DevBuf& b = ctx->slot(slot);
  int rc = b.ensure(ctx, bytes);
  if (rc) return rc;
  if (bytes) FA_HIP_CHECK(ctx, hipMemcpyAsync(b.ptr, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  *out = b.ptr;
  return FA_OK;
}

// float64 angle tables rounded to float32 (tensor/rope.go:36-50).
void rope_tables_host(double base, const int32_t* positions, int T, int D, std::vector<float>& cs,
                      std::vector<float>& sn) {
  const int half = D / 2;
  std::vector<double> inv(half);
  for (int i = 0; i < half; i++) inv[i] = std::pow(base, -(double)(2 * i) / (double)D);
  cs.resize((size_t)T * half);
  sn.resize((size_t)T * half);
  for (int t = 0; t < T; t++) {
    const double p = (double)positions[t];
    for (int i = 0; i < half; i++) {
      const double a = p * inv[i];
      cs[(size_t)t * half + i] = (float)std::cos(a);
      sn[(size_t)t * half + i] = (float)std::sin(a);
    }
  }
}

}  // namespace fa

using fa::set_error;

using namespace fa::slots;

extern "C" {

const char* fa_version(void) { return "fa_rocm 0.1 gfx950"; }

int fa_create(int device, fa_ctx** out) {
  if (!out) return set_error(nullptr, FA_ERR_ARG, "fa_create: out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return set_error(nullptr, FA_ERR_HIP, "hipGetDeviceCount: %s", hipGetErrorString(e));
  if (device < 0 || device >= n)
    return set_error(nullptr, FA_ERR_ARG, "fa_create: device %d outside 0..%d", device, n - 1);
  e = hipSetDevice(device);
  if (e != hipSuccess) return set_error(nullptr, FA_ERR_HIP, "hipSetDevice: %s", hipGetErrorString(e));
  fa_ctx* c = new fa_ctx();
  c->device = device;
  e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return set_error(nullptr, FA_ERR_HIP, "hipStreamCreate: %s", hipGetErrorString(e));
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) c->cu_count = prop.multiProcessorCount;
  const int rc = fa::noalloc_scratch_init(c);
  if (rc) {
    std::string msg = c->last_error;
    (void)hipStreamDestroy(c->stream);
    delete c;
    return set_error(nullptr, rc, "%s", msg.c_str());
  }
  {
    std::lock_guard<std::mutex> lk(fa::g_reg_mu);
    fa::g_ctxs->push_back(c);
    if (!fa::g_exit_hook) fa::g_exit_hook = std::atexit(fa::close_at_exit) == 0;
  }
  *out = c;
  return FA_OK;
}

void fa_destroy(fa_ctx* ctx) {
  if (!ctx) return;
  std::vector<std::pair<fa_model*, fa_ctx*>> models;
  {
    std::lock_guard<std::mutex> lk(fa::g_reg_mu);
    // unknown, or already closed at exit: nothing to do
    if (!fa::take(*fa::g_ctxs, [ctx](fa_ctx* c) { return c == ctx; })) return;
    // models still open on this context go first (they use its stream)
    for (size_t i = 0; i < fa::g_models->size();)
      if ((*fa::g_models)[i].second == ctx) {
        models.push_back((*fa::g_models)[i]);
        fa::g_models->erase(fa::g_models->begin() + (long)i);
      } else {
        i++;
      }
  }
  for (auto& e : models) fa::model_release(e.first);
  fa::ctx_release(ctx);
}

const char* fa_last_error(const fa_ctx* ctx) {
  if (ctx) return ctx->last_error.c_str();
  return fa::tls_error.c_str();
}

void* fa_stream(fa_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int fa_sync(fa_ctx* ctx) {
  if (!ctx) return set_error(nullptr, FA_ERR_ARG, "fa_sync: ctx is NULL");
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

int fa_device_alloc(fa_ctx* ctx, size_t bytes, void** out) {
  if (!ctx || !out) return set_error(ctx, FA_ERR_ARG, "fa_device_alloc: NULL argument");
  hipError_t e = hipMalloc(out, bytes ? bytes : 1);
  if (e != hipSuccess) return set_error(ctx, FA_ERR_OOM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  return FA_OK;
}

int fa_device_free(fa_ctx* ctx, void* ptr) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "fa_device_free: ctx is NULL");
  if (!ptr) return FA_OK;
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  FA_HIP_CHECK(ctx, hipFree(ptr));
  return FA_OK;
}

int fa_memcpy_h2d(fa_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "fa_memcpy_h2d: ctx is NULL");
  FA_HIP_CHECK(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

int fa_memcpy_d2h(fa_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "fa_memcpy_d2h: ctx is NULL");
  FA_HIP_CHECK(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

namespace fa {
namespace {

// The split-bf16 products need B as bf16 [n x k] rows, A's rows 16-byte
// aligned and k a whole number of 32-wide slabs. Other B operands (fp32,
// tensor.MatMul's [k x n] weights, matmul.go:42-72) are rewritten into that
// form in scratch first: fp32 as three planes hi + mid + lo (exact, the
// six-term product), bf16 [k x n] transposed. Shapes the fast kernels cannot
// take keep the fp32-MFMA kernel with its checked loader.
int prepare_b(fa_ctx* ctx, GemmArgs& g) {
  const bool a_ok = (reinterpret_cast<uintptr_t>(g.a) & 15) == 0 && g.lda % 4 == 0;
  if (!(g.k > 0 && g.k % 32 == 0 && a_ok) || gemm_f32_mfma_forced()) return FA_OK;
  if (g.b_dtype == FA_DT_BF16 && g.b_layout == FA_B_NK) return FA_OK;  // already the fast form (when aligned)
  const int terms = g.b_dtype == FA_DT_F32 ? 3 : 1;
  DevBuf& pb = ctx->slot(slots::S_BPLANES);
  int rc;
  if ((rc = pb.ensure(ctx, (size_t)terms * g.n * g.k * 2))) return rc;
  if ((rc = launch_split_b(ctx, g.b, g.b_dtype, g.ldb, g.b_layout, g.n, g.k, pb.as<uint16_t>(), ctx->stream)))
    return rc;
  g.b = pb.ptr;
  g.b_dtype = FA_DT_BF16;
  g.b_layout = FA_B_NK;
  g.ldb = g.k;
  g.b_terms = terms;
  g.b_plane = g.n * g.k;
  return FA_OK;
}

}  // namespace
}  // namespace fa

int fa_matmul_fused(fa_ctx* ctx, int64_t m, int64_t n, int64_t k, const float* a, int64_t lda, const void* b,
                    int64_t ldb, int b_dtype, int b_layout, const fa_epilogue* e, float* c, int64_t ldc) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "MatMulFused: ctx is NULL");
  if (m < 0 || n < 0 || k < 0)
    return set_error(ctx, FA_ERR_ARG, "MatMulFused: negative size [%lld x %lld] . [%lld x %lld]", (long long)m,
                     (long long)k, (long long)k, (long long)n);
  if (b_dtype != FA_DT_F32 && b_dtype != FA_DT_BF16)
    return set_error(ctx, FA_ERR_ARG, "MatMulFused: unknown B dtype %d", b_dtype);
  if (b_layout != FA_B_KN && b_layout != FA_B_NK)
    return set_error(ctx, FA_ERR_ARG, "MatMulFused: unknown B layout %d", b_layout);
  if (lda < (k > 0 ? k : 1) && m > 0)
    return set_error(ctx, FA_ERR_ARG, "MatMulFused: lda %lld < k %lld", (long long)lda, (long long)k);
  const int64_t brow = b_layout == FA_B_KN ? n : k, bcnt = b_layout == FA_B_KN ? k : n;
  if (ldb < brow && bcnt > 0)
    return set_error(ctx, FA_ERR_ARG, "MatMulFused: ldb %lld too small", (long long)ldb);
  if (ldc < n && m > 0) return set_error(ctx, FA_ERR_ARG, "MatMulFused: ldc %lld < n %lld", (long long)ldc, (long long)n);
  if (e && (e->act < FA_ACT_NONE || e->act > FA_ACT_TANH))
    return set_error(ctx, FA_ERR_ARG, "MatMulFused: unknown activation %d", e->act);
  if (e && e->mul && e->ldm < n) return set_error(ctx, FA_ERR_ARG, "MatMulFused: Mul leading dimension < n");
  if (e && e->residual && e->ldr < n)
    return set_error(ctx, FA_ERR_ARG, "MatMulFused: Residual leading dimension < n");
  if (m == 0 || n == 0) return FA_OK;
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "MatMulFused");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  const size_t esz = b_dtype == FA_DT_BF16 ? 2 : 4;
  void *da = nullptr, *db = nullptr, *dc = nullptr;
  int rc;
  const size_t abytes = (size_t)((m - 1) * lda + k) * 4;
  const size_t bbytes = bcnt > 0 ? (size_t)((bcnt - 1) * ldb + brow) * esz : 0;
  const size_t cbytes = (size_t)((m - 1) * ldc + n) * 4;
  if ((rc = fa::stage_h2d(ctx, S_A, a, k > 0 ? abytes : 0, &da))) return rc;
  if ((rc = fa::stage_h2d(ctx, S_B, b, bbytes, &db))) return rc;
  if ((rc = ctx->slot(S_C).ensure(ctx, cbytes))) return rc;
  dc = ctx->slot(S_C).ptr;
  fa::GemmArgs g;
  g.m = m; g.n = n; g.k = k;
  g.a = (const float*)da; g.lda = lda; g.b = db; g.ldb = ldb; g.b_dtype = b_dtype; g.b_layout = b_layout;
  g.c = (float*)dc; g.ldc = ldc;
  g.epi = fa::Epi::None;
  if (e && (e->bias || e->row_scale || e->act != FA_ACT_NONE || e->mul || e->residual)) {
    g.epi = fa::Epi::Generic;
    void* p;
    if (e->bias) { if ((rc = fa::stage_h2d(ctx, S_BIAS, e->bias, (size_t)n * 4, &p))) return rc; g.bias = (const float*)p; }
    if (e->row_scale) { if ((rc = fa::stage_h2d(ctx, S_ROWSCALE, e->row_scale, (size_t)m * 4, &p))) return rc; g.row_scale = (const float*)p; }
    if (e->mul) { if ((rc = fa::stage_h2d(ctx, S_MUL, e->mul, (size_t)((m - 1) * e->ldm + n) * 4, &p))) return rc; g.mul = (const float*)p; g.ldm = e->ldm; }
    if (e->residual) { if ((rc = fa::stage_h2d(ctx, S_RES, e->residual, (size_t)((m - 1) * e->ldr + n) * 4, &p))) return rc; g.residual = (const float*)p; g.ldr = e->ldr; }
    g.act = e->act;
  }
  if (ldc != n) {
    // rows of C with gaps: keep the caller's bytes between rows
    FA_HIP_CHECK(ctx, hipMemcpyAsync(dc, c, cbytes, hipMemcpyHostToDevice, ctx->stream));
  }
  if ((rc = fa::prepare_b(ctx, g))) return rc;
  if ((rc = fa::launch_gemm(ctx, g, ctx->stream))) return rc;
  FA_HIP_CHECK(ctx, hipMemcpyAsync(c, dc, cbytes, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

int fa_matmul_fused_dev(fa_ctx* ctx, int64_t m, int64_t n, int64_t k, const float* a, int64_t lda, const void* b,
                        int64_t ldb, int b_dtype, int b_layout, const fa_epilogue* e, float* c, int64_t ldc) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "MatMulFused: ctx is NULL");
  if (m < 0 || n < 0 || k < 0) return set_error(ctx, FA_ERR_ARG, "MatMulFused: negative size");
  if (b_dtype != FA_DT_F32 && b_dtype != FA_DT_BF16)
    return set_error(ctx, FA_ERR_ARG, "MatMulFused: unknown B dtype %d", b_dtype);
  if (b_layout != FA_B_KN && b_layout != FA_B_NK)
    return set_error(ctx, FA_ERR_ARG, "MatMulFused: unknown B layout %d", b_layout);
  const int64_t brow = b_layout == FA_B_KN ? n : k, bcnt = b_layout == FA_B_KN ? k : n;
  if ((lda < k && m > 0) || (ldb < brow && bcnt > 0) || (ldc < n && m > 0))
    return set_error(ctx, FA_ERR_ARG, "MatMulFused: leading dimension too small");
  if (e && (e->act < FA_ACT_NONE || e->act > FA_ACT_TANH))
    return set_error(ctx, FA_ERR_ARG, "MatMulFused: unknown activation %d", e->act);
  if (m == 0 || n == 0) return FA_OK;
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "MatMulFused");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  fa::GemmArgs g;
  g.m = m; g.n = n; g.k = k;
  g.a = a; g.lda = lda; g.b = b; g.ldb = ldb; g.b_dtype = b_dtype; g.b_layout = b_layout;
  g.c = c; g.ldc = ldc;
  if (e && (e->bias || e->row_scale || e->act != FA_ACT_NONE || e->mul || e->residual)) {
    g.epi = fa::Epi::Generic;
    g.bias = e->bias; g.row_scale = e->row_scale; g.act = e->act;
    g.mul = e->mul; g.ldm = e->ldm; g.residual = e->residual; g.ldr = e->ldr;
  }
  int rc;
  if ((rc = fa::prepare_b(ctx, g))) return rc;
  return fa::launch_gemm(ctx, g, ctx->stream);
}

int fa_row_sum_squares(fa_ctx* ctx, const float* x, int64_t m, int64_t n, float* out) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "RowSumSquares: ctx is NULL");
  if (m < 0 || n < 0) return set_error(ctx, FA_ERR_ARG, "RowSumSquares: negative shape");
  if (m == 0) return FA_OK;
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "RowSumSquares");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  void *dx, *dout;
  int rc;
  if ((rc = fa::stage_h2d(ctx, S_X, x, (size_t)(m * n) * 4, &dx))) return rc;
  if ((rc = ctx->slot(S_OUT).ensure(ctx, (size_t)m * 4))) return rc;
  dout = ctx->slot(S_OUT).ptr;
  if ((rc = fa::launch_row_sum_squares(ctx, (const float*)dx, m, n, (float*)dout, ctx->stream))) return rc;
  FA_HIP_CHECK(ctx, hipMemcpyAsync(out, dout, (size_t)m * 4, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

int fa_rmsnorm(fa_ctx* ctx, const float* x, const float* g, float eps, int64_t rows, int64_t n, float* out) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "RMSNorm: ctx is NULL");
  if (n <= 0) return set_error(ctx, FA_ERR_ARG, "RMSNorm: expected at least a 1-D input");
  if (rows < 0) return set_error(ctx, FA_ERR_ARG, "RMSNorm: negative row count");
  if (!g) return set_error(ctx, FA_ERR_ARG, "RMSNorm: g must have %lld elements", (long long)n);
  if (rows == 0) return FA_OK;
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "RMSNorm");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  void *dx, *dg, *dout;
  int rc;
  if ((rc = fa::stage_h2d(ctx, S_X, x, (size_t)(rows * n) * 4, &dx))) return rc;
  if ((rc = fa::stage_h2d(ctx, S_G, g, (size_t)n * 4, &dg))) return rc;
  if ((rc = ctx->slot(S_OUT).ensure(ctx, (size_t)(rows * n) * 4))) return rc;
  dout = ctx->slot(S_OUT).ptr;
  if ((rc = fa::launch_rmsnorm(ctx, (const float*)dx, (const float*)dg, eps, rows, n, (float*)dout, ctx->stream)))
    return rc;
  FA_HIP_CHECK(ctx, hipMemcpyAsync(out, dout, (size_t)(rows * n) * 4, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

int fa_rope(fa_ctx* ctx, const float* x, double base, const int32_t* positions, int64_t rows, int32_t T, int32_t D,
            float* out) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "RoPE: ctx is NULL");
  if (D <= 0 || T <= 0 || rows < 0) return set_error(ctx, FA_ERR_ARG, "RoPE: expected at least a 2-D input");
  if (D % 2 != 0) return set_error(ctx, FA_ERR_ARG, "RoPE: head dimension %d must be even", D);
  if (rows % T != 0) return set_error(ctx, FA_ERR_ARG, "RoPE: %lld rows are not a multiple of T=%d", (long long)rows, T);
  if (!positions) return set_error(ctx, FA_ERR_ARG, "RoPE: got 0 positions for %d slots", T);
  if (rows == 0) return FA_OK;
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "RoPE");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  std::vector<float> cs, sn;
  fa::rope_tables_host(base, positions, T, D, cs, sn);
  void *dx, *dc, *ds, *dout;
  int rc;
  if ((rc = fa::stage_h2d(ctx, S_X, x, (size_t)(rows * D) * 4, &dx))) return rc;
  if ((rc = fa::stage_h2d(ctx, S_COS, cs.data(), cs.size() * 4, &dc))) return rc;
  if ((rc = fa::stage_h2d(ctx, S_SIN, sn.data(), sn.size() * 4, &ds))) return rc;
  if ((rc = ctx->slot(S_OUT).ensure(ctx, (size_t)(rows * D) * 4))) return rc;
  dout = ctx->slot(S_OUT).ptr;
  if ((rc = fa::launch_rope(ctx, (const float*)dx, (const float*)dc, (const float*)ds, rows, T, D, (float*)dout,
                            ctx->stream)))
    return rc;
  FA_HIP_CHECK(ctx, hipMemcpyAsync(out, dout, (size_t)(rows * D) * 4, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));  // also keeps cs/sn alive until the copies ran
  return FA_OK;
}

// Bytes spanned by a strided [B, H, R, C] operand with unit stride on C.
static size_t span4(int32_t B, int32_t H, int32_t R, int32_t C, int64_t sb, int64_t sh, int64_t sr, int64_t sc) {
  if (B == 0 || H == 0 || R == 0 || C == 0) return 0;
  int64_t last = (B - 1) * sb + (H - 1) * sh + (int64_t)(R - 1) * sr + (int64_t)(C - 1) * sc;
  return (size_t)(last + 1) * 4;
}

namespace {
int attention_check(fa_ctx* ctx, int32_t B, int32_t H, int32_t T, int32_t S, int32_t D, int64_t q_sb, int64_t q_sh,
                    int64_t k_sb, int64_t k_sh, int64_t v_sb, int64_t v_sh, int64_t m_sb, int64_t m_sh, int64_t m_sr,
                    int64_t m_sc) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "Attention: ctx is NULL");
  if (B < 0 || H < 0 || T < 0 || S < 0 || D < 0) return set_error(ctx, FA_ERR_ARG, "Attention: negative shape");
  if (q_sb < 0 || q_sh < 0 || k_sb < 0 || k_sh < 0 || v_sb < 0 || v_sh < 0 || m_sb < 0 || m_sh < 0 || m_sr < 0 ||
      m_sc < 0)
    return set_error(ctx, FA_ERR_ARG, "Attention: negative stride");
  if ((int64_t)B * H * T > 0 && D > 0 && S == 0) return set_error(ctx, FA_ERR_ARG, "Attention: no keys (S = 0)");
  return FA_OK;
}

int attention_launch(fa_ctx* ctx, const fa::AttnGenericArgs& a) {
  // the MFMA kernel for the head dims it covers, the per-row kernel otherwise
  if (fa::attention_dense_ok(a)) return fa::launch_attention_dense(ctx, a, ctx->stream);
  return fa::launch_attention_generic(ctx, a, ctx->stream);
}
}  // namespace

int fa_attention_dev(fa_ctx* ctx, const float* q, const float* k, const float* v, int32_t B, int32_t H, int32_t T,
                     int32_t S, int32_t D, int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh, int64_t v_sb,
                     int64_t v_sh, const float* mask, int64_t m_sb, int64_t m_sh, int64_t m_sr, int64_t m_sc,
                     float scale, float* out) {
  int rc = attention_check(ctx, B, H, T, S, D, q_sb, q_sh, k_sb, k_sh, v_sb, v_sh, m_sb, m_sh, m_sr, m_sc);
  if (rc) return rc;
  if ((int64_t)B * H * T == 0 || D == 0) return FA_OK;
  if (!q || !k || !v || !out) return set_error(ctx, FA_ERR_ARG, "Attention: NULL buffer");
  if ((rc = fa::refuse_capture(ctx, ctx->stream, "Attention"))) return rc;
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  fa::AttnGenericArgs a;
  a.q = q; a.k = k; a.v = v; a.mask = mask;
  a.B = B; a.H = H; a.T = T; a.S = S; a.D = D;
  a.q_sb = q_sb; a.q_sh = q_sh; a.k_sb = k_sb; a.k_sh = k_sh; a.v_sb = v_sb; a.v_sh = v_sh;
  a.m_sb = m_sb; a.m_sh = m_sh; a.m_sr = m_sr; a.m_sc = m_sc;
  a.scale = scale;
  a.out = out;
  return attention_launch(ctx, a);
}

int fa_attention(fa_ctx* ctx, const float* q, const float* k, const float* v, int32_t B, int32_t H, int32_t T,
                 int32_t S, int32_t D, int64_t q_sb, int64_t q_sh, int64_t k_sb, int64_t k_sh, int64_t v_sb,
                 int64_t v_sh, const float* mask, int64_t m_sb, int64_t m_sh, int64_t m_sr, int64_t m_sc, float scale,
                 float* out) {
  int rc = attention_check(ctx, B, H, T, S, D, q_sb, q_sh, k_sb, k_sh, v_sb, v_sh, m_sb, m_sh, m_sr, m_sc);
  if (rc) return rc;
  if ((int64_t)B * H * T == 0 || D == 0) return FA_OK;
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "Attention");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  void *dq, *dk, *dv, *dm = nullptr, *dout;
  if ((rc = fa::stage_h2d(ctx, S_Q, q, span4(B, H, T, D, q_sb, q_sh, D, 1), &dq))) return rc;
  if ((rc = fa::stage_h2d(ctx, S_K, k, span4(B, H, S, D, k_sb, k_sh, D, 1), &dk))) return rc;
  if ((rc = fa::stage_h2d(ctx, S_V, v, span4(B, H, S, D, v_sb, v_sh, D, 1), &dv))) return rc;
  if (mask && (rc = fa::stage_h2d(ctx, S_MASK, mask, span4(B, H, T, S, m_sb, m_sh, m_sr, m_sc), &dm))) return rc;
  const size_t obytes = (size_t)B * H * T * D * 4;
  if ((rc = ctx->slot(S_OUT).ensure(ctx, obytes))) return rc;
  dout = ctx->slot(S_OUT).ptr;
  fa::AttnGenericArgs a;
  a.q = (const float*)dq; a.k = (const float*)dk; a.v = (const float*)dv; a.mask = (const float*)dm;
  a.B = B; a.H = H; a.T = T; a.S = S; a.D = D;
  a.q_sb = q_sb; a.q_sh = q_sh; a.k_sb = k_sb; a.k_sh = k_sh; a.v_sb = v_sb; a.v_sh = v_sh;
  a.m_sb = m_sb; a.m_sh = m_sh; a.m_sr = m_sr; a.m_sc = m_sc;
  a.scale = scale;
  a.out = (float*)dout;
  if ((rc = attention_launch(ctx, a))) return rc;
  FA_HIP_CHECK(ctx, hipMemcpyAsync(out, dout, obytes, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

int fa_similarities_topk_dev(fa_ctx* ctx, const float* queries, int64_t nq, const float* docs, int64_t nd, int32_t d,
                             int32_t topk, int32_t* idx, float* val) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "Similarities: ctx is NULL");
  if (nq < 0 || nd <= 0 || d <= 0)
    return set_error(ctx, FA_ERR_ARG, "Similarities: shapes [%lld x %d] and [%lld x %d]", (long long)nq, d,
                     (long long)nd, d);
  if (topk < 1 || topk > 32 || topk > nd)
    return set_error(ctx, FA_ERR_ARG, "Similarities top-k: k=%d outside 1..min(32, %lld)", topk, (long long)nd);
  if (nq == 0) return FA_OK;
  if (nq > 65535) return set_error(ctx, FA_ERR_ARG, "Similarities top-k: %lld queries > 65535", (long long)nq);
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "Similarities");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  int rc;
  // Batches of queries: the fused kernels (no score matrix; blocks of 256
  // queries share each pass over the docs; exact float32-rounded scores).
  // Few queries: the fp32-MFMA product and the two-pass top-k, which read the
  // docs once without computing a 256-query block (the fused stage computes
  // whole blocks: one query would cost what 256 do).
  if (nq >= 128 && fa::score_fused_ok(queries, d, docs, d, d, topk)) {
    const int nwg = fa::score_workgroups(nd, ctx->cu_count);
    fa::DevBuf& ws = ctx->slot(S_TOPK);
    if ((rc = ws.ensure(ctx, fa::score_scratch_bytes(d, nwg)))) return rc;
    return fa::launch_score_topk(ctx, queries, nq, d, docs, nd, d, d, topk, idx, val, ws.ptr, nwg, ctx->stream);
  }
  fa::DevBuf& sc = ctx->slot(S_C);
  if ((rc = sc.ensure(ctx, (size_t)(nq * nd) * 4))) return rc;
  fa::GemmArgs g;
  g.m = nq; g.n = nd; g.k = d;
  g.a = queries; g.lda = d; g.b = docs; g.ldb = d; g.b_dtype = FA_DT_F32; g.b_layout = FA_B_NK;
  g.c = sc.as<float>(); g.ldc = nd;
  if ((rc = fa::launch_gemm(ctx, g, ctx->stream))) return rc;
  fa::DevBuf& cand = ctx->slot(S_TOPK);
  if ((rc = cand.ensure(ctx, (size_t)fa::topk_scratch_bytes(nq, nd, topk)))) return rc;
  return fa::launch_topk(ctx, sc.as<float>(), nq, nd, topk, idx, val, cand.ptr, ctx->stream);
}

int fa_similarities_topk(fa_ctx* ctx, const float* queries, int64_t nq, const float* docs, int64_t nd, int32_t d,
                         int32_t topk, int32_t* idx, float* val) {
  if (!ctx) return set_error(ctx, FA_ERR_ARG, "Similarities: ctx is NULL");
  if (nq < 0 || nd <= 0 || d <= 0)
    return set_error(ctx, FA_ERR_ARG, "Similarities: shapes [%lld x %d] and [%lld x %d]", (long long)nq, d,
                     (long long)nd, d);
  if (topk < 1 || topk > 32 || topk > nd)
    return set_error(ctx, FA_ERR_ARG, "Similarities top-k: k=%d outside 1..min(32, %lld)", topk, (long long)nd);
  if (nq == 0) return FA_OK;
  if (nq > 65535) return set_error(ctx, FA_ERR_ARG, "Similarities top-k: %lld queries > 65535", (long long)nq);
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "Similarities");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  void *dq, *dd;
  int rc;
  if ((rc = fa::stage_h2d(ctx, S_Q, queries, (size_t)(nq * d) * 4, &dq))) return rc;
  if ((rc = fa::stage_h2d(ctx, S_K, docs, (size_t)(nd * d) * 4, &dd))) return rc;
  const size_t ib = (size_t)nq * topk * 4;
  if ((rc = ctx->slot(S_OUT).ensure(ctx, 2 * ib))) return rc;
  int32_t* di = ctx->slot(S_OUT).as<int32_t>();
  float* dv = (float*)((char*)ctx->slot(S_OUT).ptr + ib);
  if ((rc = fa_similarities_topk_dev(ctx, (const float*)dq, nq, (const float*)dd, nd, d, topk, di, dv))) return rc;
  FA_HIP_CHECK(ctx, hipMemcpyAsync(idx, di, ib, hipMemcpyDeviceToHost, ctx->stream));
  if (val) FA_HIP_CHECK(ctx, hipMemcpyAsync(val, dv, ib, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  return FA_OK;
}

}  // extern "C"
