// The EmbeddingGemma encoder on one GPU: bf16-resident weights, packed
// variable-length token rows, and the forward pass
//   gather*sqrt(d) -> 24 x [qkv GEMM, qk-norm+RoPE, attention, o GEMM,
//   post-norm+residual(+next pre-norm), gate|up GEMM with GeGLU epilogue,
//   down GEMM, post-norm+residual(+next pre-norm)] -> mean pool -> Dense head
//   -> L2
// following models/gemma/embed.go:160-240,381-475 and model.go:76-232.
// Variant 2 (EmbeddingGemma 2, embed.go:247-377) adds per-layer head dims
// and key/value heads, the v norm, the per-layer inputs (one projection of
// the scaled embeddings, normalised per layer), each layer's
// per-layer-input block (gate GEMM with GELU and the layer's input in the
// epilogue, projection GEMM, post-norm + residual, times the layer scalar)
// and the embedding projection of the pooled vector.
//
// Layout in HBM (M = sum of valid lengths; padding rows are never stored):
//   x   [M, d] fp32   residual stream
//   xn  [M, d] fp32   RMSNorm(x; 1+g) feeding the next product (the
//                     reference folds 1+g into the weights and applies the
//                     row scale in the product's epilogue, model.go:210-222,
//                     embed.go:193-197; the values agree to rounding)
//   qkv [M, (H+2Hkv)*D] fp32   q | k | v per token, normed and rotated in place
//   att [M, H*D] fp32, o [M, d] fp32, gu [M, F] fp32
// Weights: [out, in] bf16 as in the checkpoint; q|k|v stacked into one
// [(H+2Hkv)*D, d] matrix, gate and up interleaved in 32-row groups into one
// [2F, d] matrix (see gemm.hip), 1+w norm vectors in fp32.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <vector>

#include "fa_internal.h"
#include "plan.h"

namespace fa {

namespace {

constexpr int64_t kAttnSplitRows = 1024;  // key-split attention only for batches up to this many tokens

bool bf16_exact(float f, uint16_t* out) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if (u & 0xFFFFu) return false;
  *out = (uint16_t)(u >> 16);
  return true;
}

// A weight matrix [rows, cols] in HBM: bf16 values as stored in the
// checkpoint (terms = 1), or, once any of its float32 values is not
// bf16-exact, three bf16 planes hi, mid, lo of the float32 values (terms = 3,
// rows*cols elements apart; hi + mid + lo is the value exactly), which the
// products take through the six-term split kernel.
struct Mat {
  uint16_t* p = nullptr;
  int64_t rows = 0, cols = 0;
  int terms = 1;
  int64_t plane() const { return rows * cols; }
};

struct Layer {
  int D = 0, Hkv = 0, width = 0;  // head dim, key/value heads, q|k|v width (H+2Hkv)*D
  bool sliding = true;
  const float *cos_t = nullptr, *sin_t = nullptr;  // RoPE tables of this layer's base and D
  Mat wqkv;   // [(H+2Hkv)*D, d]
  Mat wo;     // [d, H*D]
  Mat wgu;    // [2F, d], 32-row groups gate/up alternating
  Mat wdown;  // [d, F]
  float *g_in = nullptr, *g_post_attn = nullptr, *g_pre_ffn = nullptr, *g_post_ffn = nullptr;
  float *g_q = nullptr, *g_k = nullptr;
  // variant 2: per-layer-input block and layer scalar
  Mat wple_gate;  // [P, d]
  Mat wple_proj;  // [d, P]
  float* g_ple_post = nullptr;
  float scalar = 1.f;
};

struct KernelStat {
  int64_t launches = 0;
  double ms = 0, flops = 0, bytes = 0;
};

struct PendingEvent {
  hipEvent_t a, b;
  int kind;
  double flops, bytes;
};

}  // namespace
}  // namespace fa

struct fa_model {
  fa_ctx* ctx = nullptr;
  fa_gemma_config cfg{};
  int variant = 0;
  int max_width = 0, max_hd = 0;  // widest q|k|v row, widest attention output H*D
  int P = 0, E = 0;               // variant 2: per-layer input width, embedding projection width
  fa::Mat wple_model;             // variant 2: [layers*P, d]
  float* g_ple_norm = nullptr;    // variant 2: [P]
  fa::Mat wemb_proj;              // variant 2: [E, d]
  std::vector<void*> allocations;
  fa::Mat embed;
  std::vector<fa::Layer> layers;
  float* g_final = nullptr;
  std::vector<fa::Mat> dense;
  std::vector<int> dense_in, dense_out, dense_act;  // dense_act: FA_ACT_NONE or FA_ACT_TANH
  float *cos_local = nullptr, *sin_local = nullptr, *cos_global = nullptr, *sin_global = nullptr;
  int d_local = 0, d_global = 0;  // head dims of the sliding and the full layers
  std::set<std::string> seen;
  bool finalized = false;
  // workspace
  fa::DevBuf ws, plan_dev;
  int64_t ws_rows = 0, ws_seqs = 0;
  int32_t* plan_host = nullptr;  // pinned
  size_t plan_host_ints = 0;
  hipEvent_t plan_done = nullptr;
  bool plan_pending = false;
  // streams of micro-batches 1.. (micro-batch 0 runs on the context's
  // stream), the fork event and one join event per extra stream
  hipStream_t mb_stream[fa::kMaxMicrobatches] = {};
  hipEvent_t ev_fork = nullptr, ev_join[fa::kMaxMicrobatches] = {};
  std::vector<int> seq_order;                 // plan scratch
  std::vector<int> plan_layer_D, plan_layer_Hkv;  // plan inputs: each layer's head dim, kv heads
  fa::DevBuf ids_dev, out_dev;
  // pinned staging of the host entry points' ids and results (asynchronous
  // copies; the entry points synchronise before returning)
  void* io_host = nullptr;
  size_t io_host_bytes = 0;
  // profiling
  bool profiling = false;
  std::vector<hipEvent_t> event_pool;
  std::vector<fa::PendingEvent> pending;
  fa::KernelStat stats[FA_K_COUNT];
};

namespace fa {
namespace {

int alloc_dev(fa_model* m, size_t bytes, void** out) {
  hipError_t e = hipMalloc(out, bytes ? bytes : 1);
  if (e != hipSuccess) return set_error(m->ctx, FA_ERR_OOM, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  m->allocations.push_back(*out);
  return FA_OK;
}

// Frees one of the model's allocations (a matrix promoted to three planes).
void free_dev(fa_model* m, void* ptr) {
  for (auto& a : m->allocations)
    if (a == ptr) {
      (void)hipFree(a);
      a = m->allocations.back();
      m->allocations.pop_back();
      return;
    }
}

// B operand of a product over w's rows [row0, ...): one bf16 plane or three.
void set_b(GemmArgs& g, const Mat& w, int64_t row0 = 0) {
  g.b = w.p + row0 * w.cols;
  g.ldb = w.cols;
  g.b_terms = w.terms;
  g.b_plane = w.plane();
}

hipEvent_t take_event(fa_model* m) {
  if (!m->event_pool.empty()) {
    hipEvent_t e = m->event_pool.back();
    m->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Token count from which a batch runs as micro-batches on several streams;
// FA_MICROBATCH=0 turns that off, FA_MICROBATCH=<rows> sets the threshold.
int64_t microbatch_min_rows() {
  static const int64_t v = [] {
    const char* e = std::getenv("FA_MICROBATCH");
    if (!e) return (int64_t)2048;
    const long long n = std::atoll(e);
    return n <= 0 ? INT64_MAX : (int64_t)n;
  }();
  return v;
}

// Number of micro-batches (2..kMaxMicrobatches; FA_MICROBATCH_GROUPS). Three
// measured best on MI355X at 5 517, 11 550 and 32 768 tokens (C2: 6.41 ms
// per forward on one stream, 5.49 with two groups, 5.43 with three, 5.92
// with four) and within 3 % of best at 17 923.
// FA_ATTN_KEY_PARTS=<1..8> forces the key runs of the short-batch attention
// (tuning); 0 when unset.
int attention_key_parts_forced() {
  static const int v = [] {
    const char* e = std::getenv("FA_ATTN_KEY_PARTS");
    if (!e) return 0;
    return std::max(1, std::min(std::atoi(e), kMaxKeyParts));
  }();
  return v;
}

// FA_ATTN_ROWS=64|128 forces the tile attention's rows per item (tuning);
// 0 when unset.
int attention_rows_forced() {
  static const int v = [] {
    const char* e = std::getenv("FA_ATTN_ROWS");
    if (!e) return 0;
    const int r = std::atoi(e);
    return r == 64 || r == 128 ? r : 0;
  }();
  return v;
}

// FA_ATTN_XCD=1|0 forces the XCD-local attention item order on or off
// (tuning); 0 when unset (chosen per group).
int attention_xcd_forced() {
  static const int v = [] {
    const char* e = std::getenv("FA_ATTN_XCD");
    if (!e) return 0;
    return e[0] == '0' ? -1 : 1;
  }();
  return v;
}

// K parts of the N = hidden products (o, down) for a few-row batch whose
// small-M tiles, times four parts, still fit one per CU (FA_SMALL_KSPLIT=2
// or 4, default 4). A small-M workgroup's time is its operand loads: with
// four parts each loads half the bytes of two (at 128 rows: o 8.5 -> 7.4
// us, down 9.8 -> 8.4 us per launch; C1 1.30 -> 1.28 ms per forward, 64
// tokens 1.25 -> 1.22 ms on MI355X), for two more partial planes read by
// the residual step.
int small_ksplit() {
  static const int v = [] {
    const char* e = std::getenv("FA_SMALL_KSPLIT");
    if (!e) return 4;
    return std::atoi(e) >= 4 ? 4 : 2;
  }();
  return v;
}

// K parts of a few-row batch's q|k|v product on the fp32 attention path,
// added by the q/k norm pass (FA_QKV_KSPLIT=1 or 2, default 2): 160 instead
// of 80 workgroups at 128 rows, each loading half the operands (11.1 ->
// 9.0 us per launch; C1 1.28 -> 1.24 ms, 64 tokens 1.22 -> 1.17 ms per
// forward on MI355X), for one more read of the product in the norm pass.
int qkv_ksplit() {
  static const int v = [] {
    const char* e = std::getenv("FA_QKV_KSPLIT");
    if (!e) return 2;
    return std::atoi(e) >= 2 ? 2 : 1;
  }();
  return v;
}

// FA_TILE_MIN_ROWS=<tokens>: the tile attention from more tokens than this
// (tuning; 1 024 when unset).
int64_t tile_min_rows() {
  static const int64_t v = [] {
    const char* e = std::getenv("FA_TILE_MIN_ROWS");
    if (!e) return (int64_t)1024;
    return (int64_t)std::max(0LL, std::atoll(e));
  }();
  return v;
}

// FA_MICROBATCH_GROUPS=<2..4> forces the group count (tuning); 0 when unset.
int microbatch_count_forced() {
  static const int v = [] {
    const char* e = std::getenv("FA_MICROBATCH_GROUPS");
    if (!e) return 0;
    return std::max(2, std::min(std::atoi(e), kMaxMicrobatches));
  }();
  return v;
}

// Group count by the batch, from sweeps of 2, 3 and 4 groups on MI355X:
// long sequences (the mean key count per token, sum L^2 / sum L, at least
// 1 024) make the forward attention-bound and gain from a fourth stream
// (C4, 8 x 1 024..2 048: 11.80 ms against 11.84 with two and 11.97 with
// three); from 24 576 tokens the products are large enough on their own and
// two groups keep their tiles full (C3, 64 x 512: 27.45 ms against 28.0 with
// three); else three (C2: 5.30 ms against 5.41 with two and 5.53 with four;
// C5, 17 923 tokens: 13.74 against 13.91 and 14.26).
int microbatch_count(int64_t tokens, double sum_l2) {
  if (const int f = microbatch_count_forced()) return f;
  if (sum_l2 >= 1024.0 * (double)tokens) return 4;
  return tokens >= 24576 ? 2 : 3;
}

// HBM bytes of one residual_norm launch: the product's K parts and x
// read, x written, and the next norm's input written when there is a next
// norm.
double resnorm_bytes(int64_t rows, int64_t d, int parts, const float* g_next) {
  return (double)rows * d * 4.0 * (2.0 + parts + (g_next ? 1.0 : 0.0));
}

// Brackets one launch with events when profiling.
struct Probe {
  fa_model* m;
  hipEvent_t a = nullptr;
  int kind;
  double flops, bytes;
  Probe(fa_model* mm, int k, double f, double b) : m(mm), kind(k), flops(f), bytes(b) {
    if (m->profiling) {
      a = take_event(m);
      if (a) (void)hipEventRecord(a, m->ctx->stream);
    }
  }
  void done() {
    if (!a) return;
    hipEvent_t b = take_event(m);
    if (!b) return;
    (void)hipEventRecord(b, m->ctx->stream);
    m->pending.push_back({a, b, kind, flops, bytes});
    a = nullptr;
  }
};

int collect_stats(fa_model* m) {
  if (m->pending.empty()) return FA_OK;
  FA_HIP_CHECK(m->ctx, hipStreamSynchronize(m->ctx->stream));
  for (auto& p : m->pending) {
    float ms = 0;
    if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
      KernelStat& s = m->stats[p.kind];
      s.launches++;
      s.ms += ms;
      s.flops += p.flops;
      s.bytes += p.bytes;
    }
    m->event_pool.push_back(p.a);
    m->event_pool.push_back(p.b);
  }
  m->pending.clear();
  return FA_OK;
}

// The pinned staging buffer of the host entry points, grown to at least bytes.
int io_staging(fa_model* m, size_t bytes, char** out) {
  if (bytes > m->io_host_bytes) {
    if (m->io_host) (void)hipHostFree(m->io_host);
    m->io_host = nullptr;
    m->io_host_bytes = 0;
    FA_HIP_CHECK(m->ctx, hipHostMalloc(&m->io_host, bytes, hipHostMallocDefault));
    m->io_host_bytes = bytes;
  }
  *out = static_cast<char*>(m->io_host);
  return FA_OK;
}

// Host-side check of a host batch: lengths in 1..T and every valid id inside
// the vocabulary (an out-of-range id would read outside the table).
int check_ids(fa_model* m, const int32_t* ids, const int32_t* lengths, int B, int T) {
  const int V = m->cfg.vocab_size;
  for (int b = 0; b < B; b++) {
    if (lengths[b] < 1 || lengths[b] > T)
      return set_error(m->ctx, FA_ERR_ARG, "gemma: length[%d] = %d outside 1..T=%d", b, lengths[b], T);
    for (int t = 0; t < lengths[b]; t++) {
      const int32_t id = ids[(size_t)b * T + t];
      if (id < 0 || id >= V)
        return set_error(m->ctx, FA_ERR_ARG, "gemma: token id %d at [%d,%d] outside 0..%d", id, b, t, V - 1);
    }
  }
  return FA_OK;
}

int parse_layer(const std::string& s, int nl, int* l, std::string* rest) {
  if (s.rfind("layers.", 0) != 0) return -1;
  size_t dot = s.find('.', 7);
  if (dot == std::string::npos) return -1;
  char* end = nullptr;
  long v = std::strtol(s.c_str() + 7, &end, 10);
  if (end != s.c_str() + dot || v < 0 || v >= nl) return -1;
  *l = (int)v;
  *rest = s.substr(dot + 1);
  return 0;
}

}  // namespace
}  // namespace fa

using fa::set_error;

extern "C" {

int fa_gemma_create(fa_ctx* ctx, const fa_gemma_config* cfg, fa_model** out) {
  if (!ctx || !cfg || !out) return set_error(ctx, FA_ERR_ARG, "gemma: NULL argument");
  *out = nullptr;
  const fa_gemma_config& c = *cfg;
  if (c.hidden_size <= 0 || c.num_hidden_layers <= 0 || c.num_attention_heads <= 0 || c.num_key_value_heads <= 0 ||
      c.head_dim <= 0 || c.intermediate_size <= 0 || c.vocab_size <= 0)
    return set_error(ctx, FA_ERR_ARG, "gemma: config sizes must be positive");
  if (c.variant != 0 && c.variant != 2) return set_error(ctx, FA_ERR_ARG, "gemma: variant %d not 0 or 2", c.variant);
  const bool v2 = c.variant == 2;
  if (c.hidden_size % 256 != 0 || c.hidden_size > 1024)
    return set_error(ctx, FA_ERR_UNSUPPORTED, "gemma: hidden_size %d not in {256,512,768,1024}", c.hidden_size);
  if (c.num_hidden_layers > FA_GEMMA_MAX_LAYERS)
    return set_error(ctx, FA_ERR_UNSUPPORTED, "gemma: %d layers, at most %d", c.num_hidden_layers, FA_GEMMA_MAX_LAYERS);
  if (!v2 && c.head_dim != 256) return set_error(ctx, FA_ERR_UNSUPPORTED, "gemma: head_dim %d != 256", c.head_dim);
  if (c.intermediate_size % 32 != 0)
    return set_error(ctx, FA_ERR_UNSUPPORTED, "gemma: intermediate_size %d not a multiple of 32", c.intermediate_size);
  if (c.n_dense < 0 || c.n_dense > 4) return set_error(ctx, FA_ERR_ARG, "gemma: n_dense %d outside 0..4", c.n_dense);
  if (c.max_tokens <= 0) return set_error(ctx, FA_ERR_ARG, "gemma: max_tokens must be positive");
  if (!v2 && c.query_pre_attn_scalar <= 0) return set_error(ctx, FA_ERR_ARG, "gemma: query_pre_attn_scalar must be > 0");
  if (v2 && (c.hidden_size_per_layer_input <= 0 || c.hidden_size_per_layer_input % 32 != 0))
    return set_error(ctx, FA_ERR_UNSUPPORTED, "gemma: hidden_size_per_layer_input %d not a positive multiple of 32",
                     c.hidden_size_per_layer_input);
  if (v2 && c.embedding_dim <= 0) return set_error(ctx, FA_ERR_ARG, "gemma: embedding_dim must be positive");
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  fa_model* m = new fa_model();
  m->ctx = ctx;
  m->cfg = c;
  m->variant = c.variant;
  if (m->cfg.sliding_window_pattern <= 0) m->cfg.sliding_window_pattern = 6;
  const int d = c.hidden_size, H = c.num_attention_heads, F = c.intermediate_size, NL = c.num_hidden_layers;
  m->layers.resize(NL);
  int rc = FA_OK;
  for (int l = 0; l < NL && !rc; l++) {
    fa::Layer& L = m->layers[l];
    L.D = v2 && c.layer_head_dim[l] > 0 ? c.layer_head_dim[l] : c.head_dim;
    L.Hkv = v2 && c.layer_kv_heads[l] > 0 ? c.layer_kv_heads[l] : c.num_key_value_heads;
    L.sliding = v2 ? c.layer_sliding[l] != 0 : (l + 1) % m->cfg.sliding_window_pattern != 0;  // config.go:213-225
    L.width = (H + 2 * L.Hkv) * L.D;
    int& dt = L.sliding ? m->d_local : m->d_global;
    if (L.D != 256 && L.D != 512)
      rc = set_error(ctx, FA_ERR_UNSUPPORTED, "gemma: layer %d head_dim %d not 256 or 512", l, L.D);
    else if (H % L.Hkv != 0)
      rc = set_error(ctx, FA_ERR_ARG, "gemma: layer %d: %d heads not a multiple of %d kv heads", l, H, L.Hkv);
    else if (dt != 0 && dt != L.D)
      rc = set_error(ctx, FA_ERR_UNSUPPORTED, "gemma: layer %d head_dim %d differs from other %s layers' %d", l, L.D,
                     L.sliding ? "sliding" : "full-attention", dt);
    dt = L.D;
    m->max_width = std::max(m->max_width, L.width);
    m->max_hd = std::max(m->max_hd, H * L.D);
  }
  if (rc) {
    delete m;
    return rc;
  }
  m->P = v2 ? c.hidden_size_per_layer_input : 0;
  m->E = v2 ? c.embedding_dim : 0;
  void* p;
  auto A = [&](size_t bytes) -> void* {
    if (rc) return nullptr;
    rc = fa::alloc_dev(m, bytes, &p);
    return rc ? nullptr : p;
  };
  auto M_ = [&](int64_t rows, int64_t cols) {
    fa::Mat w;
    w.rows = rows;
    w.cols = cols;
    w.p = (uint16_t*)A((size_t)rows * cols * 2);
    return w;
  };
  m->embed = M_(c.vocab_size, d);
  for (auto& L : m->layers) {
    L.wqkv = M_(L.width, d);
    L.wo = M_(d, (int64_t)H * L.D);
    L.wgu = M_(2LL * F, d);
    L.wdown = M_(d, F);
    L.g_in = (float*)A(d * 4);
    L.g_post_attn = (float*)A(d * 4);
    L.g_pre_ffn = (float*)A(d * 4);
    L.g_post_ffn = (float*)A(d * 4);
    L.g_q = (float*)A(L.D * 4);
    L.g_k = (float*)A(L.D * 4);
    if (v2) {
      L.wple_gate = M_(m->P, d);
      L.wple_proj = M_(d, m->P);
      L.g_ple_post = (float*)A(d * 4);
    }
  }
  m->g_final = (float*)A(d * 4);
  if (v2) {
    m->wple_model = M_((int64_t)NL * m->P, d);
    m->g_ple_norm = (float*)A(m->P * 4);
    m->wemb_proj = M_(m->E, d);
  }
  int in = v2 ? m->E : d;
  for (int i = 0; i < c.n_dense; i++) {
    if (c.dense_out[i] <= 0) rc = set_error(ctx, FA_ERR_ARG, "gemma: dense_out[%d] = %d", i, c.dense_out[i]);
    if (c.dense_act[i] != FA_ACT_NONE && c.dense_act[i] != FA_ACT_TANH)
      rc = set_error(ctx, FA_ERR_ARG, "gemma: dense_act[%d] = %d (identity or tanh)", i, c.dense_act[i]);
    m->dense_in.push_back(in);
    m->dense_out.push_back(c.dense_out[i]);
    m->dense_act.push_back(c.dense_act[i]);
    m->dense.push_back(M_(c.dense_out[i], in));
    in = c.dense_out[i];
  }
  if (m->d_local) {
    const size_t tab = (size_t)c.max_tokens * (m->d_local / 2) * 4;
    m->cos_local = (float*)A(tab);
    m->sin_local = (float*)A(tab);
  }
  if (m->d_global) {
    const size_t tab = (size_t)c.max_tokens * (m->d_global / 2) * 4;
    m->cos_global = (float*)A(tab);
    m->sin_global = (float*)A(tab);
  }
  for (auto& L : m->layers) {
    L.cos_t = L.sliding ? m->cos_local : m->cos_global;
    L.sin_t = L.sliding ? m->sin_local : m->sin_global;
  }
  if (!rc && (hipEventCreateWithFlags(&m->plan_done, hipEventDisableTiming) != hipSuccess ||
              hipEventCreateWithFlags(&m->ev_fork, hipEventDisableTiming) != hipSuccess))
    rc = set_error(ctx, FA_ERR_HIP, "hipEventCreate failed");
  for (int i = 1; i < fa::kMaxMicrobatches && !rc; i++) {
    if (hipEventCreateWithFlags(&m->ev_join[i], hipEventDisableTiming) != hipSuccess)
      rc = set_error(ctx, FA_ERR_HIP, "hipEventCreate failed");
    else if (hipStreamCreateWithFlags(&m->mb_stream[i], hipStreamNonBlocking) != hipSuccess)  // default priority
      rc = set_error(ctx, FA_ERR_HIP, "hipStreamCreate failed");
  }
  if (rc) {
    fa::model_release(m);
    return rc;
  }
  fa::register_model(m, ctx);
  *out = m;
  return FA_OK;
}

void fa_gemma_destroy(fa_model* m) {
  // unknown, already closed with its context, or at exit: nothing to do
  if (!m || !fa::unregister_model(m)) return;
  fa::model_release(m);
}

}  // extern "C"

void fa::model_release(fa_model* m) {
  (void)hipSetDevice(m->ctx->device);
  (void)hipStreamSynchronize(m->ctx->stream);
  for (hipStream_t st : m->mb_stream)
    if (st) (void)hipStreamSynchronize(st);
  for (void* p : m->allocations) (void)hipFree(p);
  m->ws.release();
  m->plan_dev.release();
  m->ids_dev.release();
  m->out_dev.release();
  if (m->plan_host) (void)hipHostFree(m->plan_host);
  if (m->io_host) (void)hipHostFree(m->io_host);
  if (m->plan_done) (void)hipEventDestroy(m->plan_done);
  if (m->ev_fork) (void)hipEventDestroy(m->ev_fork);
  for (int i = 0; i < fa::kMaxMicrobatches; i++) {
    if (m->ev_join[i]) (void)hipEventDestroy(m->ev_join[i]);
    if (m->mb_stream[i]) (void)hipStreamDestroy(m->mb_stream[i]);
  }
  for (auto& p : m->pending) {
    m->event_pool.push_back(p.a);
    m->event_pool.push_back(p.b);
  }
  for (hipEvent_t e : m->event_pool) (void)hipEventDestroy(e);
  delete m;
}

extern "C" {

int fa_gemma_set_weight(fa_model* m, const char* name, int dtype, const int64_t* shape, int32_t ndim,
                        const void* data) {
  if (!m || !name || !data || (ndim > 0 && !shape)) return set_error(m ? m->ctx : nullptr, FA_ERR_ARG, "gemma: NULL argument");
  fa_ctx* ctx = m->ctx;
  if (dtype != FA_DT_F32 && dtype != FA_DT_BF16) return set_error(ctx, FA_ERR_ARG, "gemma: weight %s: dtype %d", name, dtype);
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "gemma");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  const fa_gemma_config& c = m->cfg;
  const bool v2 = m->variant == 2;
  const int d = c.hidden_size, H = c.num_attention_heads, F = c.intermediate_size, P = m->P;
  const std::string s(name);
  auto shape_is = [&](std::initializer_list<int64_t> want) {
    if ((size_t)ndim != want.size()) return false;
    int i = 0;
    for (int64_t w : want)
      if (shape[i++] != w) return false;
    return true;
  };
  auto shape_str = [&]() {
    std::string r = "[";
    for (int i = 0; i < ndim; i++) r += (i ? "," : "") + std::to_string(shape[i]);
    return r + "]";
  };
  // matrix [rows, cols] -> rows of dst (row stride cols); source row r goes to
  // destination row dst_row(r), copied in runs of consecutive rows. bf16 data
  // and bf16-exact float32 data keep one bf16 plane; float32 data with any
  // other value turns dst into three planes (hi, mid, lo: the same split as
  // the kernels' split3), the rows written before kept as hi with zero mid
  // and lo.
  auto put_matrix = [&](fa::Mat& dst, int64_t rows, int64_t cols, auto&& dst_row) -> int {
    const size_t n = (size_t)rows * cols;
    std::vector<uint16_t> tmp;
    const uint16_t* src16 = (const uint16_t*)data;
    bool exact = true;
    if (dtype == FA_DT_F32) {
      tmp.resize(n);
      const float* src = (const float*)data;
      for (size_t i = 0; i < n && exact; i++) exact = fa::bf16_exact(src[i], &tmp[i]);
      if (!exact) {
        tmp.resize(3 * n);
        for (size_t i = 0; i < n; i++) {
          uint32_t u;
          std::memcpy(&u, &src[i], 4);
          const uint32_t hi = u & 0xFFFF0000u;
          float fh, r1;
          std::memcpy(&fh, &hi, 4);
          r1 = src[i] - fh;  // exact in float32
          uint32_t u1;
          std::memcpy(&u1, &r1, 4);
          const uint32_t mid = u1 & 0xFFFF0000u;
          float fm, r2;
          std::memcpy(&fm, &mid, 4);
          r2 = r1 - fm;  // at most 8 significant bits: exact in bf16
          uint32_t u2;
          std::memcpy(&u2, &r2, 4);
          tmp[i] = (uint16_t)(hi >> 16);
          tmp[n + i] = (uint16_t)(mid >> 16);
          tmp[2 * n + i] = (uint16_t)(u2 >> 16);
        }
      }
      src16 = tmp.data();
    }
    // the six-term kernel of a three-plane matrix takes whole 32-wide K slabs
    // (the one-plane case has the fp32-MFMA kernel for other widths): refuse
    // here rather than at the first embed
    if (!exact && cols % 32 != 0)
      return set_error(ctx, FA_ERR_UNSUPPORTED,
                       "gemma: weight %s: a float32 matrix with values bfloat16 cannot hold needs an input width "
                       "that is a multiple of 32, got %lld",
                       name, (long long)cols);
    if (!exact && dst.terms == 1) {
      // promote to three planes: the rows set so far become hi, mid = lo = 0
      void* np = nullptr;
      int rc2 = fa::alloc_dev(m, (size_t)3 * dst.plane() * 2, &np);
      if (rc2) return rc2;
      FA_HIP_CHECK(ctx, hipMemcpy(np, dst.p, (size_t)dst.plane() * 2, hipMemcpyDeviceToDevice));
      FA_HIP_CHECK(ctx, hipMemset((uint16_t*)np + dst.plane(), 0, (size_t)2 * dst.plane() * 2));
      fa::free_dev(m, dst.p);
      dst.p = (uint16_t*)np;
      dst.terms = 3;
    }
    const int src_terms = exact ? 1 : 3;
    std::vector<uint16_t> zeros;
    for (int t = 0; t < dst.terms; t++) {
      const uint16_t* from = src16 + (t < src_terms ? (size_t)t * n : 0);
      if (t >= src_terms) {  // rows of an exact matrix in a three-plane one: zero mid and lo
        if (zeros.empty()) zeros.assign(n, 0);
        from = zeros.data();
      }
      uint16_t* plane = dst.p + (size_t)t * dst.plane();
      for (int64_t r0 = 0; r0 < rows;) {
        int64_t r1 = r0 + 1;
        while (r1 < rows && dst_row(r1) == dst_row(r1 - 1) + 1) r1++;
        FA_HIP_CHECK(ctx, hipMemcpy(plane + (size_t)dst_row(r0) * cols, from + (size_t)r0 * cols,
                                    (size_t)(r1 - r0) * cols * 2, hipMemcpyHostToDevice));
        r0 = r1;
      }
    }
    return FA_OK;
  };
  auto identity = [](int64_t r) { return r; };
  auto put_norm = [&](float* dst, int64_t n) -> int {
    std::vector<float> v(n);
    for (int64_t i = 0; i < n; i++) {
      float w;
      if (dtype == FA_DT_BF16) {
        uint32_t u = (uint32_t)((const uint16_t*)data)[i] << 16;
        std::memcpy(&w, &u, 4);
      } else {
        w = ((const float*)data)[i];
      }
      v[i] = v2 ? w : w + 1.0f;  // Gemma 3's (1 + w); EmbeddingGemma 2 uses w itself (model.go:128-140)
    }
    FA_HIP_CHECK(ctx, hipMemcpy(dst, v.data(), n * 4, hipMemcpyHostToDevice));
    return FA_OK;
  };
  int rc = FA_OK;
  int l;
  std::string rest;
  if (s == "embed_tokens.weight") {
    if (!shape_is({c.vocab_size, d})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
    rc = put_matrix(m->embed, c.vocab_size, d, identity);
  } else if (s == "norm.weight") {
    if (!shape_is({d})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
    rc = put_norm(m->g_final, d);
  } else if (v2 && s == "ple.per_layer_model_projection.weight") {
    if (!shape_is({(int64_t)c.num_hidden_layers * P, d}))
      return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
    rc = put_matrix(m->wple_model, (int64_t)c.num_hidden_layers * P, d, identity);
  } else if (v2 && s == "ple.per_layer_projection_norm.weight") {
    if (!shape_is({P})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
    rc = put_norm(m->g_ple_norm, P);
  } else if (v2 && s == "embedding_projection.weight") {
    if (!shape_is({m->E, d})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
    rc = put_matrix(m->wemb_proj, m->E, d, identity);
  } else if (s.rfind("dense.", 0) == 0 && s.size() > 6) {
    char* end = nullptr;
    long i = std::strtol(s.c_str() + 6, &end, 10);
    if (i < 0 || i >= c.n_dense || std::string(end) != ".linear.weight")
      return set_error(ctx, FA_ERR_ARG, "gemma: weight \"%s\" not found", name);
    if (!shape_is({m->dense_out[i], m->dense_in[i]}))
      return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
    rc = put_matrix(m->dense[i], m->dense_out[i], m->dense_in[i], identity);
  } else if (fa::parse_layer(s, c.num_hidden_layers, &l, &rest) == 0) {
    fa::Layer& L = m->layers[l];
    const int D = L.D, Hkv = L.Hkv;
    if (rest == "input_layernorm.weight" || rest == "post_attention_layernorm.weight" ||
        rest == "pre_feedforward_layernorm.weight" || rest == "post_feedforward_layernorm.weight") {
      if (!shape_is({d})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
      float* dst = rest[0] == 'i' ? L.g_in : rest[1] == 'o' ? (rest[5] == 'a' ? L.g_post_attn : L.g_post_ffn) : L.g_pre_ffn;
      rc = put_norm(dst, d);
    } else if (rest == "self_attn.q_norm.weight" || rest == "self_attn.k_norm.weight") {
      if (!shape_is({D})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
      rc = put_norm(rest[10] == 'q' ? L.g_q : L.g_k, D);
    } else if (rest == "self_attn.q_proj.weight") {
      if (!shape_is({H * D, d})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
      rc = put_matrix(L.wqkv, H * D, d, identity);
    } else if (rest == "self_attn.k_proj.weight") {
      if (!shape_is({Hkv * D, d})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
      rc = put_matrix(L.wqkv, Hkv * D, d, [o = (int64_t)H * D](int64_t r) { return o + r; });
    } else if (rest == "self_attn.v_proj.weight") {
      if (!shape_is({Hkv * D, d})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
      rc = put_matrix(L.wqkv, Hkv * D, d, [o = (int64_t)(H + Hkv) * D](int64_t r) { return o + r; });
    } else if (rest == "self_attn.o_proj.weight") {
      if (!shape_is({d, H * D})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
      rc = put_matrix(L.wo, d, H * D, identity);
    } else if (rest == "mlp.gate_proj.weight" || rest == "mlp.up_proj.weight") {
      if (!shape_is({F, d})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
      const int64_t off = rest[4] == 'g' ? 0 : 32;  // gate rows first in each 64-row group, then up
      rc = put_matrix(L.wgu, F, d, [off](int64_t r) { return (r / 32) * 64 + off + (r % 32); });
    } else if (rest == "mlp.down_proj.weight") {
      if (!shape_is({d, F})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
      rc = put_matrix(L.wdown, d, F, identity);
    } else if (v2 && rest == "ple_block.per_layer_input_gate.weight") {
      if (!shape_is({P, d})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
      rc = put_matrix(L.wple_gate, P, d, identity);
    } else if (v2 && rest == "ple_block.per_layer_projection.weight") {
      if (!shape_is({d, P})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
      rc = put_matrix(L.wple_proj, d, P, identity);
    } else if (v2 && rest == "ple_block.post_per_layer_input_norm.weight") {
      if (!shape_is({d})) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
      rc = put_norm(L.g_ple_post, d);
    } else if (v2 && rest == "layer_scalar") {
      // one value (model.go:183-188); the checkpoint stores it with shape [1]
      if (!(shape_is({1}) || ndim == 0)) return set_error(ctx, FA_ERR_ARG, "gemma: %s shape %s", name, shape_str().c_str());
      if (dtype == FA_DT_BF16) {
        const uint32_t u = (uint32_t)((const uint16_t*)data)[0] << 16;
        std::memcpy(&L.scalar, &u, 4);
      } else {
        L.scalar = ((const float*)data)[0];
      }
    } else {
      return set_error(ctx, FA_ERR_ARG, "gemma: weight \"%s\" not found", name);
    }
  } else {
    return set_error(ctx, FA_ERR_ARG, "gemma: weight \"%s\" not found", name);
  }
  if (rc) return rc;
  m->seen.insert(s);
  m->finalized = false;
  return FA_OK;
}

int fa_gemma_finalize(fa_model* m) {
  if (!m) return set_error(nullptr, FA_ERR_ARG, "gemma: NULL model");
  fa_ctx* ctx = m->ctx;
  const fa_gemma_config& c = m->cfg;
  const size_t expected = m->variant == 2 ? 5 + (size_t)c.n_dense + 17 * (size_t)c.num_hidden_layers
                                          : 2 + (size_t)c.n_dense + 13 * (size_t)c.num_hidden_layers;
  if (m->seen.size() != expected)
    return set_error(ctx, FA_ERR_STATE, "gemma: %zu of %zu weights set", m->seen.size(), expected);
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "gemma");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  std::vector<int32_t> pos(c.max_tokens);
  for (int t = 0; t < c.max_tokens; t++) pos[t] = t;
  std::vector<float> cs, sn;
  const double local = c.rope_local_base_freq != 0 ? c.rope_local_base_freq : 10000.0;
  const double global = c.rope_theta != 0 ? c.rope_theta : 10000.0;
  if (m->d_local) {
    fa::rope_tables_host(local, pos.data(), c.max_tokens, m->d_local, cs, sn);
    FA_HIP_CHECK(ctx, hipMemcpy(m->cos_local, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    FA_HIP_CHECK(ctx, hipMemcpy(m->sin_local, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
  }
  if (m->d_global) {
    fa::rope_tables_host(global, pos.data(), c.max_tokens, m->d_global, cs, sn);
    FA_HIP_CHECK(ctx, hipMemcpy(m->cos_global, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    FA_HIP_CHECK(ctx, hipMemcpy(m->sin_global, sn.data(), sn.size() * 4, hipMemcpyHostToDevice));
  }
  m->finalized = true;
  return FA_OK;
}

}  // extern "C"

namespace fa {
namespace {

// The forward pass over device-resident ids. With hidden == nullptr: every
// layer, pooling, the head and L2 into d_out [B x dim]. With hidden != nullptr
// (encode): the packed rows [M x d] of the final hidden states (n_layers < 0)
// or of the residual stream after the first n_layers layers into hidden;
// d_out and dim are unused.
int forward(fa_model* m, const int32_t* d_ids, const int32_t* lengths, int32_t B, int32_t T, int32_t dim,
            float* d_out, int n_layers, float* hidden) {
  if (!m) return set_error(nullptr, FA_ERR_ARG, "gemma: NULL model");
  fa_ctx* ctx = m->ctx;
  const fa_gemma_config& c = m->cfg;
  if (!m->finalized) return set_error(ctx, FA_ERR_STATE, "gemma: embed before every weight was set (finalize)");
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "gemma");
    if (rc_) return rc_;
  }
  if (B < 0 || T < 0) return set_error(ctx, FA_ERR_ARG, "gemma: negative batch shape [%d x %d]", B, T);
  if (B == 0) return FA_OK;
  if (!d_ids || !lengths || !(hidden ? hidden : d_out)) return set_error(ctx, FA_ERR_ARG, "gemma: NULL buffer");
  if (T > c.max_tokens) return set_error(ctx, FA_ERR_ARG, "gemma: T=%d exceeds max_tokens %d", T, c.max_tokens);
  const bool v2 = m->variant == 2;
  const int d = c.hidden_size, H = c.num_attention_heads, F = c.intermediate_size, NL = c.num_hidden_layers,
            P = m->P;
  if (hidden && n_layers > NL)
    return set_error(ctx, FA_ERR_ARG, "gemma: encode after %d layers, the model has %d", n_layers, NL);
  const bool final_states = !hidden || n_layers < 0;
  const int n_run = final_states ? NL : n_layers;
  const int full = c.n_dense > 0 ? m->dense_out.back() : (v2 ? m->E : d);
  if (dim <= 0) dim = full;
  if (dim > full) return set_error(ctx, FA_ERR_ARG, "gemma: Dim(%d) outside 1..%d", dim, full);
  // ---- plan (host): cu_seqlens, micro-batch groups, attention work items ----
  int64_t M = 0;
  double sum_l2 = 0;
  for (int b = 0; b < B; b++) {
    if (lengths[b] < 1 || lengths[b] > T)
      return set_error(ctx, FA_ERR_ARG, "gemma: length[%d] = %d outside 1..T=%d", b, lengths[b], T);
    M += lengths[b];
    sum_l2 += (double)lengths[b] * lengths[b];
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  const int cus = ctx->cu_count > 0 ? ctx->cu_count : 256;
  // Micro-batches: with enough tokens the sequences are cut into groups of
  // about equal token count (contiguous rows) whose layers run on separate
  // streams, so that one group's kernels occupy the CUs the others leave
  // idle (the last round of GEMM tiles and attention items, the norms'
  // low-occupancy phases). Not while profiling: the probes time one stream.
  // Group g holds sequences [gb[g], gb[g+1]).
  int gb[fa::kMaxMicrobatches + 1] = {0, B};
  int groups = 1;
  if (M >= fa::microbatch_min_rows() && !m->profiling)
    groups = fa::plan_groups(lengths, B, M, fa::microbatch_count(M, sum_l2), gb);
  // each layer's attention path, the items and their key runs
  std::vector<int>& layer_D = m->plan_layer_D;
  std::vector<int>& layer_Hkv = m->plan_layer_Hkv;
  layer_D.resize(m->layers.size());
  layer_Hkv.resize(m->layers.size());
  for (size_t l = 0; l < m->layers.size(); l++) {
    layer_D[l] = m->layers[l].D;
    layer_Hkv[l] = m->layers[l].Hkv;
  }
  fa::AttnPlanIn pin;
  pin.lengths = lengths; pin.B = B; pin.T = T; pin.H = H;
  pin.layer_D = layer_D.data(); pin.layer_Hkv = layer_Hkv.data();
  pin.n_layers = (int)m->layers.size(); pin.n_run = n_run;
  pin.groups = groups; pin.gb = gb; pin.cus = cus;
  pin.tile_keys = fa::attention_tiles_keys(); pin.varlen_qblock = fa::attention_varlen_qblock();
  pin.max_key_parts = fa::kMaxKeyParts; pin.split_rows = fa::kAttnSplitRows;
  pin.forced_key_parts = fa::attention_key_parts_forced();
  pin.forced_rows = fa::attention_rows_forced();
  pin.forced_xcd = fa::attention_xcd_forced();
  pin.tile_min_rows = fa::tile_min_rows();
  fa::AttnPlan ap;
  fa::plan_attention(pin, ap);
  const int64_t n_items_t = ap.n_items_t, n_items = ap.n_items_t + ap.n_items_v, n_tiles = ap.n_tiles;
  const int hkv_t = ap.hkv_t, kparts_t = ap.kparts_t, kparts_v = ap.kparts_v, waves_t = ap.waves_t;
  const int tkeys = pin.tile_keys;
  // plan buffer: cu_seqlens, items, first tile per sequence, then (16-byte
  // aligned) each item's extent (its sequence's first packed row, length and
  // first tile) and each key tile's (its first packed row, keys, first key's
  // position), which the attention and the key/value image kernels read
  // beside the item or tile (no dependent load through a sequence table)
  const size_t ext_off = (2 * (size_t)(B + 1) + 3 * (size_t)n_items + 3) & ~(size_t)3;
  const size_t plan_ints = ext_off + 4 * (size_t)(n_items + n_tiles);
  if (m->plan_pending) {
    FA_HIP_CHECK(ctx, hipEventSynchronize(m->plan_done));  // previous upload has read the pinned buffer
    m->plan_pending = false;
  }
  if (plan_ints > m->plan_host_ints) {
    if (m->plan_host) (void)hipHostFree(m->plan_host);
    m->plan_host = nullptr;
    size_t n = plan_ints * 2;
    FA_HIP_CHECK(ctx, hipHostMalloc((void**)&m->plan_host, n * 4, hipHostMallocDefault));
    m->plan_host_ints = n;
  }
  int32_t* cu_h = m->plan_host;
  int32_t* items_h = m->plan_host + (B + 1);
  int32_t* cut_h = items_h + 3 * n_items;
  cu_h[0] = 0;
  cut_h[0] = 0;
  for (int b = 0; b < B; b++) {
    cu_h[b + 1] = cu_h[b] + lengths[b];
    cut_h[b + 1] = cut_h[b] + (ap.any_tiles ? (lengths[b] + tkeys - 1) / tkeys : 0);
  }
  fa::plan_items(pin, ap, items_h, m->seq_order);
  {
    int32_t* ext_h = m->plan_host + ext_off;
    for (int64_t i = 0; i < n_items; i++) {
      const int b = items_h[3 * i];
      ext_h[4 * i] = cu_h[b];
      ext_h[4 * i + 1] = lengths[b];
      ext_h[4 * i + 2] = cut_h[b];
      ext_h[4 * i + 3] = 0;
    }
    int32_t* text_h = ext_h + 4 * n_items;
    for (int b = 0; b < B; b++)
      for (int q = cut_h[b]; q < cut_h[b + 1]; q++) {
        const int t0 = tkeys * (q - cut_h[b]);
        text_h[4 * q] = cu_h[b] + t0;
        text_h[4 * q + 1] = std::min(tkeys, lengths[b] - t0);
        text_h[4 * q + 2] = t0;
        text_h[4 * q + 3] = 0;
      }
  }
  const int64_t* group_items_t = ap.group_items_t;
  const int64_t* group_items_v = ap.group_items_v;
  int rc;
  if ((rc = m->plan_dev.ensure(ctx, plan_ints * 4 + (size_t)M * 8))) return rc;
  int32_t* cu_d = m->plan_dev.as<int32_t>();
  int32_t* items_d = cu_d + (B + 1);
  const int32_t* ext_d = cu_d + ext_off;  // [n_items][4], 16-byte aligned
  const int32_t* text_d = ext_d + 4 * n_items;  // [n_tiles][4]
  int32_t* row_src_d = cu_d + plan_ints;   // [M] b*T + t
  int32_t* pos_d = row_src_d + M;          // [M] t
  FA_HIP_CHECK(ctx, hipMemcpyAsync(cu_d, m->plan_host, plan_ints * 4, hipMemcpyHostToDevice, ctx->stream));
  FA_HIP_CHECK(ctx, hipEventRecord(m->plan_done, ctx->stream));
  m->plan_pending = true;
  // ---- workspace ----
  // o has room for two partial products of the K-split o/down GEMMs
  // variant 2 adds the per-layer inputs [M, layers*P]; its [M, P] gate
  // output reuses gu (free after the down product)
  const int ksplit = fa::gemm_ksplit();
  // a few-row batch on one stream may split those products in four
  const bool few_rows = groups == 1 && ksplit > 1 && ((M + 31) / 32) * ((d + 63) / 64) * 4 <= cus;
  const int ks_max = few_rows ? std::max(ksplit, fa::small_ksplit()) : ksplit;
  const int64_t ncols = 2LL * d + m->max_width + m->max_hd + (int64_t)ks_max * d + std::max(F, P) +
                        (v2 ? (int64_t)NL * P : 0);
  int maxw = std::max(d, std::max(full, v2 ? m->E : d));
  for (int o : m->dense_out) maxw = std::max(maxw, o);
  const int kparts_max = std::max(kparts_t, kparts_v);
  const int64_t part_floats = kparts_max > 1 ? fa::attention_part_floats(kparts_max, M, H, m->max_hd / H) : 0;
  // key/value tile images: [tile][Hkv][key | value][3 * 32 * 256] bf16
  const size_t img_bytes = (size_t)n_tiles * hkv_t * 2 * (3 * 32 * 256) * 2;
  const size_t f32_bytes = ((size_t)M * ncols + (size_t)B * (d + 2 * (size_t)maxw) + (size_t)part_floats) * 4 + 256;
  const size_t img_off = (f32_bytes + 255) & ~(size_t)255;
  const size_t ws_bytes = img_off + img_bytes + 4096;
  if ((rc = m->ws.ensure(ctx, ws_bytes))) return rc;
  uint16_t* img = reinterpret_cast<uint16_t*>(m->ws.as<char>() + img_off);
  float* x = m->ws.as<float>();
  float* xn = x + M * d;
  float* qkv = xn + M * d;
  float* att = qkv + M * m->max_width;
  float* o = att + M * m->max_hd;
  float* gu = o + (int64_t)ks_max * M * d;
  float* ple = gu + M * std::max(F, P);
  float* pooled = ple + (v2 ? M * NL * P : 0);
  float* hbuf0 = pooled + (size_t)B * d;
  float* hbuf1 = hbuf0 + (size_t)B * maxw;
  float* attn_part = reinterpret_cast<float*>((reinterpret_cast<uintptr_t>(hbuf1 + (size_t)B * maxw) + 255) &
                                              ~(uintptr_t)255);
  hipStream_t s = ctx->stream;
  // ---- row plan on device ----
  if ((rc = fa::launch_row_plan(ctx, cu_d, B, T, M, row_src_d, pos_d, s))) return rc;
  const float eps = c.rms_norm_eps;
  const float emb_scale = (float)std::sqrt((double)d);  // embed.go:176
  // model.go:100; variant 2 does not scale the scores (model.go:105-110)
  const float att_scale = v2 ? 1.f : (float)(1.0 / std::sqrt(c.query_pre_attn_scalar));
  // window bound (config.go:331-339): variant 2 reads an inclusive radius
  const int wbound = v2 ? c.sliding_window + 1 : c.use_bidirectional ? c.sliding_window / 2 + 1 : c.sliding_window;
  {
    fa::Probe pr(m, FA_K_GATHER, 0, (double)M * (2.0 * d + 8.0 * d + 4));
    if ((rc = fa::launch_embed_gather(ctx, d_ids, row_src_d, m->embed.p, m->embed.terms == 3 ? m->embed.plane() : 0,
                                      c.vocab_size, M, d, emb_scale, m->layers[0].g_in, eps, x, xn, s)))
      return rc;
    pr.done();
  }
  if (v2) {
    // per-layer inputs: RMSNorm(x0 . W_ple^T * hidden^-1/2) per layer (embed.go:274-279)
    {
      fa::GemmArgs g;
      g.m = M; g.n = (int64_t)NL * P; g.k = d; g.a = x; g.lda = d; fa::set_b(g, m->wple_model); g.c = ple;
      g.ldc = (int64_t)NL * P;
      fa::Probe pr(m, FA_K_GEMM_PLE, 2.0 * M * NL * P * d, 0);
      if ((rc = fa::launch_gemm(ctx, g, s))) return rc;
      pr.done();
    }
    fa::Probe pr(m, FA_K_PLE_NORM, 0, (double)M * NL * P * 8.0);
    if ((rc = fa::launch_ple_norm(ctx, ple, M, NL, P, (float)(1 / std::sqrt((double)d)), m->g_ple_norm, eps, s)))
      return rc;
    pr.done();
  }
  // one layer over rows [r0, r0 + rows) (the sequences of one group, whose
  // attention items are items_t[0, n_it_t) for a tile layer, items_v[0,
  // n_it_v) otherwise) on stream st
  auto run_layer = [&](int l, int b0, int b1, const int32_t* items_t, int64_t n_it_t, const int32_t* items_v,
                       int64_t n_it_v, hipStream_t st) -> int {
    const int64_t r0 = cu_h[b0], rows = cu_h[b1] - r0;
    const fa::Layer& L = m->layers[l];
    const int D = L.D, Hkv = L.Hkv;
    const bool sliding = L.sliding;
    const bool tiles = ap.layer_tiles(D);
    // The N = hidden products (o, down, per-layer-input projection) split K
    // in two when their 128x128 tiles, counted over the concurrent groups,
    // give the CUs fewer than two each (C2: one stream 5 517 rows, or three
    // groups of about 1 840: 4 % faster split); with more tiles the second
    // partial's writes and reads cost more than the fill gains (C5's three
    // groups of about 5 970 rows: 4.7 % faster unsplit).
    const int64_t n_tiles = ((rows + 127) / 128) * ((d + 127) / 128) * groups;
    const int ks = n_tiles < 2LL * cus ? ks_max : 1;
    // per product: the most parts (ks, halved as needed) that divide K into
    // whole 32-wide slabs
    auto parts = [&](int64_t K) {
      int k = ks;
      while (k > 1 && K % (32 * k) != 0) k /= 2;
      return k;
    };
    const int ks_o = parts(H * D), ks_down = parts(F), ks_ple = parts(P);
    const float* o2_o = ks_o > 1 ? o + M * d + r0 * d : nullptr;
    const float* o2_dn = ks_down > 1 ? o + M * d + r0 * d : nullptr;
    const float* o2_pl = ks_ple > 1 ? o + M * d + r0 * d : nullptr;
    float* const xr = x + r0 * d;
    float* const xnr = xn + r0 * d;
    // per-group regions of the buffers whose row width changes with the
    // layer (EmbeddingGemma 2's head dims) or the product (gate|up vs the
    // per-layer-input gate): groups on other streams may be at other
    // layers, so each writes only inside [r0, r0 + rows) x the widest row
    float* const qkvr = qkv + r0 * m->max_width;
    float* const attr = att + r0 * m->max_hd;
    float* const gur = gu + r0 * std::max(F, P);
    float* const or_ = o + r0 * d;
    int rc;
    // a few-row batch on the fp32 attention path splits the q|k|v product
    // in K: its second part goes to o's planes (free until the o product)
    // and the q/k norm pass adds it
    const bool qkv_split = few_rows && !tiles && fa::qkv_ksplit() > 1 && d % 64 == 0 &&
                           (int64_t)ks_max * d >= m->max_width;
    const float* qkv2 = qkv_split ? o : nullptr;
    {
      fa::GemmArgs g;
      g.shared = groups > 1;
      g.m = rows; g.n = L.width; g.k = d; g.a = xnr; g.lda = d; fa::set_b(g, L.wqkv); g.c = qkvr; g.ldc = L.width;
      if (qkv_split) {
        g.ksplit = 2;
        g.c_split = o - qkvr;
      }
      fa::Probe pr(m, FA_K_GEMM_QKV, 2.0 * rows * L.width * d, 0);
      if ((rc = fa::launch_gemm(ctx, g, st))) return rc;
      pr.done();
    }
    if (tiles) {
      // read k and v (4 bytes per element); write their images (6 bytes per
      // element each, tiles padded to 32 tokens); q is normed and rotated
      // by the attention as it loads it
      const int64_t ntl = cut_h[b1] - cut_h[b0];
      // (variant 2 norms the values too: each value half-block also reads
      // the other half of its keys' values for the sum of squares)
      fa::Probe pr(m, FA_K_QKNORM_ROPE, 0,
                   (double)rows * (v2 ? 3 : 2) * Hkv * 4.0 * D + (double)ntl * Hkv * 2 * 3 * 32 * 256 * 2);
      if ((rc = fa::launch_kv_tiles(ctx, qkvr, r0, H, Hkv, L.g_k, eps, L.cos_t, L.sin_t, text_d, cut_h[b0],
                                    (int32_t)ntl, img, st, v2)))
        return rc;
      pr.done();
    } else {
      fa::Probe pr(m, FA_K_QKNORM_ROPE, 0, (double)rows * (H + (v2 ? 2 : 1) * Hkv) * D * 8.0);
      // a group of one sequence: row i is token i, no position table
      const int32_t* gpos = b1 - b0 == 1 ? nullptr : pos_d + r0;
      if ((rc = fa::launch_qknorm_rope(ctx, qkvr, rows, H, Hkv, D, L.g_q, L.g_k, eps, gpos, L.cos_t, L.sin_t,
                                       st, v2, qkv2)))
        return rc;
      pr.done();
    }
    {
      fa::AttnVarlenArgs a;
      a.qkv = qkvr; a.out = attr; a.row0 = r0;
      a.item_ext = ext_d + 4 * ((items_v - items_d) / 3);
      a.H = H; a.Hkv = Hkv; a.D = D; a.scale = att_scale;
      a.window = (sliding && c.sliding_window > 0) ? wbound : 0;
      if (kparts_v > 1) {
        a.kparts = kparts_v; a.rows = rows; a.part = attn_part;
      }
      double pairs = 0;
      if (m->profiling) {
        for (int b = 0; b < B; b++) {
          const double Lb = lengths[b];
          if (a.window > 0 && Lb > a.window) {
            // sum over i of |{j : |i-j| < w}| = L(2w-1) - w(w-1)
            pairs += Lb * (2.0 * a.window - 1) - (double)a.window * (a.window - 1);
          } else {
            pairs += Lb * Lb;
          }
        }
      }
      fa::Probe pr(m, FA_K_ATTENTION, pairs * 4.0 * H * D, 0);
      if (tiles) {
        fa::AttnTilesArgs at;
        at.qkv = qkvr; at.img = img; at.out = attr; at.row0 = r0;
        at.item_ext = ext_d + 4 * ((items_t - items_d) / 3);
        at.H = H; at.Hkv = Hkv; at.window = a.window; at.scale = a.scale;
        at.gq = L.g_q; at.eps = eps; at.cos_t = L.cos_t; at.sin_t = L.sin_t; at.waves = waves_t;
        if (kparts_t > 1) {
          at.kparts = kparts_t; at.rows = M; at.nrows = rows; at.part = attn_part;
        }
        if ((rc = fa::launch_attention_tiles(ctx, at, items_t, (int32_t)n_it_t, st))) return rc;
      } else {
        if ((rc = fa::launch_attention_varlen_items(ctx, a, items_v, (int32_t)n_it_v, st))) return rc;
      }
      pr.done();
    }
    {
      fa::GemmArgs g;
      g.shared = groups > 1;
      g.m = rows; g.n = d; g.k = H * D; g.a = attr; g.lda = H * D; fa::set_b(g, L.wo); g.c = or_;
      g.ldc = d; g.ksplit = ks_o; g.c_split = M * d;
      fa::Probe pr(m, FA_K_GEMM_O, 2.0 * rows * d * H * D, 0);
      if ((rc = fa::launch_gemm(ctx, g, st))) return rc;
      pr.done();
    }
    {
      fa::Probe pr(m, FA_K_RESIDUAL_NORM, 0, fa::resnorm_bytes(rows, d, ks_o, L.g_pre_ffn));
      if ((rc = fa::launch_residual_norm(ctx, or_, xr, xnr, rows, d, L.g_post_attn, L.g_pre_ffn, eps, st, o2_o, 1.f,
                                         ks_o - 1, M * d)))
        return rc;
      pr.done();
    }
    {
      fa::GemmArgs g;
      g.shared = groups > 1;
      g.m = rows; g.n = 2 * F; g.k = d; g.a = xnr; g.lda = d; fa::set_b(g, L.wgu); g.c = gur; g.ldc = F;
      g.epi = fa::Epi::GeGLU;
      fa::Probe pr(m, FA_K_GEMM_GATEUP, 2.0 * rows * 2 * F * d, 0);
      if ((rc = fa::launch_gemm(ctx, g, st))) return rc;
      pr.done();
    }
    {
      fa::GemmArgs g;
      g.shared = groups > 1;
      g.m = rows; g.n = d; g.k = F; g.a = gur; g.lda = F; fa::set_b(g, L.wdown); g.c = or_; g.ldc = d;
      g.ksplit = ks_down; g.c_split = M * d;
      fa::Probe pr(m, FA_K_GEMM_DOWN, 2.0 * rows * d * F, 0);
      if ((rc = fa::launch_gemm(ctx, g, st))) return rc;
      pr.done();
    }
    // the last layer's "next norm" is the final RMSNorm (embed.go:237): xn = h
    const float* g_next = (l + 1 < NL) ? m->layers[l + 1].g_in : m->g_final;
    {
      // variant 2: the per-layer-input block reads x itself, so no norm here
      fa::Probe pr(m, FA_K_RESIDUAL_NORM, 0, fa::resnorm_bytes(rows, d, ks_down, v2 ? nullptr : g_next));
      if ((rc = fa::launch_residual_norm(ctx, or_, xr, xnr, rows, d, L.g_post_ffn, v2 ? nullptr : g_next, eps, st,
                                         o2_dn, 1.f, ks_down - 1, M * d)))
        return rc;
      pr.done();
    }
    if (v2) {
      // x = (x + RMSNorm(gelu(x . Wg^T) * ple_l . Wp^T; g)) * scalar (embed.go:359-371)
      {
        fa::GemmArgs g;
        g.shared = groups > 1;
        g.m = rows; g.n = P; g.k = d; g.a = xr; g.lda = d; fa::set_b(g, L.wple_gate); g.c = gur; g.ldc = P;
        g.epi = fa::Epi::Generic; g.act = FA_ACT_GELU; g.mul = ple + r0 * NL * P + (int64_t)l * P;
        g.ldm = (int64_t)NL * P;
        fa::Probe pr(m, FA_K_GEMM_PLE, 2.0 * rows * P * d, 0);
        if ((rc = fa::launch_gemm(ctx, g, st))) return rc;
        pr.done();
      }
      {
        fa::GemmArgs g;
        g.shared = groups > 1;
        g.m = rows; g.n = d; g.k = P; g.a = gur; g.lda = P; fa::set_b(g, L.wple_proj); g.c = or_; g.ldc = d;
        g.ksplit = ks_ple; g.c_split = M * d;
        fa::Probe pr(m, FA_K_GEMM_PLE, 2.0 * rows * d * P, 0);
        if ((rc = fa::launch_gemm(ctx, g, st))) return rc;
        pr.done();
      }
      fa::Probe pr(m, FA_K_RESIDUAL_NORM, 0, fa::resnorm_bytes(rows, d, ks_ple, g_next));
      if ((rc = fa::launch_residual_norm(ctx, or_, xr, xnr, rows, d, L.g_ple_post, g_next, eps, st, o2_pl, L.scalar,
                                         ks_ple - 1, M * d)))
        return rc;
      pr.done();
    }
    return FA_OK;
  };
  if (groups == 1) {
    for (int l = 0; l < n_run; l++)
      if ((rc = run_layer(l, 0, B, items_d, group_items_t[0], items_d + 3 * n_items_t, group_items_v[0], s)))
        return rc;
  } else {
    // groups 1.. run on their own streams once the embeddings (and plan) are in
    FA_HIP_CHECK(ctx, hipEventRecord(m->ev_fork, s));
    for (int g = 1; g < groups; g++) FA_HIP_CHECK(ctx, hipStreamWaitEvent(m->mb_stream[g], m->ev_fork, 0));
    rc = FA_OK;
    for (int l = 0; l < n_run && !rc; l++) {
      int64_t it0 = 0, iv0 = n_items_t;  // the group's first tile item, first fp32 item
      for (int g = 0; g < groups && !rc; g++) {
        rc = run_layer(l, gb[g], gb[g + 1], items_d + 3 * it0, group_items_t[g], items_d + 3 * iv0, group_items_v[g],
                       g ? m->mb_stream[g] : s);
        it0 += group_items_t[g];
        iv0 += group_items_v[g];
      }
    }
    // joined also after an error: later calls reuse the workspace on s
    for (int g = 1; g < groups; g++) {
      FA_HIP_CHECK(ctx, hipEventRecord(m->ev_join[g], m->mb_stream[g]));
      FA_HIP_CHECK(ctx, hipStreamWaitEvent(s, m->ev_join[g], 0));
    }
    if (rc) return rc;
  }
  if (hidden) {
    // after the last layer xn holds the final RMSNorm of x (embed.go:237)
    const float* src = final_states ? xn : x;
    FA_HIP_CHECK(ctx, hipMemcpyAsync(hidden, src, (size_t)M * d * 4, hipMemcpyDeviceToDevice, s));
    return FA_OK;
  }
  {
    fa::Probe pr(m, FA_K_POOL_L2, 0, (double)M * d * 4.0 + (double)B * d * 4.0);
    if ((rc = fa::launch_pool(ctx, xn, cu_d, B, d, pooled, s))) return rc;
    pr.done();
  }
  const float* cur = pooled;
  int cur_w = d;
  float* bufs[2] = {hbuf0, hbuf1};
  int nb = 0;
  if (v2) {  // the embedding projection, applied to the pooled vector (embed.go:408-414)
    fa::GemmArgs g;
    g.m = B; g.n = m->E; g.k = d; g.a = pooled; g.lda = d; fa::set_b(g, m->wemb_proj); g.c = bufs[0]; g.ldc = m->E;
    fa::Probe pr(m, FA_K_GEMM_HEAD, 2.0 * B * m->E * d, 0);
    if ((rc = fa::launch_gemm(ctx, g, s))) return rc;
    pr.done();
    cur = bufs[0];
    cur_w = m->E;
    nb = 1;
  }
  // the last dense product splits K (its few rows give few tiles: 3072 -> 768
  // for one pooled row is 12 of them) and the L2 norm adds the partials,
  // unless a Tanh follows it (model.go:296-301, embed.go:415-418: applied in
  // the product's epilogue, so on the whole sum) or K splits are off
  int head_parts = 1;
  for (int i = 0; i < c.n_dense; i++) {
    fa::GemmArgs g;
    g.m = B; g.n = m->dense_out[i]; g.k = cur_w; g.a = cur; g.lda = cur_w; fa::set_b(g, m->dense[i]);
    g.c = bufs[(i + nb) & 1]; g.ldc = m->dense_out[i];
    if (m->dense_act[i] == FA_ACT_TANH) {
      g.epi = fa::Epi::Generic;
      g.act = FA_ACT_TANH;
    } else if (i + 1 == c.n_dense && ksplit > 1) {
      for (int ks : {4, 2})
        if (cur_w % (32 * ks) == 0 && (int64_t)ks * m->dense_out[i] <= maxw) {
          head_parts = ks;
          break;
        }
      g.ksplit = head_parts; g.c_split = (int64_t)B * m->dense_out[i];
    }
    fa::Probe pr(m, FA_K_GEMM_HEAD, 2.0 * B * m->dense_out[i] * cur_w, 0);
    if ((rc = fa::launch_gemm(ctx, g, s))) return rc;
    pr.done();
    cur = bufs[(i + nb) & 1];
    cur_w = m->dense_out[i];
  }
  {
    fa::Probe pr(m, FA_K_POOL_L2, 0, (double)B * dim * 8.0);
    if ((rc = fa::launch_l2norm(ctx, cur, B, cur_w, dim, d_out, s, head_parts,
                                (int64_t)B * cur_w)))
      return rc;
    pr.done();
  }
  return FA_OK;
}

}  // namespace
}  // namespace fa

extern "C" {

int fa_gemma_embed_ids_dev(fa_model* m, const int32_t* d_ids, const int32_t* lengths, int32_t B, int32_t T,
                           int32_t dim, float* d_out) {
  return fa::forward(m, d_ids, lengths, B, T, dim, d_out, 0, nullptr);
}

int fa_gemma_encode_ids_dev(fa_model* m, const int32_t* d_ids, const int32_t* lengths, int32_t B, int32_t T,
                            int32_t n_layers, float* d_hidden) {
  return fa::forward(m, d_ids, lengths, B, T, 0, nullptr, n_layers < 0 ? -1 : n_layers, d_hidden);
}

int fa_gemma_encode_ids(fa_model* m, const int32_t* ids, const int32_t* lengths, int32_t B, int32_t T,
                        int32_t n_layers, float* hidden) {
  if (!m) return set_error(nullptr, FA_ERR_ARG, "gemma: NULL model");
  fa_ctx* ctx = m->ctx;
  if (B < 0 || T < 0) return set_error(ctx, FA_ERR_ARG, "gemma: negative batch shape [%d x %d]", B, T);
  if (B == 0) return FA_OK;
  if (!ids || !lengths || !hidden) return set_error(ctx, FA_ERR_ARG, "gemma: NULL buffer");
  int rc;
  if ((rc = fa::check_ids(m, ids, lengths, B, T))) return rc;
  int64_t M = 0;
  for (int b = 0; b < B; b++) M += lengths[b];
  const int d = m->cfg.hidden_size;
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "gemma");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  if ((rc = m->ids_dev.ensure(ctx, (size_t)B * T * 4))) return rc;
  if ((rc = m->out_dev.ensure(ctx, (size_t)M * d * 4))) return rc;
  char* io;
  const size_t ib = (size_t)B * T * 4, ob = (size_t)M * d * 4;
  if ((rc = fa::io_staging(m, ib + ob, &io))) return rc;
  std::memcpy(io, ids, ib);
  FA_HIP_CHECK(ctx, hipMemcpyAsync(m->ids_dev.ptr, io, ib, hipMemcpyHostToDevice, ctx->stream));
  if ((rc = fa_gemma_encode_ids_dev(m, m->ids_dev.as<int32_t>(), lengths, B, T, n_layers, m->out_dev.as<float>())))
    return rc;
  FA_HIP_CHECK(ctx, hipMemcpyAsync(io + ib, m->out_dev.ptr, ob, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  std::memcpy(hidden, io + ib, ob);
  return FA_OK;
}

int fa_gemma_embed_ids(fa_model* m, const int32_t* ids, const int32_t* lengths, int32_t B, int32_t T, int32_t dim,
                       float* out) {
  if (!m) return set_error(nullptr, FA_ERR_ARG, "gemma: NULL model");
  fa_ctx* ctx = m->ctx;
  if (B < 0 || T < 0) return set_error(ctx, FA_ERR_ARG, "gemma: negative batch shape [%d x %d]", B, T);
  if (B == 0) return FA_OK;
  if (!ids || !lengths || !out) return set_error(ctx, FA_ERR_ARG, "gemma: NULL buffer");
  const fa_gemma_config& c = m->cfg;
  const int full = c.n_dense > 0 ? m->dense_out.back() : (m->variant == 2 ? m->E : c.hidden_size);
  const int dd = dim <= 0 ? full : dim;
  int rc;
  if ((rc = fa::check_ids(m, ids, lengths, B, T))) return rc;
  if (dd > full) return set_error(ctx, FA_ERR_ARG, "gemma: Dim(%d) outside 1..%d", dim, full);
  {
    const int rc_ = fa::refuse_capture(ctx, ctx->stream, "gemma");
    if (rc_) return rc_;
  }
  FA_HIP_CHECK(ctx, hipSetDevice(ctx->device));
  if ((rc = m->ids_dev.ensure(ctx, (size_t)B * T * 4))) return rc;
  if ((rc = m->out_dev.ensure(ctx, (size_t)B * dd * 4))) return rc;
  char* io;
  const size_t ib = (size_t)B * T * 4, ob = (size_t)B * dd * 4;
  if ((rc = fa::io_staging(m, ib + ob, &io))) return rc;
  std::memcpy(io, ids, ib);
  FA_HIP_CHECK(ctx, hipMemcpyAsync(m->ids_dev.ptr, io, ib, hipMemcpyHostToDevice, ctx->stream));
  if ((rc = fa_gemma_embed_ids_dev(m, m->ids_dev.as<int32_t>(), lengths, B, T, dd, m->out_dev.as<float>()))) return rc;
  FA_HIP_CHECK(ctx, hipMemcpyAsync(io + ib, m->out_dev.ptr, ob, hipMemcpyDeviceToHost, ctx->stream));
  FA_HIP_CHECK(ctx, hipStreamSynchronize(ctx->stream));
  std::memcpy(out, io + ib, ob);
  return FA_OK;
}

int fa_gemma_set_profiling(fa_model* m, int enabled) {
  if (!m) return set_error(nullptr, FA_ERR_ARG, "gemma: NULL model");
  m->profiling = enabled != 0;
  return FA_OK;
}

int fa_gemma_kernel_stats(fa_model* m, int kind, int64_t* launches, double* ms, double* flops, double* bytes) {
  if (!m) return set_error(nullptr, FA_ERR_ARG, "gemma: NULL model");
  if (kind < 0 || kind >= FA_K_COUNT) return set_error(m->ctx, FA_ERR_ARG, "gemma: kernel kind %d", kind);
  int rc = fa::collect_stats(m);
  if (rc) return rc;
  const fa::KernelStat& s = m->stats[kind];
  if (launches) *launches = s.launches;
  if (ms) *ms = s.ms;
  if (flops) *flops = s.flops;
  if (bytes) *bytes = s.bytes;
  return FA_OK;
}

int fa_gemma_reset_stats(fa_model* m) {
  if (!m) return set_error(nullptr, FA_ERR_ARG, "gemma: NULL model");
  int rc = fa::collect_stats(m);
  for (auto& s : m->stats) s = fa::KernelStat{};
  return rc;
}

}  // extern "C"
