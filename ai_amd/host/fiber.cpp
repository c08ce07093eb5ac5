// C++ host mirror of fiber/ai's tensor and gemma API on top of the C ABI.
// See fiber.hpp for the mapping to the reference.
#include "fiber.hpp"

#include <sys/stat.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <numeric>
#include <sstream>

#include "json.hpp"
#include "safetensors.hpp"

namespace fiber {

namespace {

fa_ctx* g_ctx = nullptr;
std::once_flag g_once;
std::string g_err;

std::string shape_str(const tensor::Shape& s) {
  std::ostringstream o;
  o << "[";
  for (size_t i = 0; i < s.size(); i++) o << (i ? " " : "") << s[i];
  o << "]";
  return o.str();
}

tensor::Shape contiguous_strides(const tensor::Shape& s) {
  tensor::Shape st(s.size());
  int64_t acc = 1;
  for (int i = (int)s.size() - 1; i >= 0; i--) {
    st[i] = acc;
    acc *= s[i];
  }
  return st;
}

int64_t prod(const tensor::Shape& s) {
  int64_t n = 1;
  for (int64_t v : s) n *= v;
  return n;
}

// Calls fn and maps a non-OK status to tensor::Error{op, message}.
void call(const char* op, int rc) {
  if (rc == FA_OK) return;
  std::string msg = fa_last_error(device());
  if (rc == FA_ERR_ARG) throw tensor::Error(op, msg);
  throw std::runtime_error(std::string("fa_rocm: ") + op + ": " + msg);
}

}  // namespace

fa_ctx* device() {
  std::call_once(g_once, [] {
    if (fa_create(0, &g_ctx) != FA_OK) g_err = fa_last_error(nullptr);
  });
  if (!g_ctx) throw std::runtime_error("fa_rocm: no GPU context: " + g_err);
  return g_ctx;
}

namespace tensor {

[[noreturn]] static void fail(const std::string& op, const std::string& msg) { throw Error(op, msg); }

Tensor Tensor::New(std::vector<float> data, Shape shape) {
  for (int64_t d : shape)
    if (d < 0) fail("New", "negative dimension in " + shape_str(shape));
  if ((int64_t)data.size() != prod(shape))
    fail("New", std::to_string(data.size()) + " values for shape " + shape_str(shape));
  Tensor t;
  t.store_ = std::make_shared<std::vector<float>>(std::move(data));
  t.shape_ = shape;
  t.strides_ = contiguous_strides(shape);
  return t;
}

Tensor Tensor::Zeros(Shape shape) { return New(std::vector<float>(prod(shape), 0.f), shape); }

int64_t Tensor::Size() const { return prod(shape_); }

bool Tensor::IsContiguous() const { return strides_ == contiguous_strides(shape_); }

float Tensor::At(std::initializer_list<int64_t> idx) const {
  if (idx.size() != shape_.size()) fail("At", "index rank does not match " + shape_str(shape_));
  int64_t off = offset_;
  int i = 0;
  for (int64_t v : idx) {
    if (v < 0 || v >= shape_[i]) fail("At", "index out of range for " + shape_str(shape_));
    off += v * strides_[i++];
  }
  return (*store_)[off];
}

std::vector<float> Tensor::Float32s() const {
  const int64_t n = Size();
  std::vector<float> out(n);
  if (n == 0) return out;
  if (IsContiguous()) {
    std::memcpy(out.data(), store_->data() + offset_, n * sizeof(float));
    return out;
  }
  std::vector<int64_t> idx(shape_.size(), 0);
  for (int64_t k = 0; k < n; k++) {
    int64_t off = offset_;
    for (size_t d = 0; d < shape_.size(); d++) off += idx[d] * strides_[d];
    out[k] = (*store_)[off];
    for (int d = (int)shape_.size() - 1; d >= 0; d--) {
      if (++idx[d] < shape_[d]) break;
      idx[d] = 0;
    }
  }
  return out;
}

Tensor Tensor::Contiguous() const {
  if (IsContiguous()) return *this;
  return New(Float32s(), shape_);
}

Tensor Tensor::Reshape(Shape shape) const {
  if (prod(shape) != Size()) fail("Reshape", "cannot reshape " + shape_str(shape_) + " to " + shape_str(shape));
  Tensor t = Contiguous();
  t.shape_ = shape;
  t.strides_ = contiguous_strides(shape);
  return t;
}

Tensor Tensor::Expand(Shape shape) const {
  if (shape.size() < shape_.size()) fail("Expand", "cannot expand " + shape_str(shape_) + " to " + shape_str(shape));
  Tensor t = *this;
  const size_t lead = shape.size() - shape_.size();
  Shape st(shape.size(), 0);
  for (size_t i = 0; i < shape.size(); i++) {
    if (i < lead) continue;  // new leading dimension: stride 0
    const int64_t have = shape_[i - lead];
    if (have == shape[i]) st[i] = strides_[i - lead];
    else if (have == 1) st[i] = 0;
    else fail("Expand", "cannot expand " + shape_str(shape_) + " to " + shape_str(shape));
  }
  t.shape_ = shape;
  t.strides_ = st;
  return t;
}

Tensor Tensor::T() const {
  if (shape_.size() != 2) fail("T", "expected a 2-D tensor, got " + shape_str(shape_));
  Tensor t = *this;
  std::swap(t.shape_[0], t.shape_[1]);
  std::swap(t.strides_[0], t.strides_[1]);
  return t;
}

static int norm_dim(const char* op, int dim, int nd) {
  const int d = dim < 0 ? dim + nd : dim;
  if (d < 0 || d >= nd) throw Error(op, "dimension " + std::to_string(dim) + " out of range for rank " + std::to_string(nd));
  return d;
}

Tensor Tensor::Transpose(int d0, int d1) const {
  const int a = norm_dim("Transpose", d0, Dims()), b = norm_dim("Transpose", d1, Dims());
  Tensor t = *this;
  std::swap(t.shape_[a], t.shape_[b]);
  std::swap(t.strides_[a], t.strides_[b]);
  return t;
}

Tensor Tensor::Select(int dim, int64_t index) const {
  const int d = norm_dim("Select", dim, Dims());
  if (index < 0 || index >= shape_[d])
    fail("Select", "index " + std::to_string(index) + " out of range for dimension of size " + std::to_string(shape_[d]));
  Tensor t = *this;
  t.offset_ += index * strides_[d];
  t.shape_.erase(t.shape_.begin() + d);
  t.strides_.erase(t.strides_.begin() + d);
  return t;
}

Tensor Tensor::Narrow(int dim, int64_t start, int64_t length) const {
  const int d = norm_dim("Narrow", dim, Dims());
  if (start < 0 || length < 0 || start + length > shape_[d])
    fail("Narrow", "range [" + std::to_string(start) + ", " + std::to_string(start + length) + ") outside dimension of size " +
                       std::to_string(shape_[d]));
  Tensor t = *this;
  if (length > 0) t.offset_ += start * strides_[d];
  t.shape_[d] = length;
  return t;
}

Tensor Tensor::Unsqueeze(int dim) const {
  const int nd = Dims();
  const int d = dim < 0 ? dim + nd + 1 : dim;
  if (d < 0 || d > nd) fail("Unsqueeze", "dimension " + std::to_string(dim) + " out of range for rank " + std::to_string(nd));
  Tensor t = *this;
  const int64_t st = d < nd ? strides_[d] * shape_[d] : 1;
  t.shape_.insert(t.shape_.begin() + d, 1);
  t.strides_.insert(t.strides_.begin() + d, st);
  return t;
}

Tensor Tensor::Squeeze(int dim) const {
  const int d = norm_dim("Squeeze", dim, Dims());
  if (shape_[d] != 1) fail("Squeeze", "dimension " + std::to_string(dim) + " has size " + std::to_string(shape_[d]));
  Tensor t = *this;
  t.shape_.erase(t.shape_.begin() + d);
  t.strides_.erase(t.strides_.begin() + d);
  return t;
}

float Tensor::Item() const {
  if (Size() != 1) fail("Item", "tensor of shape " + shape_str(shape_) + " has " + std::to_string(Size()) + " elements");
  return Float32s()[0];
}

std::vector<float> Tensor::RowSumSquares() const {
  if (shape_.size() != 2) fail("RowSumSquares", "expected a 2-D tensor, got " + shape_str(shape_));
  Tensor x = Contiguous();
  std::vector<float> out(shape_[0]);
  if (shape_[0] == 0) return out;
  call("RowSumSquares", fa_row_sum_squares(device(), x.base(), shape_[0], shape_[1], out.data()));
  return out;
}

namespace {

fa_matrix view2d(const Tensor& t) {
  fa_matrix v{};
  const int nd = t.Dims();
  v.data = t.base();
  v.rs = t.strides()[nd - 2];
  v.cs = t.strides()[nd - 1];
  return v;
}

// broadcastShapes (tensor/shape.go:94-118)
Shape broadcast_shapes(const char* op, const Shape& a, const Shape& b) {
  const size_t n = std::max(a.size(), b.size());
  Shape out(n);
  for (size_t i = 1; i <= n; i++) {
    const int64_t da = i <= a.size() ? a[a.size() - i] : 1, db = i <= b.size() ? b[b.size() - i] : 1;
    if (da == db || db == 1) out[n - i] = da;
    else if (da == 1) out[n - i] = db;
    else fail(op, "shapes " + shape_str(a) + " and " + shape_str(b) + " are not broadcastable");
  }
  return out;
}

Tensor matmul2d(const Tensor& x, const Tensor& y) {
  const int64_t m = x.Dim(0), k = x.Dim(1), n = y.Dim(1);
  if (k != y.Dim(0)) fail("MatMul", "shape mismatch " + shape_str(x.shape()) + " · " + shape_str(y.shape()));
  Tensor out = Tensor::Zeros({m, n});
  if (m == 0 || n == 0) return out;
  const fa_matrix a = view2d(x), b = view2d(y);
  call("MatMul", fa_matmul_strided(device(), 0, nullptr, m, n, k, &a, &b, nullptr, const_cast<float*>(out.base())));
  return out;
}

// matmulBatched (tensor/matmul.go:74-127)
Tensor matmul_batched(const Tensor& x, const Tensor& y) {
  const int nx = x.Dims(), ny = y.Dims();
  const int64_t m = x.Dim(nx - 2), k = x.Dim(nx - 1), n = y.Dim(ny - 1);
  if (k != y.Dim(ny - 2)) fail("MatMul", "shape mismatch " + shape_str(x.shape()) + " · " + shape_str(y.shape()));
  const Shape xb(x.shape().begin(), x.shape().end() - 2), yb(y.shape().begin(), y.shape().end() - 2);
  if (ny == 2 && x.IsContiguous()) {  // [B..., m, k] . [k, n]: the batch folds into M
    Shape shape = xb;
    shape.push_back(m);
    shape.push_back(n);
    int64_t rows = m;
    for (int64_t v : xb) rows *= v;
    return MatMul(x.Reshape({rows, k}), y).Reshape(shape);
  }
  const Shape batch = broadcast_shapes("MatMul", xb, yb);
  if (batch.size() > FA_MAX_BATCH_DIMS)
    fail("MatMul", std::to_string(batch.size()) + " batch dimensions, at most " + std::to_string(FA_MAX_BATCH_DIMS));
  Shape shape = batch;
  shape.push_back(m);
  shape.push_back(n);
  Tensor out = Tensor::Zeros(shape);
  if (out.Size() == 0) return out;
  fa_matrix a = view2d(x), b = view2d(y);
  // broadcastStrides (tensor/shape.go:122-131): stride 0 where a dimension is broadcast
  const size_t nb = batch.size();
  for (size_t d = 0; d < nb; d++) {
    const size_t offx = nb - xb.size(), offy = nb - yb.size();
    a.bstride[d] = d >= offx && xb[d - offx] != 1 ? x.strides()[d - offx] : 0;
    b.bstride[d] = d >= offy && yb[d - offy] != 1 ? y.strides()[d - offy] : 0;
  }
  call("MatMul", fa_matmul_strided(device(), (int32_t)nb, batch.data(), m, n, k, &a, &b, nullptr,
                                   const_cast<float*>(out.base())));
  return out;
}

}  // namespace

Tensor MatMulFused(const Tensor& x, const Tensor& w, const Fused& f) {
  if (x.Dims() != 2 || w.Dims() != 2)
    fail("MatMulFused", "expected 2-D operands, got " + shape_str(x.shape()) + " and " + shape_str(w.shape()));
  const int64_t m = x.Dim(0), k = x.Dim(1), n = w.Dim(1);
  if (k != w.Dim(0)) fail("MatMulFused", "shape mismatch " + shape_str(x.shape()) + " · " + shape_str(w.shape()));
  if (f.Bias && f.Bias->Size() != n)
    fail("MatMulFused", "bias has " + std::to_string(f.Bias->Size()) + " elements for " + std::to_string(n) + " columns");
  if (!f.RowScale.empty() && (int64_t)f.RowScale.size() != m)
    fail("MatMulFused", "row scale has " + std::to_string(f.RowScale.size()) + " elements for " + std::to_string(m) + " rows");
  for (const Tensor* t : {f.Mul, f.Residual})
    if (t && !(t->Dims() == 2 && t->Dim(0) == m && t->Dim(1) == n))
      fail("MatMulFused", "Mul/Residual must be [" + std::to_string(m) + "×" + std::to_string(n) + "], got " +
                              shape_str(t->shape()));
  Tensor out = Tensor::Zeros({m, n});
  if (m == 0 || n == 0) return out;
  // x and w are read through their strides (transposed views included, as
  // the reference's GemmZeroEpilogue reads blas.Mat views); the element-wise
  // operands are made contiguous as the reference does (matmul_fused.go:79-84)
  fa_epilogue e{};
  Tensor bias, mul, res;
  if (f.Bias) { bias = f.Bias->Contiguous(); e.bias = bias.base(); }
  if (!f.RowScale.empty()) e.row_scale = f.RowScale.data();
  e.act = f.Act;
  if (f.Mul) { mul = f.Mul->Contiguous(); e.mul = mul.base(); e.ldm = n; }
  if (f.Residual) { res = f.Residual->Contiguous(); e.residual = res.base(); e.ldr = n; }
  const fa_matrix a = view2d(x), b = view2d(w);
  call("MatMulFused", fa_matmul_strided(device(), 0, nullptr, m, n, k, &a, &b, &e, const_cast<float*>(out.base())));
  return out;
}

Tensor MatMul(const Tensor& x, const Tensor& w) {
  const int nx = x.Dims(), nw = w.Dims();
  if (nx == 0 || nw == 0)
    fail("MatMul", "operands must be at least 1-D, got " + shape_str(x.shape()) + " and " + shape_str(w.shape()));
  if (nx == 1 && nw == 1) {
    if (x.Dim(0) != w.Dim(0)) fail("MatMul", "shape mismatch " + shape_str(x.shape()) + " · " + shape_str(w.shape()));
    return MatMul(x.Unsqueeze(0), w.Unsqueeze(1)).Reshape({});
  }
  if (nx == 1) return MatMul(x.Unsqueeze(0), w).Squeeze(-2);
  if (nw == 1) return MatMul(x, w.Unsqueeze(1)).Squeeze(-1);
  if (nx == 2 && nw == 2) return matmul2d(x, w);
  return matmul_batched(x, w);
}

Tensor Dot(const Tensor& x, const Tensor& y) {
  if (x.Dims() != 1 || y.Dims() != 1)
    fail("Dot", "expected 1-D tensors, got " + shape_str(x.shape()) + " and " + shape_str(y.shape()));
  return MatMul(x, y);
}

Tensor Outer(const Tensor& x, const Tensor& y) {
  if (x.Dims() != 1 || y.Dims() != 1)
    fail("Outer", "expected 1-D tensors, got " + shape_str(x.shape()) + " and " + shape_str(y.shape()));
  return MatMul(x.Unsqueeze(1), y.Unsqueeze(0));
}

Tensor RMSNorm(const Tensor& x, const Tensor& g, float eps) {
  if (x.Dims() == 0) fail("RMSNorm", "expected at least a 1-D input");
  const int64_t n = x.Dim(-1);
  if (g.Size() != n)
    fail("RMSNorm", "g must have " + std::to_string(n) + " elements, got " + std::to_string(g.Size()));
  const Tensor xc = x.Contiguous(), gc = g.Contiguous();
  Tensor out = Tensor::Zeros(x.shape());
  const int64_t rows = n ? x.Size() / n : 0;
  if (rows == 0) return out;
  call("RMSNorm", fa_rmsnorm(device(), xc.base(), gc.base(), eps, rows, n, const_cast<float*>(out.base())));
  return out;
}

Tensor RoPE(const Tensor& x, double base, const std::vector<int>& positions) {
  const int nd = x.Dims();
  if (nd < 2) fail("RoPE", "expected at least a 2-D input, got " + shape_str(x.shape()));
  const int64_t T = x.Dim(-2), D = x.Dim(-1);
  if (D % 2 != 0) fail("RoPE", "head dimension " + std::to_string(D) + " must be even");
  if ((int64_t)positions.size() != T)
    fail("RoPE", "got " + std::to_string(positions.size()) + " positions for " + std::to_string(T) + " slots");
  const Tensor xc = x.Contiguous();
  Tensor out = Tensor::Zeros(x.shape());
  const int64_t rows = D ? x.Size() / D : 0;
  if (rows == 0) return out;
  std::vector<int32_t> pos(positions.begin(), positions.end());
  call("RoPE", fa_rope(device(), xc.base(), base, pos.data(), rows, (int32_t)T, (int32_t)D,
                       const_cast<float*>(out.base())));
  return out;
}

Tensor AttentionScaled(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor* mask, float scale) {
  const int nd = q.Dims();
  if (nd < 2 || k.Dims() != nd || v.Dims() != nd)
    fail("Attention", "q, k, v must have the same rank ≥ 2, got " + shape_str(q.shape()) + " " + shape_str(k.shape()) +
                          " " + shape_str(v.shape()));
  const int64_t D = q.Dim(-1);
  if (k.Dim(-1) != D || v.Dim(-2) != k.Dim(-2))
    fail("Attention", "shapes do not match: q " + shape_str(q.shape()) + ", k " + shape_str(k.shape()) + ", v " +
                          shape_str(v.shape()));
  if (nd > 4) fail("Attention", "this mirror covers up to two leading dimensions, got " + shape_str(q.shape()));
  for (int i = 0; i < nd - 2; i++)
    if (k.Dim(i) != q.Dim(i) || v.Dim(i) != q.Dim(i))
      fail("Attention", "leading dimensions of q, k, v differ");
  const int64_t T = q.Dim(-2), S = k.Dim(-2);
  // lead dims as (B, H) with element strides; rows of D must be contiguous
  auto rows_ok = [&](const Tensor& t, int64_t R) {
    return t.strides()[nd - 1] == 1 && (R <= 1 || t.strides()[nd - 2] == D);
  };
  const Tensor qc = rows_ok(q, T) ? q : q.Contiguous();
  const Tensor kc = rows_ok(k, S) ? k : k.Contiguous();
  const Tensor vc = rows_ok(v, S) ? v : v.Contiguous();
  auto lead = [&](const Tensor& t, int64_t& sb, int64_t& sh) {
    sb = sh = 0;
    if (nd == 4) { sb = t.strides()[0]; sh = t.strides()[1]; }
    else if (nd == 3) { sh = t.strides()[0]; }
  };
  const int64_t B = nd == 4 ? q.Dim(0) : 1, H = nd >= 3 ? q.Dim(nd - 3) : 1;
  int64_t qsb, qsh, ksb, ksh, vsb, vsh;
  lead(qc, qsb, qsh);
  lead(kc, ksb, ksh);
  lead(vc, vsb, vsh);
  // mask: broadcast strides over [B, H, T, S]
  Tensor mc;
  int64_t ms[4] = {0, 0, 0, 0};
  const float* mp = nullptr;
  if (mask) {
    if (mask->Dims() > 4) fail("Attention", "mask rank " + std::to_string(mask->Dims()) + " > 4");
    mc = mask->Contiguous();
    const Shape full = {B, H, T, S};
    const int off = 4 - mc.Dims();
    for (int i = 0; i < 4; i++) {
      if (i < off) continue;
      const int64_t have = mc.shape()[i - off];
      if (have == full[i]) ms[i] = mc.strides()[i - off];
      else if (have == 1) ms[i] = 0;
      else fail("Attention", "mask " + shape_str(mask->shape()) + " does not broadcast to " + shape_str(full));
    }
    mp = mc.base();
  }
  Tensor out = Tensor::Zeros(q.shape());
  if (B * H * T == 0 || D == 0) return out;
  call("Attention", fa_attention(device(), qc.base(), kc.base(), vc.base(), (int32_t)B, (int32_t)H, (int32_t)T,
                                 (int32_t)S, (int32_t)D, qsb, qsh, ksb, ksh, vsb, vsh, mp, ms[0], ms[1], ms[2], ms[3],
                                 scale, const_cast<float*>(out.base())));
  return out;
}

Tensor Attention(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor* mask) {
  const double d = (double)q.Dim(-1);
  return AttentionScaled(q, k, v, mask, (float)(1.0 / std::sqrt(d)));
}

Tensor PaddingMask(const std::vector<int>& lengths, int64_t n) {
  const int64_t b = (int64_t)lengths.size();
  std::vector<float> m(b * n, 0.f);
  for (int64_t i = 0; i < b; i++)
    for (int64_t j = std::max<int64_t>(0, lengths[i]); j < n; j++) m[i * n + j] = kMaskNeg;
  return Tensor::New(std::move(m), {b, 1, 1, n});
}

Tensor WindowMask(int64_t n, int64_t w) {
  std::vector<float> m(n * n, 0.f);
  for (int64_t i = 0; i < n; i++)
    for (int64_t j = 0; j < n; j++)
      if (j - i >= w || i - j >= w) m[i * n + j] = kMaskNeg;
  return Tensor::New(std::move(m), {n, n});
}

Tensor CausalMask(int64_t n) {
  std::vector<float> m(n * n, 0.f);
  for (int64_t i = 0; i < n; i++)
    for (int64_t j = i + 1; j < n; j++) m[i * n + j] = kMaskNeg;
  return Tensor::New(std::move(m), {n, n});
}

}  // namespace tensor

namespace gemma {

namespace {
void gcheck(fa_ctx* ctx, int rc) {
  if (rc != FA_OK) throw Error(fa_last_error(ctx));
}
}  // namespace

Model::Model(const Config& cfg) : cfg_(cfg) {
  fa_gemma_config c{};
  c.hidden_size = cfg.HiddenSize;
  c.num_hidden_layers = cfg.NumHiddenLayers;
  c.num_attention_heads = cfg.NumAttentionHeads;
  c.num_key_value_heads = cfg.NumKeyValueHeads;
  c.head_dim = cfg.HeadDim;
  c.intermediate_size = cfg.IntermediateSize;
  c.vocab_size = cfg.VocabSize;
  c.sliding_window = cfg.SlidingWindow;
  c.use_bidirectional = cfg.UseBidirectional ? 1 : 0;
  c.sliding_window_pattern = cfg.SlidingWindowPattern;
  c.rope_local_base_freq = cfg.RopeLocalBaseFreq;
  c.rope_theta = cfg.RopeTheta;
  c.query_pre_attn_scalar = cfg.QueryPreAttnScalar;
  c.rms_norm_eps = cfg.RMSNormEps;
  c.max_tokens = cfg.MaxTokens;
  if (cfg.Dense.size() > 4) throw Error("gemma: at most 4 Dense layers");
  c.n_dense = (int32_t)cfg.Dense.size();
  for (size_t i = 0; i < cfg.Dense.size(); i++) {
    c.dense_out[i] = cfg.Dense[i];
    c.dense_act[i] = i < cfg.DenseAct.size() ? cfg.DenseAct[i] : FA_ACT_NONE;
  }
  if (cfg.Variant == 2) {
    if (cfg.NumHiddenLayers > FA_GEMMA_MAX_LAYERS)
      throw Error("gemma: " + std::to_string(cfg.NumHiddenLayers) + " layers; this build runs at most " +
                  std::to_string(FA_GEMMA_MAX_LAYERS));
    c.variant = 2;
    c.hidden_size_per_layer_input = cfg.HiddenSizePerLayerInput;
    c.embedding_dim = cfg.EmbeddingDim;
    c.rope_local_base_freq = cfg.RopeBase(-1);
    c.rope_theta = cfg.RopeBase(-2);
    for (int l = 0; l < cfg.NumHiddenLayers; l++) {
      c.layer_head_dim[l] = cfg.LayerHeadDim(l);
      c.layer_kv_heads[l] = cfg.LayerKVHeads(l);
      c.layer_sliding[l] = cfg.IsSliding(l) ? 1 : 0;
    }
  }
  gcheck(device(), fa_gemma_create(device(), &c, &m_));
}

Model::~Model() { Close(); }

void Model::Close() {
  if (m_) fa_gemma_destroy(m_);
  m_ = nullptr;
}

void Model::SetWeightBF16(const std::string& name, const std::vector<int64_t>& shape, const uint16_t* data) {
  gcheck(device(), fa_gemma_set_weight(m_, name.c_str(), FA_DT_BF16, shape.data(), (int32_t)shape.size(), data));
}

void Model::SetWeightF32(const std::string& name, const std::vector<int64_t>& shape, const float* data) {
  gcheck(device(), fa_gemma_set_weight(m_, name.c_str(), FA_DT_F32, shape.data(), (int32_t)shape.size(), data));
}

void Model::Finalize() { gcheck(device(), fa_gemma_finalize(m_)); }

// model.go:336-344: the embedding projection's width when there is one, else
// the last Dense layer's, else the hidden size.
int Model::Dim() const {
  if (cfg_.Variant == 2) return cfg_.EmbeddingDim;
  return cfg_.Dense.empty() ? cfg_.HiddenSize : cfg_.Dense.back();
}

std::vector<std::vector<float>> Model::EmbedIDs(const std::vector<std::vector<int32_t>>& ids, EmbedOpts o) const {
  if (!m_) throw Error("gemma: model is closed");
  int dim = Dim();
  if (o.Dim != 0) {
    if (o.Dim < 1 || o.Dim > dim) throw Error("gemma: Dim(" + std::to_string(o.Dim) + ") outside 1.." + std::to_string(dim));
    dim = o.Dim;
  }
  const int32_t B = (int32_t)ids.size();
  if (B == 0) return {};
  int32_t T = 0;
  std::vector<int32_t> lengths(B);
  for (int32_t b = 0; b < B; b++) {
    lengths[b] = (int32_t)std::min<size_t>(ids[b].size(), (size_t)cfg_.MaxTokens);  // embed.go:40-42
    T = std::max(T, lengths[b]);
  }
  std::vector<int32_t> flat((size_t)B * T, 0);  // pad id 0 (embed.go:128-138)
  for (int32_t b = 0; b < B; b++) std::copy(ids[b].begin(), ids[b].begin() + lengths[b], flat.begin() + (size_t)b * T);
  std::vector<float> out((size_t)B * dim);
  gcheck(device(), fa_gemma_embed_ids(m_, flat.data(), lengths.data(), B, T, dim, out.data()));
  std::vector<std::vector<float>> res(B);
  for (int32_t b = 0; b < B; b++) res[b].assign(out.begin() + (size_t)b * dim, out.begin() + (size_t)(b + 1) * dim);
  return res;
}

namespace {

bool exists(const std::string& path) {
  struct stat st;
  return stat(path.c_str(), &st) == 0;
}

json::Value read_json(const std::string& path, const char* what) {
  try {
    return json::parse_file(path);
  } catch (const json::Error& e) {
    throw Error(std::string("gemma: ") + what + ": " + e.what());
  }
}

std::string layer_key(int l) {
  char b[16];
  std::snprintf(b, sizeof b, "%02d", l);
  return b;
}

const LayerOverride* override_of(const Config& c, int l) {
  auto it = c.PerLayerConfig.find(layer_key(l));
  if (it == c.PerLayerConfig.end()) it = c.PerLayerConfig.find(std::to_string(l));
  return it == c.PerLayerConfig.end() ? nullptr : &it->second;
}

}  // namespace

int Config::LayerHeadDim(int l) const {
  const LayerOverride* o = override_of(*this, l);
  return o && o->HeadDim != 0 ? o->HeadDim : HeadDim;
}

int Config::LayerKVHeads(int l) const {
  const LayerOverride* o = override_of(*this, l);
  return o && o->NumKeyValueHeads != 0 ? o->NumKeyValueHeads : NumKeyValueHeads;
}

bool Config::IsSliding(int l) const {
  if (!LayerTypes.empty()) return LayerTypes[l] == "sliding_attention";
  return (l + 1) % (SlidingWindowPattern > 0 ? SlidingWindowPattern : 6) != 0;
}

// l >= 0: that layer's base; -1 / -2: the sliding / full layers' base.
double Config::RopeBase(int l) const {
  const bool sliding = l == -1 || (l >= 0 && IsSliding(l));
  if (Variant == 2) {
    auto it = RopeThetaByType.find(sliding ? "sliding_attention" : "full_attention");
    if (it != RopeThetaByType.end() && it->second != 0) return it->second;
  }
  if (sliding) return RopeLocalBaseFreq != 0 ? RopeLocalBaseFreq : 10000;
  return RopeTheta != 0 ? RopeTheta : 10000;
}

int Config::Window() const {
  if (Variant == 2) return SlidingWindow + 1;
  return UseBidirectional ? SlidingWindow / 2 + 1 : SlidingWindow;
}

namespace {

// The text-model fields shared by both variants (config.go:19-38).
void read_text_fields(const json::Value& v, Config& c) {
  c.HiddenSize = (int)v.get_int("hidden_size");
  c.IntermediateSize = (int)v.get_int("intermediate_size");
  c.NumHiddenLayers = (int)v.get_int("num_hidden_layers");
  c.NumAttentionHeads = (int)v.get_int("num_attention_heads");
  c.NumKeyValueHeads = (int)v.get_int("num_key_value_heads");
  c.HeadDim = (int)v.get_int("head_dim");
  c.VocabSize = (int)v.get_int("vocab_size");
  c.SlidingWindow = (int)v.get_int("sliding_window");
  c.UseBidirectional = v.get_bool("use_bidirectional_attention");
  c.RopeTheta = v.get_number("rope_theta");
  c.RopeLocalBaseFreq = v.get_number("rope_local_base_freq");
  c.QueryPreAttnScalar = v.get_number("query_pre_attn_scalar");
  c.RMSNormEps = (float)v.get_number("rms_norm_eps");
  if (const json::Value* lt = v.find("layer_types"); lt && lt->is_array())
    for (const auto& t : lt->items()) c.LayerTypes.push_back(t.as_string());
  const std::string act = v.get_string("hidden_activation");
  if (!act.empty() && act != "gelu_pytorch_tanh")
    throw Error("gemma: activation \"" + act + "\" not supported (want gelu_pytorch_tanh)");
  if (const json::Value* rs = v.find("rope_scaling"); rs && !rs->is_null())
    throw Error("gemma: rope_scaling is set; not supported");
}

// fillVariant2 (config.go:247-297): EmbeddingGemma 2's defaults and checks.
void fill_variant2(const json::Value& t, Config& c) {
  c.HiddenSizePerLayerInput = (int)t.get_int("hidden_size_per_layer_input");
  c.EmbeddingDim = (int)t.get_int("embedding_dim");
  if (c.LayerTypes.empty())
    for (int i = 0; i < c.NumHiddenLayers; i++)
      c.LayerTypes.push_back((i + 1) % 6 == 0 ? "full_attention" : "sliding_attention");
  if (const json::Value* pc = t.find("per_layer_config"); pc && pc->is_object()) {
    for (const auto& kv : pc->members())
      c.PerLayerConfig[kv.first] = LayerOverride{(int)kv.second.get_int("head_dim"),
                                                 (int)kv.second.get_int("num_key_value_heads")};
  } else {
    for (int i = 0; i < (int)c.LayerTypes.size(); i++)
      if (c.LayerTypes[i] == "full_attention") c.PerLayerConfig[layer_key(i)] = LayerOverride{512, 1};
  }
  if (const json::Value* rp = t.find("rope_parameters"); rp && rp->is_object()) {
    for (const auto& kv : rp->members()) {
      const std::string type = kv.second.get_string("rope_type");
      if (!type.empty() && type != "default")
        throw Error("gemma: rope_type \"" + type + "\" for " + kv.first + " not supported");
      c.RopeThetaByType[kv.first] = kv.second.get_number("rope_theta");
    }
  } else {
    c.RopeThetaByType = {{"sliding_attention", 10000.0}, {"full_attention", 1000000.0}};
  }
  if (c.EmbeddingDim == 0) c.EmbeddingDim = 768;
  if (c.HiddenSizePerLayerInput == 0)
    throw Error("gemma: embedding_gemma2 config without hidden_size_per_layer_input");
}

}  // namespace

Config LoadConfig(const std::string& dir) {
  const json::Value v = read_json(dir + "/config.json", "config.json");
  Config c;
  int64_t maxpos = 0;
  try {
    if (v.get_string("model_type") == "embedding_gemma2") {
      // the text tower's fields sit under text_config; the placeholder ids
      // and the vision/audio configs beside it (config.go:157-208)
      const json::Value* t = v.find("text_config");
      if (!t || !t->is_object()) throw Error("gemma: config.json text_config: missing");
      c.Variant = 2;
      read_text_fields(*t, c);
      maxpos = t->get_int("max_position_embeddings");
      const struct {
        const char* key;
        const char* name;
      } marks[] = {{"image_token_id", "image"},       {"audio_token_id", "audio"},
                   {"video_token_id", "video"},       {"boi_token_id", "begin-of-image"},
                   {"eoi_token_id", "end-of-image"},  {"boa_token_id", "begin-of-audio"},
                   {"eoa_token_index", "end-of-audio"}};
      for (const auto& mk : marks)
        if (const json::Value* id = v.find(mk.key); id && !id->is_null())
          c.MultimodalTokens[(int)id->as_int()] = mk.name;
      auto has = [&](const char* k) {
        const json::Value* x = v.find(k);
        return x && !x->is_null();
      };
      if (has("image_token_id") && has("boi_token_id") && has("eoi_token_id") && has("vision_config")) {
        c.ImageToken = (int)v.find("image_token_id")->as_int();
        c.HasVision = true;
      }
      if (has("audio_token_id") && has("boa_token_id") && has("eoa_token_index") && has("audio_config")) {
        c.AudioToken = (int)v.find("audio_token_id")->as_int();
        c.HasAudio = true;
      }
      fill_variant2(*t, c);
    } else {
      read_text_fields(v, c);
      maxpos = v.get_int("max_position_embeddings");
      c.SlidingWindowPattern = (int)v.get_int("sliding_window_pattern", 6);  // config.go:211-213
      if (c.SlidingWindowPattern == 0) c.SlidingWindowPattern = 6;
      // layer_types must be the periodic pattern the GPU encoder runs:
      // full attention iff (l+1) % pattern == 0 (config.go:214-225)
      if (!c.LayerTypes.empty()) {
        const auto& t = c.LayerTypes;
        int first_full = -1;
        for (size_t i = 0; i < t.size(); i++)
          if (t[i] == "full_attention") {
            first_full = (int)i;
            break;
          }
        const int pat = first_full >= 0 ? first_full + 1 : (int)t.size() + 1;
        for (size_t i = 0; i < t.size(); i++) {
          const bool full = (int)((i + 1) % pat) == 0;
          if (t[i] != (full ? "full_attention" : "sliding_attention"))
            throw Error("gemma: layer_types is not a periodic sliding/full pattern");
        }
        c.SlidingWindowPattern = pat;
        c.LayerTypes.clear();
      }
    }
  } catch (const json::Error& e) {
    throw Error(std::string("gemma: config.json: ") + e.what());
  }
  if (c.HiddenSize == 0 || c.NumHiddenLayers == 0) throw Error("gemma: config is missing hidden_size or num_hidden_layers");
  if (c.Variant == 2 && (int)c.LayerTypes.size() != c.NumHiddenLayers)
    throw Error("gemma: " + std::to_string(c.LayerTypes.size()) + " layer types for " +
                std::to_string(c.NumHiddenLayers) + " layers");
  if (c.NumKeyValueHeads <= 0 || c.NumAttentionHeads % c.NumKeyValueHeads != 0)
    throw Error("gemma: " + std::to_string(c.NumAttentionHeads) + " query heads not a multiple of " +
                std::to_string(c.NumKeyValueHeads) + " key/value heads");
  if (c.HeadDim % 2 != 0) throw Error("gemma: head_dim " + std::to_string(c.HeadDim) + " must be even for RoPE");
  if (c.Variant == 2) {
    for (int l = 0; l < c.NumHiddenLayers; l++) {
      if (c.LayerHeadDim(l) % 2 != 0)
        throw Error("gemma: layer " + std::to_string(l) + " head_dim " + std::to_string(c.LayerHeadDim(l)) +
                    " must be even for RoPE");
      if (c.LayerKVHeads(l) <= 0 || c.NumAttentionHeads % c.LayerKVHeads(l) != 0)
        throw Error("gemma: layer " + std::to_string(l) + ": " + std::to_string(c.NumAttentionHeads) +
                    " query heads not a multiple of " + std::to_string(c.LayerKVHeads(l)) + " key/value heads");
    }
    // model.go:102-110: the model card's 8192 tokens
    c.MaxTokens = maxpos == 0 ? 8192 : (int)std::min<int64_t>(maxpos, 8192);
  } else {
    c.MaxTokens = (maxpos == 0 || maxpos > 2048) ? 2048 : (int)maxpos;  // model.go:100-104
  }
  c.Dense.clear();
  c.DenseAct.clear();
  return c;
}

std::unique_ptr<Model> Model::Load(const std::string& dir, const LoadOpts& o) {
  std::string stage = "config.json";  // names the file in JSON type errors
  try {
    Config cfg = LoadConfig(dir);
    if (o.MaxTokens > 0) cfg.MaxTokens = std::min(o.MaxTokens, cfg.Variant == 2 ? 8192 : 2048);
    if (o.BatchTokens <= 0) throw Error("gemma: BatchTokens must be positive");
    // sentence-transformers head (model.go:236-310): mean pooling, Dense
    // layers (linear.weight; identity or Tanh), Normalize
    struct DenseMod {
      std::string path;
      int in, out, act;
    };
    std::vector<DenseMod> dense;
    stage = "modules.json";
    if (exists(dir + "/modules.json")) {
      const json::Value mods = read_json(dir + "/modules.json", "modules.json");
      for (const json::Value& mod : mods.items()) {
        const std::string type = mod.get_string("type"), path = mod.get_string("path");
        const std::string mdir = dir + "/" + path;
        stage = mdir + "/config.json";
        if (type == "sentence_transformers.models.Pooling" ||
            type == "sentence_transformers.sentence_transformer.modules.pooling.Pooling") {
          const json::Value pc = read_json(mdir + "/config.json", "pooling config");
          const std::string mode = pc.get_string("pooling_mode");
          if ((!mode.empty() && mode != "mean") || pc.get_bool("pooling_mode_cls_token") ||
              pc.get_bool("pooling_mode_lasttoken") ||
              (mode.empty() && !pc.get_bool("pooling_mode_mean_tokens", true)))
            throw Error("gemma: only mean pooling is supported");
        } else if (type == "sentence_transformers.models.Dense") {
          // the reference reads the "bias" flag and loads linear.weight only
          // (model.go:277-304): a bias tensor is present but not applied
          const json::Value dc = read_json(mdir + "/config.json", "Dense config");
          (void)dc.get_bool("bias");
          const std::string act = dc.get_string("activation_function");
          int a = FA_ACT_NONE;
          if (act == "torch.nn.modules.activation.Tanh") a = FA_ACT_TANH;
          else if (!(act.empty() || act == "torch.nn.modules.linear.Identity"))
            throw Error("gemma: Dense activation \"" + act + "\" not supported");
          dense.push_back({mdir, (int)dc.get_int("in_features"), (int)dc.get_int("out_features"), a});
        }
      }
    }
    if (dense.size() > 4) throw Error("gemma: at most 4 Dense layers");
    int width = cfg.Variant == 2 ? cfg.EmbeddingDim : cfg.HiddenSize;  // after the embedding projection
    for (const auto& d : dense) {
      if (d.in != width)
        throw Error("gemma: Dense in_features " + std::to_string(d.in) + " after width " + std::to_string(width));
      cfg.Dense.push_back(d.out);
      cfg.DenseAct.push_back(d.act);
      width = d.out;
    }
    // every file is read and checked before the GPU is touched
    stage = "tokenizer.json";
    std::unique_ptr<tokenizer::Tokenizer> tok;
    try {
      tok = std::make_unique<tokenizer::Tokenizer>(tokenizer::Tokenizer::Load(dir + "/tokenizer.json"));
    } catch (const tokenizer::Error& e) {
      throw Error(e.what());
    }
    stage = "config_sentence_transformers.json";
    std::map<std::string, std::string> prompts;
    if (exists(dir + "/config_sentence_transformers.json")) {
      const json::Value sc = read_json(dir + "/config_sentence_transformers.json", "config_sentence_transformers.json");
      if (const json::Value* pr = sc.find("prompts"); pr && pr->is_object())
        for (const auto& kv : pr->members()) prompts[kv.first] = kv.second.as_string();
    }
    stage = "safetensors";
    auto open_dir = [](const std::string& d) {
      try {
        return safetensors::File::OpenDir(d);
      } catch (const safetensors::Error& e) {
        throw Error(e.what());
      }
    };
    safetensors::File f = open_dir(dir);
    std::vector<safetensors::File> dense_files;
    for (const auto& d : dense) {
      dense_files.push_back(open_dir(d.path));
      if (!dense_files.back().Find("linear.weight")) throw Error("gemma: " + d.path + ": no linear.weight");
    }
    // weights (model.go:104-191): names with or without a model./language_model. prefix
    std::vector<std::pair<std::string, std::string>> names;  // (stored, ours)
    auto want = [&](const std::string& name) {
      for (const char* prefix : {"", "model.", "language_model."})
        if (f.Find(prefix + name)) {
          names.emplace_back(prefix + name, name);
          return;
        }
      throw Error("gemma: weight \"" + name + "\" not found");
    };
    want("embed_tokens.weight");
    for (int l = 0; l < cfg.NumHiddenLayers; l++) {
      const std::string p = "layers." + std::to_string(l) + ".";
      for (const char* n : {"input_layernorm.weight", "post_attention_layernorm.weight",
                            "pre_feedforward_layernorm.weight", "post_feedforward_layernorm.weight",
                            "self_attn.q_norm.weight", "self_attn.k_norm.weight", "self_attn.q_proj.weight",
                            "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
                            "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight"})
        want(p + n);
      if (cfg.Variant == 2)
        for (const char* n : {"ple_block.per_layer_input_gate.weight", "ple_block.per_layer_projection.weight",
                              "ple_block.post_per_layer_input_norm.weight", "layer_scalar"})
          want(p + n);
    }
    want("norm.weight");
    if (cfg.Variant == 2)
      for (const char* n : {"ple.per_layer_model_projection.weight", "ple.per_layer_projection_norm.weight",
                            "embedding_projection.weight"})
        want(n);

    stage = "weights";
    auto m = std::make_unique<Model>(cfg);
    m->batch_tokens_ = o.BatchTokens;
    m->tok_ = std::move(tok);
    m->prompts_ = std::move(prompts);
    auto put = [&](const safetensors::File& file, const std::string& stored, const std::string& name) {
      const safetensors::Info* info = file.Find(stored);
      if (info->dtype == "BF16") {
        size_t nb;
        const uint8_t* raw = file.Raw(stored, &nb);
        std::vector<uint16_t> bits(nb / 2);
        std::memcpy(bits.data(), raw, nb);  // the data section need not be 2-byte aligned
        m->SetWeightBF16(name, info->shape, bits.data());
      } else {
        std::vector<float> v;
        try {
          v = file.Float32s(stored);
        } catch (const safetensors::Error& e) {
          throw Error(e.what());
        }
        m->SetWeightF32(name, info->shape, v.data());
      }
    };
    for (const auto& n : names) put(f, n.first, n.second);
    for (size_t i = 0; i < dense.size(); i++)
      put(dense_files[i], "linear.weight", "dense." + std::to_string(i) + ".linear.weight");
    m->Finalize();
    return m;
  } catch (const json::Error& e) {
    throw Error("gemma: " + stage + ": " + e.what());
  }
}

std::vector<std::vector<float>> Model::Embed(const std::vector<std::string>& texts, const EmbedOpts& o) const {
  if (!tok_) throw Error("gemma: Embed needs a model from Load (it has no tokenizer)");
  std::string prefix;  // embed.go:99-114
  if (o.has_prompt_text) {
    prefix = o.PromptText;
  } else if (!o.Prompt.empty()) {
    auto it = prompts_.find(o.Prompt);
    if (it == prompts_.end()) throw Error("gemma: no prompt named \"" + o.Prompt + "\"");
    prefix = it->second;
  }
  const int dim = Dim();
  if (o.Dim != 0 && (o.Dim < 1 || o.Dim > dim))
    throw Error("gemma: Dim(" + std::to_string(o.Dim) + ") outside 1.." + std::to_string(dim));
  const size_t n = texts.size();
  std::vector<std::vector<int32_t>> ids(n);
  for (size_t i = 0; i < n; i++) {
    const std::vector<int> seq = tok_->Encode(prefix + texts[i]);
    // checkTextOnly (embed.go:82-97): EmbeddingGemma 2's image, audio and
    // video placeholders are refused, not embedded as ordinary tokens
    for (int id : seq) {
      auto mt = cfg_.MultimodalTokens.find(id);
      if (mt == cfg_.MultimodalTokens.end()) continue;
      const std::string& name = mt->second;
      if ((id == cfg_.ImageToken && cfg_.HasVision) || (id == cfg_.AudioToken && cfg_.HasAudio))
        throw Error("text " + std::to_string(i) + ": gemma: input contains the " + name +
                    " placeholder token; pass the " + name + " with EmbedInputs");
      throw Error("text " + std::to_string(i) + ": gemma: input contains the " + name +
                  " placeholder token; EmbeddingGemma 2 video input is not supported");
    }
    const size_t L = std::min(seq.size(), (size_t)cfg_.MaxTokens);
    ids[i].assign(seq.begin(), seq.begin() + L);
  }
  // shortest first, stable (model.go:412-423); greedy batches whose longest
  // sequence times their size stays within the token budget (embed.go:45-74)
  std::vector<size_t> order(n);
  std::iota(order.begin(), order.end(), 0);
  std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) { return ids[a].size() < ids[b].size(); });
  std::vector<std::vector<float>> out(n);
  std::vector<size_t> batch;
  size_t max_len = 0;
  EmbedOpts eo;
  eo.Dim = o.Dim;
  auto flush = [&]() {
    if (batch.empty()) return;
    std::vector<std::vector<int32_t>> b;
    for (size_t i : batch) b.push_back(ids[i]);
    auto e = EmbedIDs(b, eo);
    for (size_t k = 0; k < batch.size(); k++) out[batch[k]] = std::move(e[k]);
    batch.clear();
    max_len = 0;
  };
  for (size_t i : order) {
    const size_t l = ids[i].size();
    const size_t nm = std::max(max_len, l);
    if (!batch.empty() && nm * (batch.size() + 1) > (size_t)batch_tokens_) flush();
    batch.push_back(i);
    max_len = std::max(max_len, l);
  }
  flush();
  return out;
}

}  // namespace gemma
}  // namespace fiber
