// Tensor operators of the C++ host mirror (ai_amd/host/fiber.hpp) on the
// GPU, restating the reference's own tests (file:line of each below) against
// float64 closed forms. Run by tests/test_cpp_host.py on an MI355X.
#include <algorithm>
#include <cmath>
#include <random>

#include "fiber.hpp"
#include "testing.hpp"

using namespace fiber::tensor;

static Tensor randn(std::mt19937_64& rng, Shape shape, double scale = 1.0) {
  std::normal_distribution<double> nd(0.0, 1.0);
  int64_t n = 1;
  for (auto d : shape) n *= d;
  std::vector<float> v(n);
  for (auto& x : v) x = (float)(nd(rng) * scale);
  return Tensor::New(std::move(v), shape);
}

static Tensor randu(std::mt19937_64& rng, Shape shape) {
  std::uniform_real_distribution<double> ud(-1.0, 1.0);
  int64_t n = 1;
  for (auto d : shape) n *= d;
  std::vector<float> v(n);
  for (auto& x : v) x = (float)ud(rng);
  return Tensor::New(std::move(v), shape);
}

// tensor/rope_test.go:9-25
TEST(TestRoPEKnown) {
  auto got = RoPE(Tensor::New({1, 0}, {1, 2}), 10000, {1}).Float32s();
  const float c = (float)std::cos(1.0), s = (float)std::sin(1.0);
  if (std::fabs(got[0] - c) > 1e-6 || std::fabs(got[1] - s) > 1e-6) FATAL("got [%g %g], want [%g %g]", got[0], got[1], c, s);
  auto id = RoPE(Tensor::New({3, -4, 5, 6}, {1, 4}), 10000, {0}).Float32s();
  const float want[] = {3, -4, 5, 6};
  for (int i = 0; i < 4; i++)
    if (std::fabs(id[i] - want[i]) > 1e-6) FATAL("position 0 not identity: %g", id[i]);
}

// tensor/rope_test.go:27-38
TEST(TestRoPEPreservesNorm) {
  std::mt19937_64 rng(1);
  Tensor x = randn(rng, {2, 3, 8, 16});
  Tensor y = RoPE(x, 1e6, {0, 5, 9, 100, 500, 1000, 3, 7});
  auto xv = x.Float32s(), yv = y.Float32s();
  for (int r = 0; r < 2 * 3 * 8; r++) {
    double xn = 0, yn = 0;
    for (int i = 0; i < 16; i++) {
      xn += (double)xv[r * 16 + i] * xv[r * 16 + i];
      yn += (double)yv[r * 16 + i] * yv[r * 16 + i];
    }
    if (std::fabs(xn - yn) > 1e-3 * (xn + 1)) FATAL("norm changed at %d: %g vs %g", r, xn, yn);
  }
}

// tensor/rope_test.go:66-81
TEST(TestWindowMask) {
  auto m = WindowMask(5, 2).Float32s();
  for (int i = 0; i < 5; i++)
    for (int j = 0; j < 5; j++) {
      const float want = (j - i >= 2 || i - j >= 2) ? kMaskNeg : 0.f;
      if (m[i * 5 + j] != want) FATAL("mask[%d,%d] = %g", i, j, m[i * 5 + j]);
    }
}

// tensor/rope_test.go:83-102
TEST(TestRMSNormFusedMatchesComposed) {
  std::mt19937_64 rng(7);
  for (Shape shp : {Shape{4, 5, 64}, Shape{2, 3, 8, 16}}) {
    Tensor x = randn(rng, shp);
    Tensor g = randn(rng, {shp.back()});
    auto got = RMSNorm(x, g, 1e-6f).Float32s();
    auto xv = x.Float32s(), gv = g.Float32s();
    const int64_t n = shp.back(), rows = x.Size() / n;
    for (int64_t r = 0; r < rows; r++) {
      double ms = 0;
      for (int64_t i = 0; i < n; i++) ms += (double)xv[r * n + i] * xv[r * n + i];
      const double rms = std::sqrt(ms / n + 1e-6);
      for (int64_t i = 0; i < n; i++) {
        const double want = xv[r * n + i] / rms * gv[i];
        if (std::fabs(got[r * n + i] - want) > 1e-6 + 1e-5 * std::fabs(want))
          FATAL("RMSNorm[%lld,%lld] = %g, want %g", (long long)r, (long long)i, got[r * n + i], want);
      }
    }
  }
}

// tensor/matmul_fused_test.go:62-71
TEST(TestRowSumSquares) {
  Tensor x = Tensor::New({1, 2, 3, 4, 5, 6}, {2, 3});
  auto ss = x.RowSumSquares();
  if (ss[0] != 14 || ss[1] != 77) FATAL("got %g %g", ss[0], ss[1]);
  auto st = x.T().RowSumSquares();
  if (st[0] != 17 || st[1] != 29 || st[2] != 45) FATAL("transposed: %g %g %g", st[0], st[1], st[2]);
}

static std::vector<double> ref_gemm(const Tensor& a, const Tensor& b) {
  const int64_t m = a.Dim(0), k = a.Dim(1), n = b.Dim(1);
  auto av = a.Float32s(), bv = b.Float32s();
  std::vector<double> c(m * n, 0.0);
  for (int64_t i = 0; i < m; i++)
    for (int64_t p = 0; p < k; p++)
      for (int64_t j = 0; j < n; j++) c[i * n + j] += (double)av[i * k + p] * bv[p * n + j];
  return c;
}

// internal/blas/gemm_test.go:22-56,75-79 (the product through tensor.MatMul,
// including B as a transposed view, gemm_test.go:127-143)
TEST(TestMatMulAgainstFloat64) {
  const int64_t shapes[][3] = {{1, 1, 1}, {1, 17, 5}, {5, 1, 7}, {3, 3, 3}, {13, 33, 9}, {7, 37, 19}, {64, 64, 64},
                               {129, 65, 33}, {133, 257, 300}, {100, 20, 513}, {257, 33, 1}, {31, 4097, 7}};
  std::mt19937_64 rng(2);
  for (auto& s : shapes) {
    const int64_t m = s[0], n = s[1], k = s[2];
    Tensor a = randu(rng, {m, k});
    Tensor b = randu(rng, {k, n});
    auto want = ref_gemm(a, b);
    for (int view = 0; view < 2; view++) {
      Tensor bb = view == 0 ? b : Tensor::New(b.T().Float32s(), {n, k}).T();  // B as a transposed view
      auto got = MatMul(a, bb).Float32s();
      for (int64_t i = 0; i < m * n; i++)
        if (std::fabs(got[i] - want[i]) > 1e-4 * (1 + std::fabs(want[i])))
          FATAL("m=%lld n=%lld k=%lld view=%d: C[%lld] = %g, want %g", (long long)m, (long long)n, (long long)k, view,
                (long long)i, got[i], want[i]);
    }
  }
}

// naiveMatMul (tensor/tensor_test.go:355-368): float64 sums over At(), so
// any 2-D view works.
static Tensor naive_matmul(const Tensor& a, const Tensor& b) {
  const int64_t m = a.Dim(0), k = a.Dim(1), n = b.Dim(1);
  std::vector<float> out(m * n);
  for (int64_t i = 0; i < m; i++)
    for (int64_t j = 0; j < n; j++) {
      double s = 0;
      for (int64_t p = 0; p < k; p++) s += (double)a.At({i, p}) * (double)b.At({p, j});
      out[i * n + j] = (float)s;
    }
  return Tensor::New(std::move(out), {m, n});
}

// assertClose (tensor/tensor_test.go:10-26): |got - want| <= tol (1 + |want|)
static void assert_close(const char* name, const Tensor& got, const Tensor& want, double tol) {
  if (got.shape() != want.shape()) FATAL("%s: shape of rank %d, want rank %d", name, got.Dims(), want.Dims());
  auto g = got.Float32s(), w = want.Float32s();
  for (size_t i = 0; i < g.size(); i++)
    if (!(std::fabs((double)g[i] - w[i]) <= tol * (1 + std::fabs((double)w[i]))))
      FATAL("%s: element %zu = %.9g, want %.9g", name, i, g[i], w[i]);
}

template <class F>
static void expect_tensor_error(const char* name, F fn) {
  try {
    fn();
  } catch (const Error&) {
    return;
  }
  FATAL("%s: expected a tensor error", name);
}

// tensor/tensor_test.go:370-433 (TestMatMul), restated: plain and transposed
// operands at the reference's shapes, the vector forms, batched products
// with broadcasting, the fold of a batch into M, strided batch operands and
// many small products; then offset, stride-0 and empty views.
TEST(TestMatMul) {
  std::mt19937_64 rng(56);
  const int64_t shapes[][3] = {{1, 1, 1}, {2, 3, 4}, {7, 5, 9}, {64, 64, 64}, {33, 17, 65}, {1, 40, 50}, {50, 40, 1}, {130, 70, 90}};
  for (auto& s : shapes) {
    const int64_t m = s[0], k = s[1], n = s[2];
    Tensor a = randn(rng, {m, k}), b = randn(rng, {k, n});
    assert_close("MatMul", MatMul(a, b), naive_matmul(a, b), 1e-4);
    Tensor at = randn(rng, {k, m}).T(), bt = randn(rng, {n, k}).T();  // transposed views, not copied
    assert_close("MatMul AtB", MatMul(at, b), naive_matmul(at, b), 1e-4);
    assert_close("MatMul ABt", MatMul(a, bt), naive_matmul(a, bt), 1e-4);
    assert_close("MatMul AtBt", MatMul(at, bt), naive_matmul(at, bt), 1e-4);
  }
  // vector forms
  Tensor v = Tensor::New({1, 2, 3}, {3});
  Tensor mm = Tensor::New({1, 2, 3, 4, 5, 6}, {2, 3});
  Tensor d = Dot(v, v);
  if (d.Dims() != 0 || d.Item() != 14) FATAL("Dot: rank %d value %g", d.Dims(), d.Item());
  assert_close("M.v", MatMul(mm, v), Tensor::New({14, 32}, {2}), 0);
  assert_close("v.Mt", MatMul(v, mm.T()), Tensor::New({14, 32}, {2}), 0);
  assert_close("Outer", Outer(Tensor::New({1, 2}, {2}), v), Tensor::New({1, 2, 3, 2, 4, 6}, {2, 3}), 0);
  // batched with broadcasting
  Tensor a = randn(rng, {3, 2, 4, 5}), b = randn(rng, {2, 5, 6});
  Tensor got = MatMul(a, b);
  if (got.shape() != Shape{3, 2, 4, 6}) FATAL("batched shape of rank %d", got.Dims());
  for (int64_t i = 0; i < 3; i++)
    for (int64_t j = 0; j < 2; j++)
      assert_close("batched", got.Select(0, i).Select(0, j), naive_matmul(a.Select(0, i).Select(0, j), b.Select(0, j)),
                   1e-4);
  // batched x 2-D folds the batch into M
  Tensor c = randn(rng, {5, 7});
  got = MatMul(a, c);
  for (int64_t i = 0; i < 3; i++)
    for (int64_t j = 0; j < 2; j++)
      assert_close("batched 2D", got.Select(0, i).Select(0, j), naive_matmul(a.Select(0, i).Select(0, j), c), 1e-4);
  // batched with strided (transposed) batch operands
  Tensor bt = randn(rng, {2, 6, 5}).Transpose(1, 2);
  got = MatMul(a, bt);
  for (int64_t i = 0; i < 3; i++)
    for (int64_t j = 0; j < 2; j++)
      assert_close("batched transposed", got.Select(0, i).Select(0, j),
                   naive_matmul(a.Select(0, i).Select(0, j), bt.Select(0, j)), 1e-4);
  // many small products over the batch
  Tensor x = randn(rng, {64, 8, 8}), y = randn(rng, {64, 8, 8});
  got = MatMul(x, y);
  for (int64_t i = 0; i < 64; i += 7)
    assert_close("small batch", got.Select(0, i), naive_matmul(x.Select(0, i), y.Select(0, i)), 1e-4);
  // a strided (non-contiguous) batched left operand against a 2-D right
  // operand: no fold into M, the batch broadcasts the 2-D operand
  Tensor xt = randn(rng, {3, 9, 4}).Transpose(1, 2);  // [3, 4, 9], rows strided
  Tensor w2 = randn(rng, {9, 33});
  got = MatMul(xt, w2);
  for (int64_t i = 0; i < 3; i++) assert_close("strided batch x 2-D", got.Select(0, i), naive_matmul(xt.Select(0, i), w2), 1e-4);
  // offset views (Narrow, Select) and stride-0 broadcasts (Expand)
  Tensor big = randn(rng, {70, 90});
  Tensor an = big.Narrow(0, 3, 40).Narrow(1, 5, 64);   // offset rows and columns, row stride 90
  Tensor bn = randn(rng, {100, 50}).Narrow(0, 17, 64);  // offset rows
  assert_close("narrowed", MatMul(an, bn), naive_matmul(an, bn), 1e-4);
  Tensor brow = randn(rng, {1, 50}).Expand({64, 50});    // every row the same (row stride 0)
  assert_close("expanded", MatMul(an, brow), naive_matmul(an, brow), 1e-4);
  Tensor e3 = randn(rng, {4, 8}).Expand({5, 4, 8});      // batch stride 0 on the left
  Tensor r3 = randn(rng, {5, 8, 3});
  got = MatMul(e3, r3);
  for (int64_t i = 0; i < 5; i++) assert_close("expanded batch", got.Select(0, i), naive_matmul(e3.Select(0, i), r3.Select(0, i)), 1e-4);
  // empty operands: k = 0 gives zeros, m = 0 an empty result
  assert_close("k = 0", MatMul(Tensor::Zeros({3, 0}), Tensor::Zeros({0, 4})), Tensor::Zeros({3, 4}), 0);
  assert_close("m = 0", MatMul(Tensor::Zeros({0, 5}), randn(rng, {5, 4})), Tensor::Zeros({0, 4}), 0);
  expect_tensor_error("shape", [] { MatMul(Tensor::Zeros({2, 3}), Tensor::Zeros({2, 3})); });
  expect_tensor_error("scalar", [] { MatMul(Tensor::Zeros({}), Tensor::Zeros({2})); });
  expect_tensor_error("batch broadcast", [] { MatMul(Tensor::Zeros({2, 3, 4}), Tensor::Zeros({3, 4, 5})); });
}

// MatMulFused reads strided operands as the reference's GemmZeroEpilogue
// does (blas.Mat views, tensor/matmul_fused.go:86-89): a transposed x and w
// give the product of their values.
TEST(TestMatMulFusedStridedOperands) {
  std::mt19937_64 rng(57);
  Tensor x = randn(rng, {48, 33}).T(), w = randn(rng, {70, 48}).T();  // x [33 x 48], w [48 x 70]
  Tensor bias = randn(rng, {70});
  Fused f;
  f.Bias = &bias;
  f.Act = ReLUAct;
  Tensor got = MatMulFused(x, w, f);
  Tensor base = naive_matmul(x, w);
  auto bv = bias.Float32s(), pv = base.Float32s();
  std::vector<float> want(pv.size());
  for (size_t i = 0; i < pv.size(); i++) want[i] = std::max(0.f, pv[i] + bv[i % 70]);
  assert_close("fused strided", got, Tensor::New(want, {33, 70}), 1e-4);
}

// tensor/matmul_fused_test.go:8-44: MatMulFused equals the composed
// operations for every epilogue combination.
TEST(TestMatMulFusedMatchesComposed) {
  std::mt19937_64 rng(3);
  const int64_t m = 33, k = 130, n = 77;
  Tensor x = randu(rng, {m, k}), w = randu(rng, {k, n});
  Tensor bias = randu(rng, {n}), mul = randu(rng, {m, n}), res = randu(rng, {m, n});
  std::vector<float> rs(m);
  for (int64_t i = 0; i < m; i++) rs[i] = 0.5f + (float)i / m;
  auto base = ref_gemm(x, w);
  auto bv = bias.Float32s(), mv = mul.Float32s(), rv = res.Float32s();
  for (int mask = 0; mask < 32; mask++) {
    for (Activation act : {NoAct, ReLUAct, GELUAct}) {
      Fused f;
      if (mask & 1) f.Bias = &bias;
      if (mask & 2) f.RowScale = rs;
      if (mask & 4) f.Mul = &mul;
      if (mask & 8) f.Residual = &res;
      f.Act = act;
      auto got = MatMulFused(x, w, f).Float32s();
      for (int64_t i = 0; i < m; i++)
        for (int64_t j = 0; j < n; j++) {
          double v = (float)base[i * n + j];
          if (f.Bias) v += bv[j];
          if (!f.RowScale.empty()) v *= rs[i];
          if (act == ReLUAct) v = std::max(v, 0.0);
          if (act == GELUAct) v = 0.5 * v * (1 + std::tanh(0.7978845608028654 * (v + 0.044715 * v * v * v)));
          if (f.Mul) v *= mv[i * n + j];
          if (f.Residual) v += rv[i * n + j];
          const double d = std::fabs(got[i * n + j] - v);
          if (d > 1e-4 * (1 + std::fabs(v)))
            FATAL("combo %d act %d: C[%lld,%lld] = %g, want %g", mask, (int)act, (long long)i, (long long)j,
                  got[i * n + j], v);
        }
    }
  }
}

static double naive_att(const std::vector<float>& q, const std::vector<float>& k, const std::vector<float>& v,
                        const std::vector<float>* mask, int T, int S, int D, int i, int c, int64_t qo, int64_t ko,
                        int64_t mo) {
  std::vector<double> w(S);
  double mx = -INFINITY;
  for (int j = 0; j < S; j++) {
    double s = 0;
    for (int d = 0; d < D; d++) s += (double)q[qo + (int64_t)i * D + d] * k[ko + (int64_t)j * D + d];
    s /= std::sqrt((double)D);
    if (mask) s += (*mask)[mo + j];
    w[j] = s;
    mx = std::max(mx, s);
  }
  double sum = 0, out = 0;
  for (int j = 0; j < S; j++) sum += (w[j] = std::exp(w[j] - mx));
  for (int j = 0; j < S; j++) out += w[j] / sum * v[ko + (int64_t)j * D + c];
  return out;
}

// tensor/attention_test.go:56-92
TEST(TestAttentionMatchesNaive) {
  std::mt19937_64 rng(41);
  const int B = 2, H = 3, T = 5, S = 7, D = 4;
  Tensor q = randn(rng, {B, H, T, D}), k = randn(rng, {B, H, S, D}), v = randn(rng, {B, H, S, D});
  auto qv = q.Float32s(), kv = k.Float32s(), vv = v.Float32s();
  for (int withMask = 0; withMask < 2; withMask++) {
    Tensor mask = PaddingMask({S, 3}, S);
    auto mv = mask.Float32s();
    Tensor out = Attention(q, k, v, withMask ? &mask : nullptr);
    for (int b = 0; b < B; b++)
      for (int h = 0; h < H; h++)
        for (int i = 0; i < T; i++)
          for (int c = 0; c < D; c++) {
            const double want = naive_att(qv, kv, vv, withMask ? &mv : nullptr, T, S, D, i, c,
                                          ((int64_t)b * H + h) * T * D, ((int64_t)b * H + h) * S * D, (int64_t)b * S);
            const double got = out.At({b, h, i, c});
            if (std::fabs(got - want) > 1e-4)
              FATAL("mask=%d b=%d h=%d out[%d,%d] = %g, want %g", withMask, b, h, i, c, got, want);
          }
  }
}

// tensor/attention_test.go:94-118
TEST(TestCausalMaskHidesTheFuture) {
  std::mt19937_64 rng(1);
  const int T = 6, D = 8;
  Tensor q = randn(rng, {1, 1, T, D}), k = randn(rng, {1, 1, T, D}), v = randn(rng, {1, 1, T, D});
  Tensor cm = CausalMask(T);
  Tensor out = Attention(q, k, v, &cm);
  auto k2 = k.Float32s(), v2 = v.Float32s();
  for (int c = 0; c < D; c++) {
    k2[(T - 1) * D + c] += 5;
    v2[(T - 1) * D + c] -= 3;
  }
  Tensor out2 = Attention(q, Tensor::New(k2, {1, 1, T, D}), Tensor::New(v2, {1, 1, T, D}), &cm);
  for (int i = 0; i < T - 1; i++)
    for (int c = 0; c < D; c++)
      if (out.At({0, 0, i, c}) != out2.At({0, 0, i, c})) FATAL("position %d changed when the last key changed", i);
  if (out.At({0, 0, T - 1, 0}) == out2.At({0, 0, T - 1, 0})) FATAL("the last position ignored its own key");
}

// tensor/attention_test.go:266-285
TEST(TestMaskedAttentionWeightsAreExactZeros) {
  std::mt19937_64 rng(11);
  const int n = 64, d = 16;
  Tensor q = randn(rng, {1, 1, n, d}), k = randn(rng, {1, 1, n, d}), v = randn(rng, {1, 1, n, d});
  Tensor cm = CausalMask(n);
  Tensor out = Attention(q, k, v, &cm);
  for (int c = 0; c < d; c++)
    if (std::fabs(out.At({0, 0, 0, c}) - v.At({0, 0, 0, c})) > 1e-6) FATAL("position 0 must reproduce v[0]");
}

// Grouped-query attention through Expand (models/gemma/embed.go:209): one
// key/value head viewed as three gives the same result as three copies.
TEST(TestAttentionGQAExpand) {
  std::mt19937_64 rng(5);
  const int B = 2, H = 3, T = 40, D = 256;
  Tensor q = randn(rng, {B, H, T, D});
  Tensor k1 = randn(rng, {B, 1, T, D}), v1 = randn(rng, {B, 1, T, D});
  Tensor mask = PaddingMask({40, 23}, T);
  Tensor a = AttentionScaled(q, k1.Expand({B, H, T, D}), v1.Expand({B, H, T, D}), &mask, 0.0625f);
  Tensor b = AttentionScaled(q, k1.Expand({B, H, T, D}).Contiguous(), v1.Expand({B, H, T, D}).Contiguous(), &mask,
                             0.0625f);
  auto av = a.Float32s(), bv = b.Float32s();
  for (size_t i = 0; i < av.size(); i++)
    if (av[i] != bv[i]) FATAL("Expand view and copy differ at %zu: %g vs %g", i, av[i], bv[i]);
}

template <class F>
static void expect_error(const char* op, F&& f) {
  try {
    f();
  } catch (const Error& e) {
    if (e.Op != op) FATAL("error Op %s, want %s (%s)", e.Op.c_str(), op, e.what());
    return;
  }
  FATAL("expected a tensor.Error from %s", op);
}

// The reference panics with *tensor.Error{Op, Msg} on shape errors.
TEST(TestShapeErrors) {
  expect_error("MatMul", [] { MatMul(Tensor::Zeros({2, 3}), Tensor::Zeros({4, 5})); });
  expect_error("MatMulFused", [] {
    Tensor bias = Tensor::Zeros({4});
    Fused f;
    f.Bias = &bias;
    MatMulFused(Tensor::Zeros({2, 3}), Tensor::Zeros({3, 5}), f);
  });
  expect_error("RMSNorm", [] { RMSNorm(Tensor::Zeros({2, 8}), Tensor::Zeros({7}), 1e-6f); });
  expect_error("RoPE", [] { RoPE(Tensor::Zeros({2, 3}), 1e4, {0, 1}); });
  expect_error("RoPE", [] { RoPE(Tensor::Zeros({2, 4}), 1e4, {0}); });
  expect_error("Attention", [] { Attention(Tensor::Zeros({1, 2, 4}), Tensor::Zeros({2, 4}), Tensor::Zeros({2, 4}), nullptr); });
  expect_error("RowSumSquares", [] { Tensor::Zeros({2, 3, 4}).RowSumSquares(); });
  expect_error("Expand", [] { Tensor::Zeros({2, 3}).Expand({4, 3}); });
}

int main(int argc, char** argv) { return ctest::run_all(argc, argv); }
