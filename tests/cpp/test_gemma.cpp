// gemma.Model of the C++ host mirror (ai_amd/host/fiber.hpp) on the GPU:
// a small random-init encoder of the real widths, checked for the
// properties the reference's model tests assert (models/gemma/gemma_test.go:
// unit-norm embeddings, batch/padding invariance :117-135, Matryoshka Dim
// :137-161) and for its error behaviour (embed.go:24-30). Parity with the
// CPU oracle is covered by tests/test_gpu_model.py and tests/test_golden.py.
#include <cmath>
#include <random>

#include "fa_synth.h"
#include "fiber.hpp"
#include "testing.hpp"

using namespace fiber::gemma;

static Config small_config() {
  Config c;
  c.NumHiddenLayers = 2;
  c.VocabSize = 4096;
  c.SlidingWindowPattern = 2;  // layer 0 sliding, layer 1 global
  c.MaxTokens = 512;
  return c;
}

static void load_synthetic(Model& m, const Config& c) {
  const int d = c.HiddenSize, H = c.NumAttentionHeads, Hkv = c.NumKeyValueHeads, D = c.HeadDim, F = c.IntermediateSize;
  const uint64_t seed = 99;
  auto mat = [&](const std::string& name, int64_t out, int64_t in) {
    std::vector<uint16_t> w((size_t)(out * in));
    fa_synth_normal_bf16(seed, name.c_str(), 0.02, out * in, w.data());
    m.SetWeightBF16(name, {out, in}, w.data());
  };
  auto norm = [&](const std::string& name, int64_t n) {
    std::vector<float> w((size_t)n);
    fa_synth_normal_f32(seed, name.c_str(), 0.1, n, w.data());
    m.SetWeightF32(name, {n}, w.data());
  };
  mat("embed_tokens.weight", c.VocabSize, d);
  for (int l = 0; l < c.NumHiddenLayers; l++) {
    const std::string p = "layers." + std::to_string(l) + ".";
    for (const char* n : {"input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                          "post_feedforward_layernorm"})
      norm(p + n + ".weight", d);
    norm(p + "self_attn.q_norm.weight", D);
    norm(p + "self_attn.k_norm.weight", D);
    mat(p + "self_attn.q_proj.weight", (int64_t)H * D, d);
    mat(p + "self_attn.k_proj.weight", (int64_t)Hkv * D, d);
    mat(p + "self_attn.v_proj.weight", (int64_t)Hkv * D, d);
    mat(p + "self_attn.o_proj.weight", d, (int64_t)H * D);
    mat(p + "mlp.gate_proj.weight", F, d);
    mat(p + "mlp.up_proj.weight", F, d);
    mat(p + "mlp.down_proj.weight", d, F);
  }
  norm("norm.weight", d);
  int64_t in = d;
  for (size_t i = 0; i < c.Dense.size(); i++) {
    mat("dense." + std::to_string(i) + ".linear.weight", c.Dense[i], in);
    in = c.Dense[i];
  }
  m.Finalize();
}

static std::vector<std::vector<int32_t>> sequences() {
  std::mt19937 rng(3);
  std::uniform_int_distribution<int> tok(3, 4095);
  std::vector<std::vector<int32_t>> s;
  for (int L : {300, 41, 1, 128}) {  // one longer than the 257 window bound
    std::vector<int32_t> ids(L);
    ids[0] = 2;  // BOS
    for (int i = 1; i < L; i++) ids[i] = tok(rng);
    s.push_back(ids);
  }
  return s;
}

static double cosine(const std::vector<float>& a, const std::vector<float>& b, size_t n) {
  double d = 0, na = 0, nb = 0;
  for (size_t i = 0; i < n; i++) {
    d += (double)a[i] * b[i];
    na += (double)a[i] * a[i];
    nb += (double)b[i] * b[i];
  }
  return d / (std::sqrt(na) * std::sqrt(nb) + 1e-12);
}

TEST(TestEmbedUnitNormAndBatchInvariance) {
  Config c = small_config();
  Model m(c);
  load_synthetic(m, c);
  auto seqs = sequences();
  auto all = m.EmbedIDs(seqs);
  if ((int)all.size() != 4 || (int)all[0].size() != m.Dim()) FATAL("shape %zu x %zu", all.size(), all[0].size());
  for (size_t i = 0; i < seqs.size(); i++) {
    double n2 = 0;
    for (float v : all[i]) n2 += (double)v * v;
    if (std::fabs(std::sqrt(n2) - 1) > 1e-5) FATAL("row %zu norm %g", i, std::sqrt(n2));
    auto alone = m.EmbedIDs({seqs[i]});
    const double cs = cosine(alone[0], all[i], all[i].size());
    if (cs < 0.9999) FATAL("sequence %zu alone vs batched: cosine %.8f", i, cs);
  }
}

TEST(TestEmbedDimTruncatesBeforeL2) {
  Config c = small_config();
  Model m(c);
  load_synthetic(m, c);
  auto seqs = sequences();
  auto full = m.EmbedIDs(seqs);
  EmbedOpts o;
  o.Dim = 256;
  auto cut = m.EmbedIDs(seqs, o);
  for (size_t i = 0; i < seqs.size(); i++) {
    if (cut[i].size() != 256) FATAL("Dim(256) gave %zu values", cut[i].size());
    double n2 = 0;
    for (float v : cut[i]) n2 += (double)v * v;
    if (std::fabs(std::sqrt(n2) - 1) > 1e-5) FATAL("truncated row %zu norm %g", i, std::sqrt(n2));
    // the truncated vector is the normalised prefix of the same head output
    if (cosine(cut[i], full[i], 256) < 0.99999) FATAL("row %zu prefix direction differs", i);
  }
}

TEST(TestEmbedErrors) {
  Config c = small_config();
  Model m(c);
  bool threw = false;
  try {
    m.EmbedIDs(sequences());  // before Finalize
  } catch (const Error&) {
    threw = true;
  }
  if (!threw) FATAL("embedding before every weight is set must fail");
  load_synthetic(m, c);
  for (int bad : {-1, 769}) {
    threw = false;
    try {
      EmbedOpts o;
      o.Dim = bad;
      m.EmbedIDs(sequences(), o);
    } catch (const Error& e) {
      threw = std::string(e.what()).find("Dim(") != std::string::npos;
    }
    if (!threw) FATAL("Dim(%d) must fail with the reference's message", bad);
  }
  threw = false;
  try {
    m.EmbedIDs({{2, 5, 4096}});  // id outside the vocabulary
  } catch (const Error&) {
    threw = true;
  }
  if (!threw) FATAL("an id outside the vocabulary must fail");
}

int main(int argc, char** argv) { return ctest::run_all(argc, argv); }
