// gemma.LoadConfig of the C++ host mirror on the CPU (no weights, no GPU):
// the reference's TestConfig2 (models/gemma/gemma2_test.go:44-95) restated,
// plus EmbeddingGemma 2's defaults and refusals (config.go:247-297) and the
// Gemma 3 encoder's config. Run by tests/test_cpp_host.py.
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <string>

#include "fiber.hpp"
#include "testing.hpp"

using namespace fiber;

static std::string temp_dir() {
  char tmpl[] = "/tmp/fa_config_XXXXXX";
  const char* d = mkdtemp(tmpl);
  if (!d) FATAL("mkdtemp failed");
  return d;
}

static gemma::Config load(const std::string& json) {
  const std::string dir = temp_dir();
  std::ofstream(dir + "/config.json") << json;
  gemma::Config c = gemma::LoadConfig(dir);
  std::remove((dir + "/config.json").c_str());
  std::remove(dir.c_str());
  return c;
}

static std::string load_error(const std::string& json) {
  try {
    load(json);
  } catch (const gemma::Error& e) {
    return e.what();
  }
  return "";
}

static const char* kConfig2 = R"({"model_type": "embedding_gemma2", "vision_config": {"hidden_size": 768},
  "text_config": {"hidden_size": 512, "intermediate_size": 2048, "num_hidden_layers": 12,
    "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 256, "vocab_size": 262144,
    "sliding_window": 512, "rms_norm_eps": 1e-6, "hidden_activation": "gelu_pytorch_tanh",
    "hidden_size_per_layer_input": 512, "embedding_dim": 768, "max_position_embeddings": 262144,
    "per_layer_config": {"05": {"head_dim": 512, "num_key_value_heads": 1},
                         "11": {"head_dim": 512, "num_key_value_heads": 1}},
    "rope_parameters": {"full_attention": {"rope_theta": 1000000.0, "rope_type": "default"},
                        "sliding_attention": {"rope_theta": 10000.0, "rope_type": "default"}}}})";

// gemma2_test.go:44-95
TEST(TestConfig2) {
  const gemma::Config c = load(kConfig2);
  if (c.Variant != 2 || c.HiddenSize != 512 || c.EmbeddingDim != 768)
    FATAL("variant %d, hidden %d, embedding %d", c.Variant, c.HiddenSize, c.EmbeddingDim);
  const struct {
    int layer, head_dim, kv;
    bool sliding;
    double base;
  } cases[] = {{0, 256, 2, true, 1e4}, {4, 256, 2, true, 1e4}, {5, 512, 1, false, 1e6}, {11, 512, 1, false, 1e6}};
  for (const auto& tc : cases) {
    if (c.LayerHeadDim(tc.layer) != tc.head_dim) FATAL("layer %d head_dim %d, want %d", tc.layer, c.LayerHeadDim(tc.layer), tc.head_dim);
    if (c.LayerKVHeads(tc.layer) != tc.kv) FATAL("layer %d kv heads %d, want %d", tc.layer, c.LayerKVHeads(tc.layer), tc.kv);
    if (c.IsSliding(tc.layer) != tc.sliding) FATAL("layer %d sliding %d", tc.layer, (int)c.IsSliding(tc.layer));
    if (c.RopeBase(tc.layer) != tc.base) FATAL("layer %d rope base %g, want %g", tc.layer, c.RopeBase(tc.layer), tc.base);
  }
  // an inclusive radius of 512: attend while |i-j| < 513
  if (c.Window() != 513) FATAL("window bound %d, want 513", c.Window());
  if (c.MaxTokens != 8192) FATAL("max tokens %d, want the model card's 8192", c.MaxTokens);
}

// fillVariant2's defaults (config.go:249-281): layer types 5:1, full layers
// head_dim 512 with one key/value head, rope bases 1e4 / 1e6, embedding 768.
TEST(TestVariant2Defaults) {
  const gemma::Config c = load(R"({"model_type": "embedding_gemma2", "image_token_id": 258880,
    "boi_token_id": 255999, "eoi_token_id": 258882, "vision_config": {"hidden_size": 768},
    "text_config": {"hidden_size": 512, "intermediate_size": 2048, "num_hidden_layers": 12,
    "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 256, "vocab_size": 1000,
    "sliding_window": 512, "rms_norm_eps": 1e-6, "hidden_size_per_layer_input": 256}})");
  if (c.LayerTypes.size() != 12 || c.LayerTypes[5] != "full_attention" || c.LayerTypes[4] != "sliding_attention")
    FATAL("default layer types");
  if (c.LayerHeadDim(11) != 512 || c.LayerKVHeads(11) != 1 || c.LayerHeadDim(10) != 256 || c.LayerKVHeads(10) != 2)
    FATAL("default per-layer geometry");
  if (c.RopeBase(0) != 1e4 || c.RopeBase(5) != 1e6) FATAL("default rope bases");
  if (c.EmbeddingDim != 768 || c.HiddenSizePerLayerInput != 256) FATAL("embedding %d ple %d", c.EmbeddingDim, c.HiddenSizePerLayerInput);
  if (!c.HasVision || c.ImageToken != 258880 || c.MultimodalTokens.at(255999) != "begin-of-image")
    FATAL("multimodal placeholders");
}

TEST(TestVariant2Refusals) {
  std::string e = load_error(R"({"model_type": "embedding_gemma2", "text_config": {"hidden_size": 512,
    "num_hidden_layers": 2, "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 256}})");
  if (e.find("without hidden_size_per_layer_input") == std::string::npos) FATAL("missing ple: %s", e.c_str());
  e = load_error(R"({"model_type": "embedding_gemma2", "text_config": {"hidden_size": 512, "num_hidden_layers": 2,
    "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 256, "hidden_size_per_layer_input": 64,
    "rope_parameters": {"full_attention": {"rope_theta": 1e6, "rope_type": "proportional"}}}})");
  if (e.find("rope_type \"proportional\"") == std::string::npos) FATAL("rope type: %s", e.c_str());
  e = load_error(R"({"model_type": "embedding_gemma2", "text_config": {"hidden_size": 512, "num_hidden_layers": 2,
    "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 256, "hidden_size_per_layer_input": 64,
    "layer_types": ["sliding_attention"]}})");
  if (e.find("1 layer types for 2 layers") == std::string::npos) FATAL("layer types: %s", e.c_str());
  e = load_error(R"({"model_type": "embedding_gemma2", "text_config": {"hidden_size": 512, "num_hidden_layers": 2,
    "num_attention_heads": 4, "num_key_value_heads": 2, "head_dim": 256, "hidden_size_per_layer_input": 64,
    "per_layer_config": {"01": {"head_dim": 512, "num_key_value_heads": 3}}}})");
  if (e.find("layer 1: 4 query heads not a multiple of 3") == std::string::npos) FATAL("kv heads: %s", e.c_str());
}

// The Gemma 3 encoder's config (config.go:153-240): window bound w/2+1 when
// bidirectional, (1+w) norms, 2048-token cap.
TEST(TestConfigGemma3) {
  const gemma::Config c = load(R"({"model_type": "gemma3_text", "hidden_size": 768, "intermediate_size": 1152,
    "num_hidden_layers": 24, "num_attention_heads": 3, "num_key_value_heads": 1, "head_dim": 256,
    "vocab_size": 262144, "sliding_window": 512, "use_bidirectional_attention": true, "rope_theta": 1000000.0,
    "rope_local_base_freq": 10000.0, "query_pre_attn_scalar": 256, "rms_norm_eps": 1e-6,
    "max_position_embeddings": 2048, "hidden_activation": "gelu_pytorch_tanh"})");
  if (c.Variant != 0 || c.Window() != 257 || c.MaxTokens != 2048) FATAL("variant %d window %d", c.Variant, c.Window());
  if (!c.IsSliding(4) || c.IsSliding(5) || c.RopeBase(5) != 1e6 || c.RopeBase(0) != 1e4) FATAL("layer pattern");
}

int main(int argc, char** argv) { return ctest::run_all(argc, argv); }
