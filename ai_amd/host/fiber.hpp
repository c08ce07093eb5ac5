// fiber.hpp — C++ host mirror of fiber/ai's Go API on the EmbeddingGemma
// path, computed on the GPU through the C ABI (include/fa_rocm.h).
//
// The names, argument meaning and error behaviour follow the reference:
//   tensor.MatMul / MatMulFused / Fused        tensor/matmul.go:19, matmul_fused.go:17-96
//   (*Tensor).RowSumSquares                    tensor/matmul_fused.go:125-143
//   tensor.RMSNorm                             tensor/attention.go:292-337
//   tensor.RoPE                                tensor/rope.go:20-61
//   tensor.Attention / AttentionScaled         tensor/attention.go:56-83
//   tensor.PaddingMask / WindowMask / CausalMask   tensor/attention.go:21-42,97-107
//   (*Tensor).Expand (stride-0 views)          tensor/view.go
//   gemma.Load / LoadConfig / Model.Embed (texts, prompts, Dim), Dim, Close
//                                              models/gemma/model.go:76-330,336-382; config.go:153-240;
//                                              embed.go:15-114 (EmbedIDs: the ids-level core, embed.go:118-157)
//   tokenizer.Tokenizer                        tokenizer/tokenizer.go (tokenizer.hpp)
//   safetensors.File                           safetensors/safetensors.go (safetensors.hpp)
//   cluster.Normalize / KMeans / Nearest / Cosine / Similarities
//                                              cluster/cluster.go (cluster.hpp)
// Shape errors throw fiber::tensor::Error{Op, Msg}, where the reference
// panics with *tensor.Error (tensor/errors.go:5-31); gemma's functions throw
// fiber::gemma::Error where the reference returns error.
//
// Tensors here are host arrays (float32, row-major, with strides so that
// Expand views exist); every operator copies its operands to the device,
// computes there and returns a new contiguous tensor, like the reference's
// operators return fresh tensors.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "fa_rocm.h"
#include "tokenizer.hpp"

namespace fiber {

// The process-wide GPU context (device 0), created on first use.
fa_ctx* device();

namespace tensor {

struct Error : std::runtime_error {
  std::string Op, Msg;
  Error(std::string op, std::string msg)
      : std::runtime_error("tensor: " + op + ": " + msg), Op(std::move(op)), Msg(std::move(msg)) {}
};

using Shape = std::vector<int64_t>;

class Tensor {
 public:
  Tensor() = default;
  // New copies data into a fresh tensor of the given shape (tensor.New).
  static Tensor New(std::vector<float> data, Shape shape);
  static Tensor Zeros(Shape shape);

  const Shape& shape() const { return shape_; }
  const Shape& strides() const { return strides_; }
  int64_t Dim(int i) const { return shape_[i < 0 ? i + (int)shape_.size() : i]; }
  int Dims() const { return (int)shape_.size(); }
  int64_t Size() const;
  bool IsContiguous() const;
  // Element access by full index (views included).
  float At(std::initializer_list<int64_t> idx) const;
  // Contiguous copy of the values in row-major order (Float32s).
  std::vector<float> Float32s() const;
  Tensor Contiguous() const;
  Tensor Reshape(Shape shape) const;
  // View broadcasting dimensions of size 1 to shape (stride 0), tensor.Expand.
  Tensor Expand(Shape shape) const;
  // Transposed view of a 2-D tensor (T).
  Tensor T() const;
  // Views (tensor/view.go): dimensions d0 and d1 swapped (negative dims count
  // from the end); the slice at index of dimension dim, which is removed;
  // length elements of dimension dim from start; a new dimension of size 1
  // at dim; dimension dim (of size 1) removed.
  Tensor Transpose(int d0, int d1) const;
  Tensor Select(int dim, int64_t index) const;
  Tensor Narrow(int dim, int64_t start, int64_t length) const;
  Tensor Unsqueeze(int dim) const;
  Tensor Squeeze(int dim) const;
  // The single value of a tensor with one element (Item).
  float Item() const;

  // (*Tensor).RowSumSquares: sum of squares of each row of a 2-D tensor.
  std::vector<float> RowSumSquares() const;

  const float* base() const { return store_ ? store_->data() + offset_ : nullptr; }

 private:
  std::shared_ptr<std::vector<float>> store_;
  int64_t offset_ = 0;
  Shape shape_, strides_;
  friend Tensor AttentionScaled(const Tensor&, const Tensor&, const Tensor&, const Tensor*, float);
};

enum Activation { NoAct = FA_ACT_NONE, ReLUAct = FA_ACT_RELU, GELUAct = FA_ACT_GELU };

// Epilogue of MatMulFused, applied in the order Bias, RowScale, Act, Mul,
// Residual (tensor/matmul_fused.go:11-23). Null pointers / empty RowScale
// are skipped.
struct Fused {
  const Tensor* Bias = nullptr;
  Activation Act = NoAct;
  const Tensor* Mul = nullptr;
  std::vector<float> RowScale;
  const Tensor* Residual = nullptr;
};

// tensor.MatMul (tensor/matmul.go:10-36): NumPy semantics. 2-D x 2-D is the
// matrix product; a 1-D operand is promoted to a row (left) or column
// (right) and the added dimension removed; with more dimensions the batch
// dimensions broadcast. Strided views (T, Transpose, Select, Narrow,
// Expand) are read through their strides on the device, not copied.
Tensor MatMul(const Tensor& x, const Tensor& w);
// Inner product of two 1-D tensors as a 0-D tensor; outer product of two
// 1-D tensors (tensor/matmul.go:131-150).
Tensor Dot(const Tensor& x, const Tensor& y);
Tensor Outer(const Tensor& x, const Tensor& y);
Tensor MatMulFused(const Tensor& x, const Tensor& w, const Fused& f);
Tensor RMSNorm(const Tensor& x, const Tensor& g, float eps);
Tensor RoPE(const Tensor& x, double base, const std::vector<int>& positions);
Tensor Attention(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor* mask);
Tensor AttentionScaled(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor* mask, float scale);
Tensor PaddingMask(const std::vector<int>& lengths, int64_t n);
Tensor WindowMask(int64_t n, int64_t w);
Tensor CausalMask(int64_t n);

constexpr float kMaskNeg = -1e9f;  // tensor/attention.go:17

}  // namespace tensor

namespace gemma {

struct Error : std::runtime_error {
  explicit Error(const std::string& m) : std::runtime_error(m) {}
};

// Per-layer geometry override of EmbeddingGemma 2 (config.go:141-144).
struct LayerOverride {
  int HeadDim = 0, NumKeyValueHeads = 0;
};

// Hyper-parameters of config.json (models/gemma/config.go:19-58) and the
// sentence-transformers Dense head; defaults are EmbeddingGemma-300M
// (Variant 0). Variant 2 is EmbeddingGemma 2's text tower, read from the
// nested text_config with its defaults (config.go:247-297).
struct Config {
  int HiddenSize = 768, NumHiddenLayers = 24, NumAttentionHeads = 3, NumKeyValueHeads = 1, HeadDim = 256;
  int IntermediateSize = 1152, VocabSize = 262144, SlidingWindow = 512, SlidingWindowPattern = 6;
  bool UseBidirectional = true;
  double RopeLocalBaseFreq = 1e4, RopeTheta = 1e6, QueryPreAttnScalar = 256;
  float RMSNormEps = 1e-6f;
  int MaxTokens = 2048;
  std::vector<int> Dense = {3072, 768};
  std::vector<int> DenseAct;  // per Dense layer: FA_ACT_NONE (identity) or FA_ACT_TANH; empty: all identity
  // EmbeddingGemma 2 only (zero / empty for Variant 0)
  int Variant = 0;
  int HiddenSizePerLayerInput = 0, EmbeddingDim = 0;
  std::vector<std::string> LayerTypes;              // "sliding_attention" / "full_attention" per layer
  std::map<std::string, LayerOverride> PerLayerConfig;  // keyed by zero-padded layer index ("05")
  std::map<std::string, double> RopeThetaByType;    // rope_parameters (config.go:147-150): type -> rope_theta
  std::map<int, std::string> MultimodalTokens;      // placeholder ids -> name (embed.go:82-97)
  int ImageToken = -1, AudioToken = -1;
  bool HasVision = false, HasAudio = false;

  // config.go:299-366: a layer's head dim and key/value heads (with the
  // per-layer override), whether it uses the sliding window, its RoPE base,
  // and the window bound (positions attend while |i-j| < Window()).
  int LayerHeadDim(int l) const;
  int LayerKVHeads(int l) const;
  bool IsSliding(int l) const;
  double RopeBase(int l) const;
  int Window() const;
};

// Options of Embed (model.go:372-379): Dim truncates before L2
// (Matryoshka); Prompt names a prompt of config_sentence_transformers.json,
// PromptText gives the prefix itself (has_prompt_text marks it as set).
struct EmbedOpts {
  int Dim = 0;
  std::string Prompt;
  std::string PromptText;
  bool has_prompt_text = false;
};

// Options of Load (model.go:352-359): MaxTokens truncates sequences (0: the
// config's max_position_embeddings, at most 2048); BatchTokens bounds
// batch size x longest length per forward pass.
struct LoadOpts {
  int MaxTokens = 0;
  int BatchTokens = 8192;
};

// config.json of a Gemma 3 text model or an EmbeddingGemma 2 checkpoint
// (config.go:153-297): the fields the encoder uses, defaults filled and
// validated as the reference does.
Config LoadConfig(const std::string& dir);

class Model {
 public:
  // Reads a model directory in the Hugging Face / sentence-transformers
  // layout: config.json, tokenizer.json, *.safetensors (+ index), and the
  // modules.json Pooling (mean), Dense (no bias; identity or Tanh) and
  // Normalize modules with config_sentence_transformers.json prompts
  // (model.go:76-330).
  // EmbeddingGemma 2 directories add the per-layer-input weights, the layer
  // scalars and the embedding projection (model.go:163-205).
  static std::unique_ptr<Model> Load(const std::string& dir, const LoadOpts& o = {});
  explicit Model(const Config& cfg);
  ~Model();
  Model(const Model&) = delete;
  Model& operator=(const Model&) = delete;
  // One checkpoint tensor by its Hugging Face name (gemma.Load's names,
  // model.go:142-191); bf16 bits or float32, shape [out, in] for matrices.
  void SetWeightBF16(const std::string& name, const std::vector<int64_t>& shape, const uint16_t* data);
  void SetWeightF32(const std::string& name, const std::vector<int64_t>& shape, const float* data);
  void Finalize();
  // Embeddings of token-id sequences (each already tokenised with BOS),
  // batched in one forward pass; sequences longer than MaxTokens are
  // truncated (embed.go:40-42). Returns one row per sequence.
  std::vector<std::vector<float>> EmbedIDs(const std::vector<std::vector<int32_t>>& ids, EmbedOpts o = {}) const;
  // Embeddings of texts (embed.go:15-80): prompt prefix, tokenizer with its
  // BOS/EOS template, truncation to MaxTokens, batches of similar length
  // under BatchTokens, input order restored. Needs a model from Load.
  std::vector<std::vector<float>> Embed(const std::vector<std::string>& texts, const EmbedOpts& o = {}) const;
  int Dim() const;
  const Config& GetConfig() const { return cfg_; }
  const tokenizer::Tokenizer* GetTokenizer() const { return tok_.get(); }
  void Close();

 private:
  Config cfg_;
  fa_model* m_ = nullptr;
  std::unique_ptr<tokenizer::Tokenizer> tok_;
  std::map<std::string, std::string> prompts_;
  int batch_tokens_ = 8192;
};

}  // namespace gemma
}  // namespace fiber
