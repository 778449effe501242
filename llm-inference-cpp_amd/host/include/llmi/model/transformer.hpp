// llmi::Transformer and llmi::KVCache on the MI355X: the interface of the
// reference's include/llmi/model/transformer.hpp:14-120 for the quantized
// path.  Every weight matrix, the activations and the KV cache live in HBM;
// only token ids go in and logits (or ids) come out.  Logits and greedy ids
// are bit-identical to the reference's for the same weights.
//
// load() takes the reference's ModelConfig fields and a reader that returns
// each tensor (by its expected_tensors() name) as fp32.  Built inside the
// reference engine (LLMI_GPU_WITH_REFERENCE_MODEL defined, its include
// directory on the path), ModelConfig / Arch / TokenId are the reference's
// own and the reference's load(const Model&, quant::Type) signature is
// available too (host/integration/load_from_model.cpp).
#pragma once

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "llmi/model/quant.hpp"
#include "llmi/model/sampling.hpp"
#include "llmi/util/result.hpp"

struct llmi_hip_model;
struct llmi_hip_cache;

#if defined(LLMI_GPU_WITH_REFERENCE_MODEL)
#include "llmi/model/model.hpp"
#include "llmi/tokenizer/tokenizer.hpp"
#endif

namespace llmi {

#if !defined(LLMI_GPU_WITH_REFERENCE_MODEL)
using TokenId = std::int32_t;

enum class Arch : std::uint8_t { Llama, Qwen2 };

// The fields of the reference's ModelConfig (include/llmi/model/model.hpp:21-36).
struct ModelConfig {
  Arch arch = Arch::Llama;
  std::uint32_t vocab_size = 0;
  std::uint32_t hidden_size = 0;
  std::uint32_t intermediate_size = 0;
  std::uint32_t num_layers = 0;
  std::uint32_t num_heads = 0;
  std::uint32_t num_kv_heads = 0;
  std::uint32_t head_dim = 0;
  std::uint32_t max_position_embeddings = 0;
  double rms_norm_eps = 0;
  double rope_theta = 0;
  bool tie_word_embeddings = false;
  bool qkv_bias = false;
  std::vector<std::int32_t> eos_token_ids;
};
#endif

// Tensor names in the reference's expected_tensors() order
// (src/model/model.cpp:135-162).
std::vector<std::string> expected_tensor_names(const ModelConfig& cfg);

struct ForwardTrace {
  std::vector<std::vector<float>> states;
};

class KVCache {
 public:
  [[nodiscard]] std::size_t length() const;
  [[nodiscard]] std::size_t capacity() const;
  void reset();

 private:
  friend class Transformer;
  std::shared_ptr<llmi_hip_cache> dev_;
};

using TensorReader = std::function<Result<std::vector<float>>(const std::string& name)>;

class Transformer {
 public:
  static Result<Transformer> load(const ModelConfig& cfg, const TensorReader& read, quant::Type weight_type);
#if defined(LLMI_GPU_WITH_REFERENCE_MODEL)
  // The reference's signature (transformer.hpp:58).
  static Result<Transformer> load(const Model& model, quant::Type weight_type = quant::Type::F32);
#endif

  [[nodiscard]] const ModelConfig& config() const { return cfg_; }
  [[nodiscard]] std::size_t weight_bytes() const;

  [[nodiscard]] Result<std::vector<float>> forward(const std::vector<TokenId>& tokens, bool all_positions = false,
                                                   ForwardTrace* trace = nullptr) const;
  [[nodiscard]] Result<std::vector<TokenId>> generate_greedy(std::vector<TokenId> tokens, std::size_t max_new,
                                                             const std::vector<TokenId>& stop_ids) const;
  [[nodiscard]] Result<KVCache> new_cache(std::size_t max_len) const;
  [[nodiscard]] Result<std::vector<float>> forward_cached(const std::vector<TokenId>& tokens, KVCache& cache,
                                                          bool all_positions = false,
                                                          ForwardTrace* trace = nullptr) const;
  [[nodiscard]] Result<std::vector<TokenId>> generate_greedy_cached(const std::vector<TokenId>& prompt,
                                                                    std::size_t max_new,
                                                                    const std::vector<TokenId>& stop_ids) const;

  // One serving step without the logits leaving the GPU: forward_cached(tokens,
  // cache) followed by sample(logits, cfg, rng), as the loop of
  // src/server/server.cpp:109-195 does, with the same draws from rng and the
  // same token.  (No counterpart in the reference's class.)
  [[nodiscard]] Result<TokenId> forward_sample(const std::vector<TokenId>& tokens, KVCache& cache,
                                               const SamplingConfig& cfg, std::mt19937_64& rng) const;

 private:
  ModelConfig cfg_;
  std::shared_ptr<llmi_hip_model> dev_;
};

// Index of the first maximum (transformer.hpp:118-120).
std::size_t argmax(const float* x, std::size_t n);

}  // namespace llmi
