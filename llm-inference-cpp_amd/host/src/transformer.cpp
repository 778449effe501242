// llmi::Transformer on the GPU (the reference's src/model/transformer.cpp
// interface): the device-resident model of libllmi_hip.so behind the
// reference's load / forward / forward_cached / generate API.
#include "llmi/model/transformer.hpp"

#include <algorithm>
#include <stdexcept>
#include <string>

#include "llmi_hip.h"

namespace llmi::quant {
void init_for_host_api();
}

namespace llmi {

namespace {

llmi_model_config abi_config(const ModelConfig& c) {
  llmi_model_config a{};
  a.arch = c.arch == Arch::Qwen2 ? 1 : 0;
  a.vocab_size = c.vocab_size;
  a.hidden_size = c.hidden_size;
  a.intermediate_size = c.intermediate_size;
  a.num_layers = c.num_layers;
  a.num_heads = c.num_heads;
  a.num_kv_heads = c.num_kv_heads;
  a.max_position_embeddings = c.max_position_embeddings;
  a.rms_norm_eps = c.rms_norm_eps;
  a.rope_theta = c.rope_theta;
  a.tie_word_embeddings = c.tie_word_embeddings ? 1 : 0;
  a.qkv_bias = c.qkv_bias ? 1 : 0;
  return a;
}

std::vector<std::size_t> expected_sizes(const ModelConfig& c) {
  const std::size_t h = c.hidden_size, hd = c.hidden_size / c.num_heads, q = c.num_heads * hd,
                    kv = c.num_kv_heads * hd, ff = c.intermediate_size, v = c.vocab_size;
  std::vector<std::size_t> out{v * h};
  for (std::uint32_t i = 0; i < c.num_layers; ++i) {
    out.insert(out.end(), {h, q * h, kv * h, kv * h});
    if (c.qkv_bias) out.insert(out.end(), {q, kv, kv});
    out.insert(out.end(), {h * q, h, ff * h, ff * h, h * ff});
  }
  out.push_back(h);
  if (!c.tie_word_embeddings) out.push_back(v * h);
  return out;
}

Error hip_error(const char* what) { return fail(std::string(what) + ": " + llmi_hip_last_error()); }

}  // namespace

std::vector<std::string> expected_tensor_names(const ModelConfig& c) {
  std::vector<std::string> out{"model.embed_tokens.weight"};
  for (std::uint32_t i = 0; i < c.num_layers; ++i) {
    const std::string p = "model.layers." + std::to_string(i) + ".";
    out.push_back(p + "input_layernorm.weight");
    out.push_back(p + "self_attn.q_proj.weight");
    out.push_back(p + "self_attn.k_proj.weight");
    out.push_back(p + "self_attn.v_proj.weight");
    if (c.qkv_bias) {
      out.push_back(p + "self_attn.q_proj.bias");
      out.push_back(p + "self_attn.k_proj.bias");
      out.push_back(p + "self_attn.v_proj.bias");
    }
    out.push_back(p + "self_attn.o_proj.weight");
    out.push_back(p + "post_attention_layernorm.weight");
    out.push_back(p + "mlp.gate_proj.weight");
    out.push_back(p + "mlp.up_proj.weight");
    out.push_back(p + "mlp.down_proj.weight");
  }
  out.push_back("model.norm.weight");
  if (!c.tie_word_embeddings) out.push_back("lm_head.weight");
  return out;
}

std::size_t KVCache::length() const { return dev_ ? llmi_hip_cache_length(dev_.get()) : 0; }
std::size_t KVCache::capacity() const { return dev_ ? llmi_hip_cache_capacity(dev_.get()) : 0; }
void KVCache::reset() {
  if (dev_) llmi_hip_cache_reset(dev_.get());
}

Result<Transformer> Transformer::load(const ModelConfig& cfg, const TensorReader& read, quant::Type weight_type) {
  const int abi_type = weight_type == quant::Type::Q8_0   ? LLMI_TYPE_Q8_0
                       : weight_type == quant::Type::Q4_0 ? LLMI_TYPE_Q4_0
                                                          : LLMI_TYPE_F32;
  if (cfg.num_heads == 0 || cfg.hidden_size % cfg.num_heads != 0) return fail("load: inconsistent head counts");
  try {
    quant::init_for_host_api();
  } catch (const std::exception& e) {
    return fail(e.what());
  }
  const auto names = expected_tensor_names(cfg);
  const auto sizes = expected_sizes(cfg);
  std::vector<std::vector<float>> tensors;
  tensors.reserve(names.size());
  for (std::size_t i = 0; i < names.size(); ++i) {
    auto t = read(names[i]);
    if (!t) return fail(t.error());
    if (t->size() != sizes[i]) return fail("load: tensor " + names[i] + " has the wrong number of values");
    tensors.push_back(std::move(t.value()));
  }
  std::vector<const float*> ptrs;
  for (const auto& t : tensors) ptrs.push_back(t.data());
  const llmi_model_config abi = abi_config(cfg);
  llmi_hip_model* m = nullptr;
  if (llmi_hip_model_create(&abi, ptrs.data(), abi_type, &m) != LLMI_OK)
    return hip_error("load");
  Transformer t;
  t.cfg_ = cfg;
  t.cfg_.head_dim = cfg.hidden_size / cfg.num_heads;
  t.dev_ = std::shared_ptr<llmi_hip_model>(m, [](llmi_hip_model* p) { llmi_hip_model_free(p); });
  return t;
}

std::size_t Transformer::weight_bytes() const { return dev_ ? llmi_hip_model_weight_bytes(dev_.get()) : 0; }

Result<KVCache> Transformer::new_cache(std::size_t max_len) const {
  llmi_hip_cache* c = nullptr;
  if (llmi_hip_model_new_cache(dev_.get(), max_len, &c) != LLMI_OK) return fail(llmi_hip_last_error());
  KVCache cache;
  cache.dev_ = std::shared_ptr<llmi_hip_cache>(c, [](llmi_hip_cache* p) { llmi_hip_cache_free(p); });
  return cache;
}

Result<std::vector<float>> Transformer::forward_cached(const std::vector<TokenId>& tokens, KVCache& cache,
                                                       bool all_positions, ForwardTrace* trace) const {
  const std::size_t T = tokens.size();
  std::vector<float> logits((all_positions ? std::max<std::size_t>(T, 1) : 1) * cfg_.vocab_size);
  std::vector<float> states;
  if (trace != nullptr) states.resize((cfg_.num_layers + 2) * T * cfg_.hidden_size);
  if (llmi_hip_model_forward_cached_trace(dev_.get(), cache.dev_.get(), tokens.data(), T, all_positions ? 1 : 0,
                                          logits.data(), trace != nullptr ? states.data() : nullptr) != LLMI_OK)
    return fail(llmi_hip_last_error());
  if (trace != nullptr) {
    const std::size_t n = T * cfg_.hidden_size;
    trace->states.clear();
    for (std::size_t k = 0; k < cfg_.num_layers + 2; ++k)
      trace->states.emplace_back(states.begin() + static_cast<std::ptrdiff_t>(k * n),
                                 states.begin() + static_cast<std::ptrdiff_t>((k + 1) * n));
  }
  return logits;
}

Result<TokenId> Transformer::forward_sample(const std::vector<TokenId>& tokens, KVCache& cache,
                                            const SamplingConfig& cfg, std::mt19937_64& rng) const {
  const double target = detail::sample_draw(cfg, rng);
  const llmi_hip_sampling c{cfg.temperature, cfg.top_k, cfg.top_p};
  std::int32_t id = 0;
  if (llmi_hip_model_forward_sample(dev_.get(), cache.dev_.get(), tokens.data(), tokens.size(), &c, target, &id) !=
      LLMI_OK)
    return fail(llmi_hip_last_error());
  return static_cast<TokenId>(id);
}

// forward() recomputes the whole sequence (transformer.cpp:78-166) through the
// model's own device cache, which the library reuses across calls; the
// reference's own tests hold it bit-identical to forward_cached on a fresh
// cache (transformer_test.cpp:322-339).
Result<std::vector<float>> Transformer::forward(const std::vector<TokenId>& tokens, bool all_positions,
                                                ForwardTrace* trace) const {
  const std::size_t T = tokens.size();
  std::vector<float> logits((all_positions ? std::max<std::size_t>(T, 1) : 1) * cfg_.vocab_size);
  std::vector<float> states;
  if (trace != nullptr) states.resize((cfg_.num_layers + 2) * T * cfg_.hidden_size);
  if (llmi_hip_model_forward(dev_.get(), tokens.data(), T, all_positions ? 1 : 0, logits.data(),
                             trace != nullptr ? states.data() : nullptr) != LLMI_OK)
    return fail(llmi_hip_last_error());
  if (trace != nullptr) {
    const std::size_t n = T * cfg_.hidden_size;
    trace->states.clear();
    for (std::size_t k = 0; k < cfg_.num_layers + 2; ++k)
      trace->states.emplace_back(states.begin() + static_cast<std::ptrdiff_t>(k * n),
                                 states.begin() + static_cast<std::ptrdiff_t>((k + 1) * n));
  }
  return logits;
}

Result<std::vector<TokenId>> Transformer::generate_greedy_cached(const std::vector<TokenId>& prompt,
                                                                 std::size_t max_new,
                                                                 const std::vector<TokenId>& stop_ids) const {
  std::vector<TokenId> ids(std::max<std::size_t>(max_new, 1));
  std::size_t n = 0;
  if (llmi_hip_model_generate_greedy(dev_.get(), prompt.data(), prompt.size(), max_new, stop_ids.data(),
                                     stop_ids.size(), ids.data(), &n) != LLMI_OK)
    return fail(llmi_hip_last_error());
  ids.resize(n);
  return ids;
}

// generate_greedy (transformer.cpp:168-180) produces the same tokens as the
// cached version (transformer_test.cpp:383-398); it is served by it.
Result<std::vector<TokenId>> Transformer::generate_greedy(std::vector<TokenId> tokens, std::size_t max_new,
                                                          const std::vector<TokenId>& stop_ids) const {
  return generate_greedy_cached(tokens, max_new, stop_ids);
}

std::size_t argmax(const float* x, std::size_t n) { return static_cast<std::size_t>(std::max_element(x, x + n) - x); }

}  // namespace llmi
