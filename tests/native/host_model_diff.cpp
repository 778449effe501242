// Differential test of the C++ host layer's model API (llmi::Transformer and
// llmi::KVCache of libllmi_gpu.so: load, forward, forward_cached,
// generate_greedy_cached, forward_sample -- all on the GPU) against the CPU
// oracle's restatement of src/model/transformer.cpp:22-327.  For every model
// of a table (both architectures, tied and untied heads, F32 / Q8_0 / Q4_0
// weights, head sizes 4 and 64 so that both the generic and the fused
// one-token kernels run) a scripted session -- a prefill, single-token steps,
// a fresh-sequence forward, greedy generation and a sampled serving loop --
// must give the oracle's logits and ids bit for bit, and the failures the
// reference reports must come back as Result errors with its messages.
#include <map>
#include <random>
#include <stdexcept>

#include "check.hpp"
#include "llmi/model/transformer.hpp"
#include "llmi_hip.h"

extern "C" {
void* oracle_model_create(const llmi_model_config* cfg, const float* const* tensors, int type);
void oracle_model_free(void* m);
int oracle_model_new_cache(void* m, std::size_t max_len);
int oracle_model_forward_cached(void* m, const std::int32_t* tokens, std::size_t n, int all_positions, float* logits);
int oracle_generate_greedy_cached(void* m, const std::int32_t* prompt, std::size_t n, std::size_t max_new,
                                  std::int32_t* ids, float* margins);
std::size_t oracle_sample_target(const float* logits, std::size_t n, float temperature, std::size_t top_k, float top_p,
                                 double target);
}

using namespace llmi;

namespace {

struct ModelCase {
  const char* what;
  Arch arch;
  bool tied;
  quant::Type type;
  std::uint32_t hidden, heads, kv_heads, inter, layers, vocab, ctx;
};

const ModelCase kModels[] = {
    {"llama tied q8 hd4", Arch::Llama, true, quant::Type::Q8_0, 16, 4, 2, 24, 2, 32, 64},
    {"qwen untied q4 hd4", Arch::Qwen2, false, quant::Type::Q4_0, 16, 4, 2, 24, 2, 32, 64},
    {"qwen tied f32 hd4", Arch::Qwen2, true, quant::Type::F32, 16, 4, 1, 40, 2, 40, 64},
    {"llama untied q4 hd64", Arch::Llama, false, quant::Type::Q4_0, 192, 3, 1, 320, 2, 96, 128},
    {"qwen tied q8 hd64 gqa7", Arch::Qwen2, true, quant::Type::Q8_0, 448, 7, 1, 512, 2, 64, 128},
};

int abi_type(quant::Type t) {
  return t == quant::Type::Q8_0 ? LLMI_TYPE_Q8_0 : t == quant::Type::Q4_0 ? LLMI_TYPE_Q4_0 : LLMI_TYPE_F32;
}

ModelConfig config_of(const ModelCase& m) {
  ModelConfig c;
  c.arch = m.arch;
  c.vocab_size = m.vocab;
  c.hidden_size = m.hidden;
  c.intermediate_size = m.inter;
  c.num_layers = m.layers;
  c.num_heads = m.heads;
  c.num_kv_heads = m.kv_heads;
  c.head_dim = m.hidden / m.heads;
  c.max_position_embeddings = m.ctx;
  c.rms_norm_eps = m.arch == Arch::Qwen2 ? 1e-6 : 1e-5;
  c.rope_theta = m.arch == Arch::Qwen2 ? 1e6 : 1e5;
  c.tie_word_embeddings = m.tied;
  c.qkv_bias = m.arch == Arch::Qwen2;
  return c;
}

llmi_model_config abi_of(const ModelConfig& c) {
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

// Tensor sizes in expected_tensor_names() order; norms ~ 1, everything else
// ~ N(0, 0.1).
std::vector<std::vector<float>> make_tensors(const ModelConfig& c, const std::vector<std::string>& names,
                                             std::uint64_t seed) {
  const std::size_t h = c.hidden_size, hd = h / c.num_heads, q = c.num_heads * hd, kv = c.num_kv_heads * hd,
                    f = c.intermediate_size, v = c.vocab_size;
  std::vector<std::vector<float>> t;
  for (std::size_t i = 0; i < names.size(); ++i) {
    const std::string& n = names[i];
    std::size_t count = f * h;  // gate / up / down
    if (n == "model.embed_tokens.weight" || n == "lm_head.weight") count = v * h;
    else if (n.find("norm") != std::string::npos) count = h;
    else if (n.find("q_proj.weight") != std::string::npos || n.find("o_proj") != std::string::npos) count = q * h;
    else if (n.find("_proj.weight") != std::string::npos && n.find("self_attn") != std::string::npos) count = kv * h;
    else if (n.find("q_proj.bias") != std::string::npos) count = q;
    else if (n.find(".bias") != std::string::npos) count = kv;
    const bool norm = n.find("norm") != std::string::npos;
    t.push_back(check::normal(seed + 31 * i, count, norm ? 1.0 : 0.0, norm ? 0.05 : 0.1));
  }
  return t;
}

bool same(const std::vector<float>& a, const std::vector<float>& b) {
  return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0;
}

// The oracle model of the same weights, with helpers for one session.
struct Oracle {
  void* m = nullptr;
  std::size_t V = 0;
  ~Oracle() { oracle_model_free(m); }
  std::vector<float> step(const std::vector<TokenId>& ids, bool all) const {
    std::vector<float> out((all ? ids.size() : 1) * V);
    if (oracle_model_forward_cached(m, ids.data(), ids.size(), all ? 1 : 0, out.data()) != 0)
      throw std::runtime_error("oracle forward failed");
    return out;
  }
};

}  // namespace

TEST(ModelDiff, ScriptedSessionsEqualTheOracle) {
  std::uint64_t seed = 500;
  for (const ModelCase& mc : kModels) {
    const std::string tag = mc.what;
    const ModelConfig cfg = config_of(mc);
    const auto names = expected_tensor_names(cfg);
    const auto tensors = make_tensors(cfg, names, seed += 1000);
    std::map<std::string, std::size_t> index;
    for (std::size_t i = 0; i < names.size(); ++i) index[names[i]] = i;
    auto loaded = Transformer::load(
        cfg, [&](const std::string& n) -> Result<std::vector<float>> { return tensors[index.at(n)]; }, mc.type);
    if (!loaded) {
      check::report(__FILE__, __LINE__, tag + ": load: " + loaded.error());
      continue;
    }
    const Transformer& tf = *loaded;
    Oracle o;
    std::vector<const float*> ptrs;
    for (const auto& t : tensors) ptrs.push_back(t.data());
    const llmi_model_config abi = abi_of(cfg);
    o.m = oracle_model_create(&abi, ptrs.data(), abi_type(mc.type));
    o.V = cfg.vocab_size;

    // 1. A prefill of 9 tokens (all positions), then 6 single-token steps.
    std::vector<TokenId> seq;
    for (std::size_t i = 0; i < 15; ++i) seq.push_back(static_cast<TokenId>(check::splitmix(seed, i) % cfg.vocab_size));
    const std::vector<TokenId> prompt(seq.begin(), seq.begin() + 9);
    ASSERT_TRUE(oracle_model_new_cache(o.m, seq.size()) == 0);
    auto cache = tf.new_cache(seq.size());
    ASSERT_TRUE(cache.ok());
    auto pre = tf.forward_cached(prompt, *cache, true);
    ASSERT_TRUE(pre.ok());
    if (!same(*pre, o.step(prompt, true))) check::report(__FILE__, __LINE__, tag + ": prefill logits");
    for (std::size_t t = 9; t < seq.size(); ++t) {
      auto got = tf.forward_cached({seq[t]}, *cache);
      ASSERT_TRUE(got.ok());
      if (!same(*got, o.step({seq[t]}, false)))
        check::report(__FILE__, __LINE__, tag + ": step " + std::to_string(t));
    }
    EXPECT_EQ(cache->length(), seq.size());
    // The cache is full now: one more token is the reference's error.
    auto over = tf.forward_cached({seq[0]}, *cache);
    EXPECT_TRUE(!over.ok() && over.error().find("cache is full") != std::string::npos);

    // 2. forward() of the whole sequence equals a fresh oracle prefill.
    ASSERT_TRUE(oracle_model_new_cache(o.m, seq.size()) == 0);
    auto fwd = tf.forward(seq, true);
    ASSERT_TRUE(fwd.ok());
    if (!same(*fwd, o.step(seq, true))) check::report(__FILE__, __LINE__, tag + ": forward all positions");

    // 3. Greedy generation: the oracle's ids.
    const std::size_t max_new = 20;
    auto ids = tf.generate_greedy_cached(prompt, max_new, {});
    ASSERT_TRUE(ids.ok());
    std::vector<std::int32_t> want(max_new);
    ASSERT_TRUE(oracle_generate_greedy_cached(o.m, prompt.data(), prompt.size(), max_new, want.data(), nullptr) == 0);
    EXPECT_TRUE(*ids == std::vector<TokenId>(want.begin(), want.end()));

    // 4. A sampled serving loop through forward_sample: the oracle's logits,
    //    the oracle's sample() of them with the draws a replica generator
    //    takes, fed back each step.
    const SamplingConfig sc{0.9F, 10, 0.95F};
    std::mt19937_64 rng(seed), replica(seed);
    std::uniform_real_distribution<double> u(0.0, 1.0);
    auto c2 = tf.new_cache(prompt.size() + 12);
    ASSERT_TRUE(c2.ok());
    ASSERT_TRUE(oracle_model_new_cache(o.m, prompt.size() + 12) == 0);
    std::vector<TokenId> feed = prompt;
    for (int step = 0; step < 12; ++step) {
      auto got = tf.forward_sample(feed, *c2, sc, rng);
      ASSERT_TRUE(got.ok());
      const std::vector<float> logits = o.step(feed, false);
      const auto expect = static_cast<TokenId>(
          oracle_sample_target(logits.data(), o.V, sc.temperature, sc.top_k, sc.top_p, u(replica)));
      if (*got != expect) check::report(__FILE__, __LINE__, tag + ": sampled step " + std::to_string(step));
      feed = {*got};
    }
    EXPECT_TRUE(rng == replica);

    // 5. What the reference reports as errors.
    auto bad_id = tf.forward({static_cast<TokenId>(cfg.vocab_size)});
    EXPECT_TRUE(!bad_id.ok() && bad_id.error().find("out of range") != std::string::npos);
    auto empty = tf.forward({});
    EXPECT_TRUE(!empty.ok() && empty.error().find("no tokens") != std::string::npos);
    auto too_long = tf.generate_greedy_cached(std::vector<TokenId>(cfg.max_position_embeddings - 2, 1), 8, {});
    EXPECT_TRUE(!too_long.ok() && too_long.error().find("cache is full") != std::string::npos);
  }
}
