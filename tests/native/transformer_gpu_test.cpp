// The reference's tests/transformer_test.cpp model and KV-cache cases, run
// against the GPU drop-in (llmi::Transformer of libllmi_gpu.so) on the
// reference's 2-layer test architecture, plus bit-exact logits against the
// CPU oracle (oracle/liboracle.so).
#include <map>
#include <random>

#include "check.hpp"
#include "llmi/model/transformer.hpp"
#include "llmi_hip.h"

extern "C" {
void* oracle_model_create(const llmi_model_config* cfg, const float* const* tensors, int type);
void oracle_model_free(void* m);
int oracle_model_new_cache(void* m, std::size_t max_len);
int oracle_model_forward_cached(void* m, const std::int32_t* tokens, std::size_t n, int all_positions, float* logits);
}

using namespace llmi;

namespace {

ModelConfig tiny_config(Arch arch, bool tied) {
  ModelConfig c;
  c.arch = arch;
  c.vocab_size = 32;
  c.hidden_size = 16;
  c.intermediate_size = 24;
  c.num_layers = 2;
  c.num_heads = 4;
  c.num_kv_heads = 2;
  c.head_dim = 4;
  c.max_position_embeddings = 64;
  c.rms_norm_eps = 1e-6;
  c.rope_theta = 10000.0;
  c.tie_word_embeddings = tied;
  c.qkv_bias = arch == Arch::Qwen2;
  c.eos_token_ids = {3};
  return c;
}

// Random weights like the reference's make_tiny (transformer_test.cpp:162-197):
// N(0, 0.3), norm weights 1 + 0.1 * N(0, 0.3).
struct Tiny {
  ModelConfig cfg;
  std::vector<std::string> names;
  std::vector<std::vector<float>> tensors;
};

Tiny make_tiny(Arch arch, bool tied, unsigned seed) {
  Tiny t;
  t.cfg = tiny_config(arch, tied);
  t.names = expected_tensor_names(t.cfg);
  const std::size_t h = 16, q = 16, kv = 8, ff = 24, v = 32;
  for (std::size_t i = 0; i < t.names.size(); ++i) {
    const std::string& n = t.names[i];
    std::size_t count = 0;
    if (n.find("embed") != std::string::npos || n.find("lm_head") != std::string::npos) count = v * h;
    else if (n.find("norm") != std::string::npos) count = h;
    else if (n.find("q_proj.weight") != std::string::npos) count = q * h;
    else if (n.find("k_proj.weight") != std::string::npos || n.find("v_proj.weight") != std::string::npos) count = kv * h;
    else if (n.find("q_proj.bias") != std::string::npos) count = q;
    else if (n.find("bias") != std::string::npos) count = kv;
    else if (n.find("o_proj") != std::string::npos) count = h * q;
    else count = ff * h;
    const bool norm = n.find("norm") != std::string::npos;
    t.tensors.push_back(check::normal(seed * 1000 + i, count, norm ? 1.0 : 0.0, norm ? 0.03 : 0.3));
  }
  return t;
}

Transformer load(const Tiny& t, quant::Type type) {
  std::map<std::string, const std::vector<float>*> by_name;
  for (std::size_t i = 0; i < t.names.size(); ++i) by_name[t.names[i]] = &t.tensors[i];
  auto r = Transformer::load(t.cfg, [&](const std::string& n) -> Result<std::vector<float>> { return *by_name.at(n); },
                             type);
  if (!r) throw std::runtime_error(r.error());
  return std::move(r.value());
}

llmi_model_config abi(const ModelConfig& c) {
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
  a.tie_word_embeddings = c.tie_word_embeddings;
  a.qkv_bias = c.qkv_bias;
  return a;
}

bool same(const std::vector<float>& a, const std::vector<float>& b) {
  return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * 4) == 0;
}

}  // namespace

TEST(Transformer, IsCausal) {
  for (Arch arch : {Arch::Llama, Arch::Qwen2}) {
    auto tiny = make_tiny(arch, true, 3);
    auto tf = load(tiny, quant::Type::Q8_0);
    const std::vector<TokenId> a = {5, 9, 1, 30, 7};
    std::vector<TokenId> b = a;
    b[3] = 2;
    auto la = tf.forward(a, true);
    auto lb = tf.forward(b, true);
    ASSERT_TRUE(la && lb);
    for (std::size_t i = 0; i < 3 * 32; ++i) EXPECT_EQ((*la)[i], (*lb)[i]);
    bool differs = false;
    for (std::size_t i = 3 * 32; i < 5 * 32; ++i) differs = differs || (*la)[i] != (*lb)[i];
    EXPECT_TRUE(differs);
  }
}

TEST(Transformer, LastPositionMatchesAllPositions) {
  auto tiny = make_tiny(Arch::Llama, false, 4);
  auto tf = load(tiny, quant::Type::Q4_0);
  auto all = tf.forward({1, 2, 3, 4}, true);
  auto last = tf.forward({1, 2, 3, 4}, false);
  ASSERT_TRUE(all && last);
  ASSERT_TRUE(last->size() == 32U);
  for (std::size_t i = 0; i < 32; ++i) EXPECT_EQ((*last)[i], (*all)[3 * 32 + i]);
}

TEST(Transformer, TracesEveryLayer) {
  auto tiny = make_tiny(Arch::Qwen2, false, 5);
  auto tf = load(tiny, quant::Type::Q8_0);
  ForwardTrace trace;
  ASSERT_TRUE(tf.forward({7, 8, 9}, false, &trace));
  ASSERT_TRUE(trace.states.size() == 2U + 2U);
  for (const auto& s : trace.states) EXPECT_EQ(s.size(), 3U * 16U);
}

TEST(Transformer, RejectsBadInput) {
  auto tiny = make_tiny(Arch::Llama, true, 6);
  auto tf = load(tiny, quant::Type::Q8_0);
  EXPECT_FALSE(tf.forward({}));
  EXPECT_FALSE(tf.forward({32}));
  EXPECT_FALSE(tf.forward({-1}));
  EXPECT_FALSE(tf.forward(std::vector<TokenId>(65, 1)));
}

TEST(Transformer, QuantizedWeightBytes) {
  auto tiny = make_tiny(Arch::Llama, true, 12);
  auto q8 = load(tiny, quant::Type::Q8_0);
  auto q4 = load(tiny, quant::Type::Q4_0);
  EXPECT_TRUE(q8.weight_bytes() > q4.weight_bytes());
  EXPECT_FALSE(Transformer::load(tiny.cfg, [](const std::string&) -> Result<std::vector<float>> { return fail("x"); },
                                 quant::Type::F32));
}

TEST(Transformer, LogitsAreBitExactAgainstTheOracle) {
  for (Arch arch : {Arch::Llama, Arch::Qwen2})
    for (bool tied : {true, false})
      for (quant::Type type : {quant::Type::Q8_0, quant::Type::Q4_0}) {
        auto tiny = make_tiny(arch, tied, 21);
        auto tf = load(tiny, type);
        std::vector<const float*> ptrs;
        for (const auto& t : tiny.tensors) ptrs.push_back(t.data());
        const llmi_model_config c = abi(tiny.cfg);
        void* o = oracle_model_create(&c, ptrs.data(), type == quant::Type::Q8_0 ? 1 : 2);
        const std::vector<TokenId> ids = {5, 9, 1, 30, 7, 2, 2, 31};
        ASSERT_TRUE(oracle_model_new_cache(o, ids.size()) == 0);
        std::vector<float> want(ids.size() * 32);
        ASSERT_TRUE(oracle_model_forward_cached(o, ids.data(), ids.size(), 1, want.data()) == 0);
        oracle_model_free(o);
        auto got = tf.forward(ids, true);
        ASSERT_TRUE(got);
        EXPECT_TRUE(same(*got, want));
      }
}

TEST(KVCache, PrefillInOneCallMatchesForward) {
  for (Arch arch : {Arch::Llama, Arch::Qwen2}) {
    auto tiny = make_tiny(arch, false, 10);
    auto tf = load(tiny, quant::Type::Q8_0);
    const std::vector<TokenId> ids = {5, 9, 1, 30, 7};
    auto baseline = tf.forward(ids, true);
    auto cache = tf.new_cache(ids.size());
    ASSERT_TRUE(cache);
    auto cached = tf.forward_cached(ids, *cache, true);
    ASSERT_TRUE(baseline && cached);
    EXPECT_TRUE(same(*baseline, *cached));
    EXPECT_EQ(cache->length(), ids.size());
  }
}

TEST(KVCache, OneTokenAtATimeMatchesForward) {
  for (Arch arch : {Arch::Llama, Arch::Qwen2}) {
    auto tiny = make_tiny(arch, true, 11);
    auto tf = load(tiny, quant::Type::Q4_0);
    const std::vector<TokenId> ids = {2, 17, 4, 9, 21, 0, 13};
    auto cache = tf.new_cache(ids.size());
    ASSERT_TRUE(cache);
    for (std::size_t t = 0; t < ids.size(); ++t) {
      auto baseline = tf.forward(std::vector<TokenId>(ids.begin(), ids.begin() + static_cast<long>(t) + 1));
      auto cached = tf.forward_cached({ids[t]}, *cache);
      ASSERT_TRUE(baseline && cached);
      EXPECT_TRUE(same(*baseline, *cached));
    }
    EXPECT_EQ(cache->length(), ids.size());
  }
}

TEST(KVCache, PrefillThenStepsMatchesForward) {
  auto tiny = make_tiny(Arch::Qwen2, false, 12);
  auto tf = load(tiny, quant::Type::Q8_0);
  const std::vector<TokenId> prompt = {3, 8, 14};
  auto cache = tf.new_cache(6);
  ASSERT_TRUE(cache);
  ASSERT_TRUE(tf.forward_cached(prompt, *cache));
  std::vector<TokenId> grown = prompt;
  for (const TokenId next : {6, 19, 2}) {
    grown.push_back(next);
    auto baseline = tf.forward(grown);
    auto cached = tf.forward_cached({next}, *cache);
    ASSERT_TRUE(baseline && cached);
    EXPECT_TRUE(same(*baseline, *cached));
  }
}

TEST(KVCache, GenerateGreedyCachedMatchesGenerateGreedyAndStops) {
  for (Arch arch : {Arch::Llama, Arch::Qwen2}) {
    auto tiny = make_tiny(arch, true, 13);
    auto tf = load(tiny, quant::Type::Q8_0);
    auto cached = tf.generate_greedy_cached({1, 2, 3}, 12, {});
    ASSERT_TRUE(cached);
    EXPECT_EQ(cached->size(), 12U);
    // The same ids one forward() at a time (transformer.cpp:168-180).
    std::vector<TokenId> toks = {1, 2, 3};
    for (std::size_t step = 0; step < 12; ++step) {
      auto l = tf.forward(toks);
      ASSERT_TRUE(l);
      const auto next = static_cast<TokenId>(argmax(l->data(), l->size()));
      EXPECT_EQ(next, (*cached)[step]);
      toks.push_back(next);
    }
    const TokenId stop = (*cached)[2];
    auto stopped = tf.generate_greedy_cached({1, 2, 3}, 12, {stop});
    ASSERT_TRUE(stopped);
    std::size_t first = 0;
    while ((*cached)[first] != stop) ++first;
    EXPECT_EQ(stopped->size(), first + 1);
  }
}

TEST(KVCache, RejectsOverfullOrUnknownCache) {
  auto tiny = make_tiny(Arch::Llama, true, 14);
  auto tf = load(tiny, quant::Type::Q8_0);
  auto other = load(make_tiny(Arch::Llama, true, 15), quant::Type::Q8_0);
  auto cache = tf.new_cache(3);
  ASSERT_TRUE(cache);
  ASSERT_TRUE(tf.forward_cached({1, 2, 3}, *cache));
  EXPECT_FALSE(tf.forward_cached({4}, *cache));
  EXPECT_FALSE(other.forward_cached({4}, *cache));
  cache->reset();
  EXPECT_TRUE(tf.forward_cached({1, 2, 3}, *cache));
  EXPECT_FALSE(tf.new_cache(0));
}

TEST(Transformer, GreedyIsDeterministic) {
  auto tiny = make_tiny(Arch::Llama, true, 7);
  auto tf = load(tiny, quant::Type::Q4_0);
  auto a = tf.generate_greedy({1, 2}, 10, {});
  auto b = tf.generate_greedy({1, 2}, 10, {});
  ASSERT_TRUE(a && b);
  EXPECT_EQ(a->size(), 10U);
  EXPECT_TRUE(a.value() == b.value());
  auto stopped = tf.generate_greedy({1, 2}, 10, {(*a)[0]});
  ASSERT_TRUE(stopped);
  EXPECT_EQ(stopped->size(), 1U);
}

// The serving loop (server.cpp:109-195): forward_cached, sample(), feed the
// token back -- and forward_sample doing both on the device, with the same
// generator: the same tokens and the same generator state after.
TEST(Transformer, ForwardSampleMatchesForwardCachedThenSample) {
  for (quant::Type type : {quant::Type::Q8_0, quant::Type::Q4_0}) {
    auto tiny = make_tiny(Arch::Qwen2, true, 21);
    auto tf = load(tiny, type);
    const SamplingConfig cfg{0.9F, 8, 0.95F};
    auto c1 = tf.new_cache(40);
    auto c2 = tf.new_cache(40);
    ASSERT_TRUE(c1 && c2);
    std::mt19937_64 r1(99), r2(99);
    std::vector<TokenId> in = {1, 2, 3, 4};
    auto logits = tf.forward_cached(in, *c1);
    ASSERT_TRUE(logits);
    TokenId want = sample(logits->data(), logits->size(), cfg, r1);
    auto got = tf.forward_sample(in, *c2, cfg, r2);
    ASSERT_TRUE(got);
    EXPECT_EQ(*got, want);
    for (int step = 0; step < 20; ++step) {
      logits = tf.forward_cached({want}, *c1);
      ASSERT_TRUE(logits);
      want = sample(logits->data(), logits->size(), cfg, r1);
      got = tf.forward_sample({*got}, *c2, cfg, r2);
      ASSERT_TRUE(got);
      EXPECT_EQ(*got, want);
    }
    EXPECT_TRUE(r1 == r2);
    EXPECT_EQ(c1->length(), c2->length());
  }
}
