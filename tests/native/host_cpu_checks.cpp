// The host layer's paths that need no GPU, for sanitizer builds on the CPU
// (tests/test_sanitizers.py compiles this with host/src/*.cpp under
// -fsanitize=address,undefined): the checkpoint's tensor names, Result<T>,
// the load's own validation, the sampling draw rule, and clean failures --
// error Results and the exceptions the reference's callers expect -- when no
// device is present (skipped where one is).
#include <optional>
#include <random>
#include <stdexcept>

#include "check.hpp"
#include "llmi/model/quant.hpp"
#include "llmi/model/sampling.hpp"
#include "llmi/model/transformer.hpp"
#include "llmi/model/weight.hpp"
#include "llmi_hip.h"

using namespace llmi;

namespace {

ModelConfig small(Arch arch, bool tied) {
  ModelConfig c;
  c.arch = arch;
  c.vocab_size = 40;
  c.hidden_size = 16;
  c.intermediate_size = 24;
  c.num_layers = 3;
  c.num_heads = 4;
  c.num_kv_heads = 2;
  c.head_dim = 4;
  c.max_position_embeddings = 32;
  c.rms_norm_eps = 1e-6;
  c.rope_theta = 1e4;
  c.tie_word_embeddings = tied;
  c.qkv_bias = arch == Arch::Qwen2;
  return c;
}

bool device_present() { return llmi_hip_init(0) == LLMI_OK; }

}  // namespace

TEST(HostCpu, TensorNamesFollowTheCheckpointLayout) {
  for (const Arch arch : {Arch::Llama, Arch::Qwen2})
    for (const bool tied : {true, false}) {
      const ModelConfig c = small(arch, tied);
      const auto names = expected_tensor_names(c);
      const std::size_t per_layer = arch == Arch::Qwen2 ? 12 : 9;
      EXPECT_EQ(names.size(), 2 + per_layer * c.num_layers + (tied ? 0 : 1));
      EXPECT_TRUE(names.front() == "model.embed_tokens.weight");
      EXPECT_TRUE(names[1] == "model.layers.0.input_layernorm.weight");
      EXPECT_TRUE(names[per_layer] == "model.layers.0.mlp.down_proj.weight");
      EXPECT_TRUE(names[per_layer + 1] == "model.layers.1.input_layernorm.weight");
      EXPECT_TRUE((arch == Arch::Qwen2) == (names[5] == "model.layers.0.self_attn.q_proj.bias"));
      EXPECT_TRUE(names.back() == (tied ? "model.norm.weight" : "lm_head.weight"));
    }
}

TEST(HostCpu, ResultHoldsAValueOrAnError) {
  Result<std::vector<int>> ok = std::vector<int>{1, 2, 3};
  EXPECT_TRUE(ok.ok() && static_cast<bool>(ok) && ok->size() == 3 && ok.error().empty());
  Result<std::vector<int>> moved = std::move(ok);
  EXPECT_TRUE(moved.ok() && (*moved)[2] == 3);
  Result<std::vector<int>> bad = fail("nope");
  EXPECT_TRUE(!bad.ok() && bad.error() == "nope");
  bool threw = false;
  try {
    (void)bad.value();
  } catch (const std::bad_optional_access&) {
    threw = true;
  }
  EXPECT_TRUE(threw);
}

TEST(HostCpu, LoadRejectsInconsistentHeadsBeforeTouchingTheDevice) {
  ModelConfig c = small(Arch::Llama, true);
  c.num_heads = 0;
  const auto r0 = Transformer::load(c, [](const std::string&) -> Result<std::vector<float>> { return fail("unread"); },
                                    quant::Type::Q8_0);
  EXPECT_TRUE(!r0.ok() && r0.error() == "load: inconsistent head counts");
  c.num_heads = 5;  // 16 % 5 != 0
  const auto r1 = Transformer::load(c, [](const std::string&) -> Result<std::vector<float>> { return fail("unread"); },
                                    quant::Type::Q8_0);
  EXPECT_TRUE(!r1.ok() && r1.error() == "load: inconsistent head counts");
}

TEST(HostCpu, SamplingDrawsOneUniformPerCallAboveZeroTemperature) {
  std::mt19937_64 rng(5), replica(5);
  EXPECT_TRUE(detail::sample_draw(SamplingConfig{0.0F, 0, 1.0F}, rng) == 0.0);
  EXPECT_TRUE(detail::sample_draw(SamplingConfig{-2.0F, 3, 0.5F}, rng) == 0.0);
  EXPECT_TRUE(rng == replica);
  std::uniform_real_distribution<double> u(0.0, 1.0);
  for (int i = 0; i < 5; ++i) {
    const double d = detail::sample_draw(SamplingConfig{0.7F, 40, 0.9F}, rng);
    EXPECT_TRUE(d == u(replica));
  }
  EXPECT_TRUE(rng == replica);
}

TEST(HostCpu, WithoutADeviceCallsFailCleanly) {
  if (device_present()) {
    std::printf("  (a device is present: skipped)\n");
    return;
  }
  const ModelConfig c = small(Arch::Qwen2, false);
  std::size_t reads = 0;
  const auto r = Transformer::load(
      c, [&](const std::string&) -> Result<std::vector<float>> { ++reads; return std::vector<float>(4, 0.0F); },
      quant::Type::Q4_0);
  EXPECT_TRUE(!r.ok() && r.error().find("llmi_hip_init") != std::string::npos);
  EXPECT_EQ(reads, std::size_t{0});
  const std::vector<float> w(64, 0.5F), logits(8, 1.0F);
  bool threw = false;
  try {
    (void)quant::quantize(w.data(), 2, 32, quant::Type::Q8_0);
  } catch (const std::runtime_error& e) {
    threw = std::string(e.what()).find("llmi_hip_init") != std::string::npos;
  }
  EXPECT_TRUE(threw);
  threw = false;
  std::mt19937_64 rng(1);
  try {
    (void)sample(logits.data(), logits.size(), SamplingConfig{}, rng);
  } catch (const std::runtime_error&) {
    threw = true;
  }
  EXPECT_TRUE(threw);
  threw = false;
  const Weight empty;
  std::vector<float> y(2);
  try {
    empty.matmul(logits.data(), 1, 8, 2, nullptr, y.data());
  } catch (const std::logic_error&) {
    threw = true;
  }
  EXPECT_TRUE(threw);
  EXPECT_TRUE(quant::type_name(quant::Type::Q4_0) == "q4_0" && quant::type_name(quant::Type::F32) == "f32");
}
