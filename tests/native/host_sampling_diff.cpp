// Differential test of the C++ host layer's sampling API (llmi::sample and
// llmi::sampling_probabilities of libllmi_gpu.so, computed on the GPU)
// against the CPU oracle's restatement of src/model/sampling.cpp:11-77: a
// table of vocabularies (sizes, spreads, ties, masked entries) crossed with a
// table of SamplingConfigs; for each pair the filtered distribution must be
// the oracle's bit for bit, and a seeded run of sample() must give the
// oracle's token for every draw while taking exactly the draws the reference
// takes from the generator.
#include <cmath>
#include <cstring>
#include <limits>
#include <random>
#include <stdexcept>

#include "check.hpp"
#include "llmi/model/sampling.hpp"

extern "C" {
void oracle_sampling_probabilities(const float* logits, std::size_t n, float temperature, std::size_t top_k,
                                   float top_p, float* out);
std::size_t oracle_sample_target(const float* logits, std::size_t n, float temperature, std::size_t top_k, float top_p,
                                 double target);
}

namespace {

struct Vocab {
  const char* what;
  std::vector<float> logits;
};

std::vector<Vocab> vocabularies() {
  std::vector<Vocab> v;
  v.push_back({"one entry", {0.25F}});
  v.push_back({"small, spread 2", check::normal(1, 7, 0.0, 2.0)});
  std::vector<float> ties(300, 1.5F);
  for (std::size_t i = 0; i < ties.size(); i += 3) ties[i] = -0.5F;
  v.push_back({"many ties", ties});
  std::vector<float> masked = check::normal(2, 2000, 0.0, 1.0);
  for (std::size_t i = 0; i < masked.size(); ++i)
    if (i % 5 != 1) masked[i] = -std::numeric_limits<float>::infinity();
  v.push_back({"mostly masked (-inf)", masked});
  std::vector<float> peaked = check::normal(3, 49152, 0.0, 0.5);
  peaked[40000] = 30.0F;
  v.push_back({"SmolLM2 vocabulary, one dominant", peaked});
  v.push_back({"Qwen2.5 vocabulary, spread 3", check::normal(4, 151936, 0.0, 3.0)});
  return v;
}

const llmi::SamplingConfig kConfigs[] = {
    {1.0F, 0, 1.0F},   {0.7F, 0, 1.0F},  {1.3F, 5, 1.0F},  {0.8F, 40, 0.9F}, {1.0F, 0, 0.5F},
    {2.0F, 1, 1.0F},   {0.9F, 0, 0.0F},  {0.0F, 0, 1.0F},  {-1.0F, 3, 0.3F},
};

std::string name(const Vocab& v, const llmi::SamplingConfig& c) {
  return std::string(v.what) + " / t=" + std::to_string(c.temperature) + " k=" + std::to_string(c.top_k) +
         " p=" + std::to_string(c.top_p);
}

}  // namespace

TEST(SamplingDiff, DistributionsAndSeededDrawsEqualTheOracle) {
  for (const Vocab& v : vocabularies()) {
    const std::size_t n = v.logits.size();
    for (const llmi::SamplingConfig& c : kConfigs) {
      if (c.temperature > 0.0F) {
        std::vector<float> want(n);
        oracle_sampling_probabilities(v.logits.data(), n, c.temperature, c.top_k, c.top_p, want.data());
        const std::vector<float> got = llmi::sampling_probabilities(v.logits.data(), n, c);
        if (got.size() != n || std::memcmp(got.data(), want.data(), n * sizeof(float)) != 0)
          check::report(__FILE__, __LINE__, "probabilities: " + name(v, c));
      }
      // The generator is shared by the reference's loop; a replica advanced
      // by the reference's rule (one uniform double per call when
      // temperature > 0) must stay in step with it.
      std::mt19937_64 rng(7 + n), replica(7 + n);
      std::uniform_real_distribution<double> u(0.0, 1.0);
      for (int call = 0; call < 12; ++call) {
        const double target = c.temperature > 0.0F ? u(replica) : 0.0;
        const llmi::TokenId got = llmi::sample(v.logits.data(), n, c, rng);
        const std::size_t want = oracle_sample_target(v.logits.data(), n, c.temperature, c.top_k, c.top_p, target);
        if (static_cast<std::size_t>(got) != want)
          check::report(__FILE__, __LINE__, "sample call " + std::to_string(call) + ": " + name(v, c));
      }
      EXPECT_TRUE(rng == replica);
    }
  }
}

// Where the reference's result is undefined (n == 0, NaN, +inf after the
// temperature) the host layer throws std::invalid_argument.
TEST(SamplingDiff, UndefinedInputsAreRejected) {
  const float inf = std::numeric_limits<float>::infinity();
  const std::vector<std::vector<float>> bad = {{0.5F, std::nanf("")}, {1.0F, inf}, {3e38F, 1.0F}};
  llmi::SamplingConfig cold{1e-3F, 0, 1.0F};  // 3e38 / 1e-3 overflows to +inf
  for (std::size_t i = 0; i < bad.size(); ++i) {
    std::mt19937_64 rng(11);
    bool threw = false;
    try {
      (void)llmi::sample(bad[i].data(), bad[i].size(), i == 2 ? cold : llmi::SamplingConfig{}, rng);
    } catch (const std::invalid_argument&) {
      threw = true;
    }
    EXPECT_TRUE(threw);
  }
  bool threw = false;
  try {
    (void)llmi::sampling_probabilities(bad[0].data(), 0, llmi::SamplingConfig{});
  } catch (const std::invalid_argument&) {
    threw = true;
  }
  EXPECT_TRUE(threw);
}
