// The reference's tests/sampling_test.cpp cases run against the GPU drop-in
// (llmi::sample / llmi::sampling_probabilities of libllmi_gpu.so), plus whole
// seeded sample() sequences and filtered distributions bit for bit against
// the CPU oracle (oracle/liboracle.so).
#include <algorithm>
#include <numeric>
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

using namespace llmi;

namespace {
double sum(const std::vector<float>& v) { return std::accumulate(v.begin(), v.end(), 0.0); }
}  // namespace

TEST(Sampling, TemperatureZeroIsGreedy) {
  const float logits[] = {1, 5, 3, 5, 2};
  SamplingConfig cfg;
  cfg.temperature = 0.0F;
  std::mt19937_64 rng(1);
  for (int i = 0; i < 5; ++i) EXPECT_EQ(sample(logits, 5, cfg, rng), 1);
  EXPECT_TRUE(rng == std::mt19937_64(1));  // nothing drawn
}

TEST(Sampling, ProbabilitiesSumToOneAndFollowSoftmax) {
  const float logits[] = {1, 2, 3, 4};
  auto p = sampling_probabilities(logits, 4, SamplingConfig{});
  EXPECT_NEAR(sum(p), 1.0, 1e-6);
  for (std::size_t i = 0; i + 1 < 4; ++i) EXPECT_TRUE(p[i] < p[i + 1]);
  double denom = 0;
  for (float x : logits) denom += std::exp(static_cast<double>(x));
  for (std::size_t i = 0; i < 4; ++i) EXPECT_NEAR(p[i], std::exp(static_cast<double>(logits[i])) / denom, 1e-5);
}

TEST(Sampling, TemperatureFlattensOrSharpensTheDistribution) {
  const float logits[] = {0, 1, 2};
  SamplingConfig hot, cold;
  hot.temperature = 100.0F;
  cold.temperature = 0.01F;
  auto ph = sampling_probabilities(logits, 3, hot);
  auto pc = sampling_probabilities(logits, 3, cold);
  EXPECT_NEAR(ph[0], ph[2], 0.05);
  EXPECT_TRUE(pc[2] > 0.99F);
}

TEST(Sampling, TopKKeepsOnlyTheKHighest) {
  const float logits[] = {5, 1, 4, 2, 3};
  SamplingConfig cfg;
  cfg.top_k = 2;
  auto p = sampling_probabilities(logits, 5, cfg);
  EXPECT_TRUE(p[0] > 0.0F && p[2] > 0.0F);
  EXPECT_TRUE(p[1] == 0.0F && p[3] == 0.0F && p[4] == 0.0F);
  EXPECT_NEAR(sum(p), 1.0, 1e-6);
}

TEST(Sampling, TopPKeepsTheSmallestSufficientNucleus) {
  const float logits[] = {10, 0, 0, 0, 0};
  SamplingConfig cfg;
  cfg.top_p = 0.5F;
  auto p = sampling_probabilities(logits, 5, cfg);
  EXPECT_NEAR(p[0], 1.0F, 1e-5);
  for (std::size_t i = 1; i < 5; ++i) EXPECT_EQ(p[i], 0.0F);
}

TEST(Sampling, TopPAlwaysKeepsAtLeastOneToken) {
  const float logits[] = {1, 1, 1, 1};
  SamplingConfig cfg;
  cfg.top_p = 0.0F;
  auto p = sampling_probabilities(logits, 4, cfg);
  EXPECT_NEAR(sum(p), 1.0, 1e-6);
  EXPECT_EQ(std::count_if(p.begin(), p.end(), [](float x) { return x > 0; }), 1);
}

TEST(Sampling, SameSeedReproducesTheSameDraws) {
  const float logits[] = {1, 2, 3, 2, 1};
  SamplingConfig cfg;
  std::mt19937_64 a(42), b(42);
  std::vector<TokenId> da, db;
  for (int i = 0; i < 20; ++i) {
    da.push_back(sample(logits, 5, cfg, a));
    db.push_back(sample(logits, 5, cfg, b));
  }
  EXPECT_TRUE(da == db);
}

TEST(Sampling, DifferentSeedsCanDiffer) {
  const float logits[] = {1, 2, 3, 2, 1};
  SamplingConfig cfg;
  std::mt19937_64 a(1), b(2);
  bool any_different = false;
  for (int i = 0; i < 50; ++i) any_different = any_different || sample(logits, 5, cfg, a) != sample(logits, 5, cfg, b);
  EXPECT_TRUE(any_different);
}

TEST(Sampling, DrawsStayWithinTheFilteredSet) {
  const float logits[] = {5, 1, 4, 2, 3};
  SamplingConfig cfg;
  cfg.top_k = 2;
  std::mt19937_64 rng(7);
  for (int i = 0; i < 200; ++i) {
    const TokenId t = sample(logits, 5, cfg, rng);
    EXPECT_TRUE(t == 0 || t == 2);
  }
}

// A seeded run of sample() gives the oracle's tokens for the same draws, and
// consumes the generator exactly as the reference does (one number a call).
TEST(Sampling, SeededSequenceMatchesTheOracle) {
  const std::vector<float> logits = check::normal(5, 49152, 0.0, 3.0);
  const SamplingConfig cfgs[] = {{1.0F, 0, 1.0F}, {0.8F, 40, 0.9F}, {1.2F, 0, 0.6F}, {0.0F, 0, 1.0F}};
  for (const SamplingConfig& cfg : cfgs) {
    std::mt19937_64 rng(2024), mirror(2024);
    for (int i = 0; i < 16; ++i) {
      double target = 0.0;
      if (cfg.temperature > 0.0F) target = std::uniform_real_distribution<double>(0.0, 1.0)(mirror);
      const TokenId got = sample(logits.data(), logits.size(), cfg, rng);
      EXPECT_EQ(static_cast<std::size_t>(got),
                oracle_sample_target(logits.data(), logits.size(), cfg.temperature, cfg.top_k, cfg.top_p, target));
    }
    EXPECT_TRUE(rng == mirror);
    std::vector<float> want(logits.size());
    oracle_sampling_probabilities(logits.data(), logits.size(), cfg.temperature, cfg.top_k, cfg.top_p, want.data());
    const auto p = sampling_probabilities(logits.data(), logits.size(), cfg);
    EXPECT_TRUE(std::memcmp(p.data(), want.data(), want.size() * 4) == 0);
  }
}

TEST(Sampling, RejectsWhatTheReferenceLeavesUndefined) {
  const float nan_logits[] = {1.0F, std::nanf("")};
  std::mt19937_64 rng(3);
  bool threw = false;
  try {
    (void)sample(nan_logits, 2, SamplingConfig{}, rng);
  } catch (const std::invalid_argument&) {
    threw = true;
  }
  EXPECT_TRUE(threw);
  threw = false;
  try {
    (void)sampling_probabilities(nan_logits, 0, SamplingConfig{});
  } catch (const std::invalid_argument&) {
    threw = true;
  }
  EXPECT_TRUE(threw);
}
