// llmi::sampling_probabilities and llmi::sample on the MI355X: the interface
// of the reference's include/llmi/model/sampling.hpp:20-39, computed on the
// GPU (llmi_hip_sampling_probabilities / llmi_hip_sample) with the
// reference's results bit for bit.  sample() draws its number from the
// caller's std::mt19937_64 exactly as the reference does (one
// std::uniform_real_distribution<double>(0, 1) draw per call unless
// temperature <= 0), so a seed replays the same tokens in both engines.
//
// Differences, both where the reference's result is undefined: n == 0, and
// logits that are NaN or +inf after the division by temperature, throw
// std::invalid_argument instead of returning an arbitrary index.  HIP
// failures throw std::runtime_error.
#pragma once

#include <cstddef>
#include <cstdint>
#include <random>
#include <vector>

#if defined(LLMI_GPU_WITH_REFERENCE_MODEL)
#include "llmi/tokenizer/tokenizer.hpp"
#endif

namespace llmi {

#if !defined(LLMI_GPU_WITH_REFERENCE_MODEL)
using TokenId = std::int32_t;
#endif

struct SamplingConfig {
  float temperature = 1.0F;
  std::size_t top_k = 0;  // 0 = no top-k filter
  float top_p = 1.0F;     // 1 = no nucleus filter
};

std::vector<float> sampling_probabilities(const float* logits, std::size_t n, const SamplingConfig& cfg);

TokenId sample(const float* logits, std::size_t n, const SamplingConfig& cfg, std::mt19937_64& rng);

namespace detail {
// The number sample() takes from rng (sampling.cpp:64-65), or 0 (and no
// draw) when temperature <= 0.
double sample_draw(const SamplingConfig& cfg, std::mt19937_64& rng);
}  // namespace detail

}  // namespace llmi
