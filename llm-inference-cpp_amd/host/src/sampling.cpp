// llmi::sampling_probabilities / llmi::sample on the GPU (the reference's
// src/model/sampling.cpp interface).
#include "llmi/model/sampling.hpp"

#include <stdexcept>
#include <string>

#include "llmi_hip.h"

namespace llmi {
namespace quant {
void init_for_host_api();
}

namespace {
llmi_hip_sampling abi(const SamplingConfig& cfg) { return llmi_hip_sampling{cfg.temperature, cfg.top_k, cfg.top_p}; }

void check(int rc, const char* what) {
  if (rc == LLMI_OK) return;
  const std::string msg = std::string(what) + ": " + llmi_hip_last_error();
  if (rc == LLMI_ERR_ARG) throw std::invalid_argument(msg);
  throw std::runtime_error(msg);
}
}  // namespace

double detail::sample_draw(const SamplingConfig& cfg, std::mt19937_64& rng) {
  if (cfg.temperature <= 0.0F) return 0.0;
  std::uniform_real_distribution<double> u(0.0, 1.0);
  return u(rng);
}

std::vector<float> sampling_probabilities(const float* logits, std::size_t n, const SamplingConfig& cfg) {
  quant::init_for_host_api();
  std::vector<float> p(n);
  const llmi_hip_sampling c = abi(cfg);
  check(llmi_hip_sampling_probabilities(logits, n, &c, p.data()), "sampling_probabilities");
  return p;
}

TokenId sample(const float* logits, std::size_t n, const SamplingConfig& cfg, std::mt19937_64& rng) {
  quant::init_for_host_api();
  const double target = detail::sample_draw(cfg, rng);
  const llmi_hip_sampling c = abi(cfg);
  std::int32_t id = 0;
  check(llmi_hip_sample(logits, n, &c, target, &id), "sample");
  return static_cast<TokenId>(id);
}

}  // namespace llmi
