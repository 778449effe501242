// Device twin of the "synth-v1" deterministic generator
// (llm-inference-cpp_amd/synth.py): splitmix64 hashing, eight 16-bit lanes
// summed, (s - 4) * sqrt(1.5), then mean + std * z, each double operation
// rounded once (explicit _rn intrinsics, so nothing is contracted into an
// fma) and a single rounding to float32.  Used to build multi-GB synthetic
// weights on the GPU without a host round trip; tests check it against the
// host generator bit for bit.
#include "common.hpp"

namespace llmi_hip {
namespace {

__device__ __forceinline__ std::uint64_t splitmix(std::uint64_t seed, std::uint64_t c) {
  std::uint64_t z = seed + (c + 1ull) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__device__ __forceinline__ std::uint64_t lane_sum(std::uint64_t h) {
  return (h & 0xFFFFull) + ((h >> 16) & 0xFFFFull) + ((h >> 32) & 0xFFFFull) + (h >> 48);
}

__global__ void __launch_bounds__(256) synth_normal(float* __restrict__ dst, std::size_t n, std::uint64_t seed,
                                                    std::uint64_t offset, double mean, double stdev, double sqrt15) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const std::uint64_t idx = offset + i;
  const std::uint64_t total = lane_sum(splitmix(seed, 2 * idx)) + lane_sum(splitmix(seed, 2 * idx + 1));
  const double s = __ddiv_rn(__dadd_rn(static_cast<double>(total), 4.0), 65536.0);
  const double z = __dmul_rn(__dadd_rn(s, -4.0), sqrt15);
  dst[i] = static_cast<float>(__dadd_rn(mean, __dmul_rn(stdev, z)));
}

}  // namespace

int launch_synth_normal(float* dst, std::size_t n, std::uint64_t seed, std::uint64_t offset, double mean, double stdev,
                        hipStream_t s) {
  if (n == 0) return LLMI_OK;
  const double sqrt15 = 0x1.3988e1409212ep+0;  // the correctly rounded double of sqrt(1.5)
  synth_normal<<<static_cast<unsigned>(ceil_div(n, 256)), 256, 0, s>>>(dst, n, seed, offset, mean, stdev, sqrt15);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

}  // namespace llmi_hip
