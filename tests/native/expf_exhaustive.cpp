// Compares llmi_hip::exact::expf (llm-inference-cpp_amd/csrc/exact_math.hpp)
// with the host libm's expf on every float bit pattern (or a stride of them).
// Prints "mismatches N first X".  Built and run by tests/test_exact_math.py.
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "../../llm-inference-cpp_amd/csrc/exact_math.hpp"

int main(int argc, char** argv) {
  const std::uint64_t stride = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 1;
  const unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  std::atomic<std::uint64_t> bad{0}, first{~0ull};
  std::vector<std::thread> pool;
  for (unsigned t = 0; t < nt; ++t)
    pool.emplace_back([&, t] {
      std::uint64_t b = 0;
      for (std::uint64_t u = t * stride; u < (1ull << 32); u += nt * stride) {
        const std::uint32_t bits = static_cast<std::uint32_t>(u);
        float x;
        std::memcpy(&x, &bits, 4);
        const float want = expf(x);
        const float got = llmi_hip::exact::expf(x);
        if (std::isnan(want) && std::isnan(got)) continue;
        if (llmi_hip::exact::f2u(want) != llmi_hip::exact::f2u(got)) {
          std::uint64_t f = first.load();
          while (u < f && !first.compare_exchange_weak(f, u)) {
          }
          ++b;
        }
      }
      bad += b;
    });
  for (auto& th : pool) th.join();
  std::printf("mismatches %llu first %llx\n", static_cast<unsigned long long>(bad.load()),
              static_cast<unsigned long long>(first.load()));
  return bad.load() == 0 ? 0 : 1;
}
