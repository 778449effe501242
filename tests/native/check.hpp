// Minimal test harness for the C++ tests (GoogleTest is not available
// offline): TEST(Suite, Name) registers a function; EXPECT_* record failures
// and keep going, ASSERT_* return from the test.  main() runs them all and
// prints one line per test.
#pragma once

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

namespace check {
struct Case {
  const char* suite;
  const char* name;
  std::function<void()> fn;
};
inline std::vector<Case>& cases() {
  static std::vector<Case> c;
  return c;
}
inline int& failures() {
  static int f = 0;
  return f;
}
struct Reg {
  Reg(const char* s, const char* n, std::function<void()> f) { cases().push_back({s, n, std::move(f)}); }
};
inline void report(const char* file, int line, const std::string& what) {
  std::printf("  FAILED %s:%d: %s\n", file, line, what.c_str());
  ++failures();
}

// Deterministic inputs: splitmix64 counter hash + Irwin-Hall(8), the
// synth-v1 generator of llm-inference-cpp_amd/synth.py.
inline std::uint64_t splitmix(std::uint64_t seed, std::uint64_t c) {
  std::uint64_t z = seed + (c + 1) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
inline std::vector<float> normal(std::uint64_t seed, std::size_t n, double mean, double sd) {
  std::vector<float> v(n);
  auto lanes = [](std::uint64_t h) { return (h & 0xFFFF) + ((h >> 16) & 0xFFFF) + ((h >> 32) & 0xFFFF) + (h >> 48); };
  for (std::size_t i = 0; i < n; ++i) {
    const double total = static_cast<double>(lanes(splitmix(seed, 2 * i)) + lanes(splitmix(seed, 2 * i + 1)));
    const double s = (total + 4.0) / 65536.0;
    const double z = (s - 4.0) * 1.2247448713915889;
    v[i] = static_cast<float>(mean + sd * z);
  }
  return v;
}
inline bool same_bits(float a, float b) {
  std::uint32_t x, y;
  std::memcpy(&x, &a, 4);
  std::memcpy(&y, &b, 4);
  return x == y;
}
}  // namespace check

#define TEST(S, N)                                         \
  static void S##_##N();                                   \
  static check::Reg S##_##N##_reg(#S, #N, S##_##N);        \
  static void S##_##N()
#define EXPECT_TRUE(c) \
  do { if (!(c)) check::report(__FILE__, __LINE__, #c); } while (0)
#define EXPECT_FALSE(c) EXPECT_TRUE(!(c))
#define EXPECT_EQ(a, b) EXPECT_TRUE((a) == (b))
#define EXPECT_NEAR(a, b, t) EXPECT_TRUE(std::fabs(static_cast<double>(a) - static_cast<double>(b)) <= (t))
#define ASSERT_TRUE(c) \
  do { if (!(c)) { check::report(__FILE__, __LINE__, #c); return; } } while (0)

int main() {
  int failed_tests = 0;
  for (auto& c : check::cases()) {
    const int before = check::failures();
    try {
      c.fn();
    } catch (const std::exception& e) {
      check::report(c.suite, 0, std::string("exception: ") + e.what());
    }
    const bool ok = check::failures() == before;
    failed_tests += ok ? 0 : 1;
    std::printf("[%s] %s.%s\n", ok ? "  OK  " : "FAILED", c.suite, c.name);
  }
  std::printf("%zu tests, %d failed\n", check::cases().size(), failed_tests);
  return failed_tests == 0 ? 0 : 1;
}
