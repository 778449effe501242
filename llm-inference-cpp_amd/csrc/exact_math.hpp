// Bit-exact restatements of the two libm routines the reference's glue
// kernels call in single precision, for use on the GPU.
//
// expf: the reference's softmax and SiLU call std::exp(float)
// (src/model/kernels.cpp:141, :148), i.e. glibc's expf.  glibc (>= 2.28) uses
// the published ARM optimized-routines algorithm (math/expf.c): reduce
// x*N/ln2 = k + r with N = 32, look up 2^(k/N) in a 32-entry table, evaluate
// a degree-3 polynomial for 2^(r/N) in double, multiply, round to float once.
// The table below is tab[i] = bits(2^(i/32) rounded to double) - (i << 47)
// (derived independently and checked); the polynomial coefficients are the
// published ones.  glibc's x86-64 FMA build fuses the argument reduction
// (kd = x*N/ln2 + shift, r = x*N/ln2 - kd) and the polynomial steps; this
// restatement writes those fusions out.  It equals the host's expf on all
// 2^32 float inputs (tests/test_exact_math.py runs that comparison).
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define LLMI_HD __host__ __device__ __forceinline__
#else
#define LLMI_HD inline
#endif

namespace llmi_hip {
namespace exact {

LLMI_HD std::uint32_t f2u(float f) { return __builtin_bit_cast(std::uint32_t, f); }
LLMI_HD std::uint64_t d2u(double d) { return __builtin_bit_cast(std::uint64_t, d); }
LLMI_HD double u2d(std::uint64_t u) { return __builtin_bit_cast(double, u); }

#if defined(__HIP_DEVICE_COMPILE__)
#define LLMI_EXPF_TABLE_SPACE __constant__
#else
#define LLMI_EXPF_TABLE_SPACE
#endif

LLMI_EXPF_TABLE_SPACE static const std::uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// tab: the 32-entry table above, or a copy of it (e.g. in LDS, where a
// kernel calls expf many times per thread: a table index differs per lane, so
// every lookup is a memory load).
LLMI_HD float expf_with(float x, const std::uint64_t* tab) {
  constexpr double kN = 32.0;
  constexpr double kInvLn2N = 0x1.71547652b82fep+0 * kN;
  constexpr double kShift = 0x1.8p+52;
  constexpr double kC0 = 0x1.c6af84b912394p-5 / kN / kN / kN;
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / kN / kN;
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / kN;
  const std::uint32_t ux = f2u(x);
  const std::uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {  // |x| >= 88, or x is inf / nan
    if (ux == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8u) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double xd = static_cast<double>(x);
  double kd = __builtin_fma(kInvLn2N, xd, kShift);  // round(x*N/ln2) in the low bits
  const std::uint64_t ki = d2u(kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  std::uint64_t t = tab[ki % 32];
  t += ki << 47;
  const double s = u2d(t);
  const double zp = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(zp, r2, y);
  y = y * s;
  return static_cast<float>(y);
}

LLMI_HD float expf(float x) { return expf_with(x, kExp2Tab); }

}  // namespace exact
}  // namespace llmi_hip
