// Exact glue arithmetic shared by the model kernels and the fused GEMV
// prologues: the reference's RMSNorm scale and SiLU (src/model/kernels.cpp:
// 115-120, :148) and the bound that lets a parallel double sum stand in for
// the reference's sequential one.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "exact_math.hpp"

namespace llmi_hip {

// Bound on |sequential - parallel| for a sum of n non-negative doubles:
// both are within (n-1)u of the exact sum (u = 2^-53); 4nu covers both.
__device__ __forceinline__ double sum_slack(int n) { return 4.0 * static_cast<double>(n) * 0x1p-53; }

// kernels.cpp:115-120: scale = float(1 / sqrt(ss / n + eps)), ss the double
// sum of squares.
__device__ __forceinline__ float rms_scale(double ss, int n, float eps) {
  return static_cast<float>(1.0 / sqrt(ss / static_cast<double>(n) + static_cast<double>(eps)));
}

// kernels.cpp:148: x / (1 + exp(-x)) in float (IEEE division), with the
// exact expf (table `tab`: exact::kExp2Tab or a copy of it).
__device__ __forceinline__ float silu_exact(float v, const std::uint64_t* tab) {
  return v / (1.0f + exact::expf_with(-v, tab));
}

// The scalar part of kernels::dot (kernels.cpp:40-49, dot_scalar as the
// reference's build vectorises it) on the n < 16 elements left after the
// 16-lane chunks: 8 fused lanes over one 8-element chunk, then the leftovers
// (when 4 or more remain, the first 4 products are rounded on their own and
// added in order, the rest fused), the 8 lanes reduced pairwise, plus the
// leftovers.
__device__ __forceinline__ float ref_dot_rest(const float* __restrict__ a, const float* __restrict__ b, int n) {
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
  int i = 0;
  for (; i + 8 <= n; i += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = __builtin_fmaf(a[i + j], b[i + j], acc[j]);
  }
  float tail = 0.0f;
  if (n - i >= 4) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float p = a[i + j] * b[i + j];
      tail = tail + p;
    }
    i += 4;
  }
  for (; i < n; ++i) tail = __builtin_fmaf(a[i], b[i], tail);
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7])) + tail;
}

// The value of lane l of the wavefront (l uniform), broadcast to every lane.
__device__ __forceinline__ float readlane_f32(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ double readlane_f64(double v, int l) {
  const std::uint64_t u = __builtin_bit_cast(std::uint64_t, v);
  const std::uint32_t lo = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u), l));
  const std::uint32_t hi = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u >> 32), l));
  return __builtin_bit_cast(double, (static_cast<std::uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = v + __shfl_xor(v, o, 64);
  return v;
}

// v of lane l - N within its row of 16 lanes, 0.0 for the first N lanes of
// the row (DPP row_shr on both halves of the double).
template <int N>
__device__ __forceinline__ double row_shr_f64(double v) {
  const std::uint64_t u = __builtin_bit_cast(std::uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(u), 0x110 + N, 0xF, 0xF, true);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(u >> 32), 0x110 + N, 0xF, 0xF, true);
  return __builtin_bit_cast(double, (static_cast<std::uint64_t>(static_cast<std::uint32_t>(hi)) << 32) |
                                        static_cast<std::uint32_t>(lo));
}

// Sum of v over each row of 16 lanes, complete in the row's last lane
// (lanes 15, 31, 47, 63).  The order is a tree; callers use it only where
// any order of the double additions is acceptable.
__device__ __forceinline__ double row_sum16_f64(double v) {
  v = v + row_shr_f64<1>(v);
  v = v + row_shr_f64<2>(v);
  v = v + row_shr_f64<4>(v);
  v = v + row_shr_f64<8>(v);
  return v;
}

// Float reductions over each row of 16 lanes with DPP row shifts (complete
// in the row's last lane: 15, 31, 47, 63), and over the wavefront (the four
// row results read into scalars, so the result is uniform).  Tree orders:
// for the tolerance paths only.
template <int N>
__device__ __forceinline__ float row_shr_f32(float v, float fill) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v), 0x110 + N, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_max16_f32(float v) {
  v = fmaxf(v, row_shr_f32<1>(v, v));
  v = fmaxf(v, row_shr_f32<2>(v, v));
  v = fmaxf(v, row_shr_f32<4>(v, v));
  return fmaxf(v, row_shr_f32<8>(v, v));
}
__device__ __forceinline__ float row_sum16_f32(float v) {
  v += row_shr_f32<1>(v, 0.0f);
  v += row_shr_f32<2>(v, 0.0f);
  v += row_shr_f32<4>(v, 0.0f);
  return v + row_shr_f32<8>(v, 0.0f);
}
// Each lane gets its row's value from the row's last lane.
__device__ __forceinline__ float row_last_bcast(float v, int lane) {
  const float r0 = readlane_f32(v, 15), r1 = readlane_f32(v, 31), r2 = readlane_f32(v, 47), r3 = readlane_f32(v, 63);
  return lane < 32 ? (lane < 16 ? r0 : r1) : (lane < 48 ? r2 : r3);
}
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = row_max16_f32(v);
  return fmaxf(fmaxf(readlane_f32(v, 15), readlane_f32(v, 31)), fmaxf(readlane_f32(v, 47), readlane_f32(v, 63)));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v = row_sum16_f32(v);
  return (readlane_f32(v, 15) + readlane_f32(v, 31)) + (readlane_f32(v, 47) + readlane_f32(v, 63));
}

}  // namespace llmi_hip
