// fp32 weights on the GPU: the reference's kernels::matmul
// (src/model/kernels.cpp:97-113, y[r][o] = dot(x_r, w_o, in) + bias[o]) and
// the Weight::row copy (src/model/weight.cpp:39-45) for Type::F32 weights.
//
// Storage: row-major [out][in] floats, as the reference keeps them.  One
// group of 16 lanes computes one dot exactly as the AVX2 kernels::dot does:
// lane j accumulates fused products of elements 16c + j over the full
// 16-element chunks, the lanes are reduced by the same tree ((j + j+8),
// (+4), (+2), (+1), as DPP row shifts), and the group's first lane adds the
// scalar part on the fewer than 16 elements left (ref_dot_rest).  The
// result, its bias and the optional residual update are the reference's
// operations in its order, so y is bit-identical.  Weight reads are 64-byte
// pieces per group and lane; x is shared by the workgroup's 16 dots.
#include "common.hpp"
#include "glue_math.hpp"

namespace llmi_hip {

namespace {

template <int N>
__device__ __forceinline__ float add_row_shl(float v) {
  const int src = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + N, 0xF, 0xF, true);
  return v + __int_as_float(src);
}

// grid (ceil(out / 16), rows), 256 threads: group g of 16 lanes computes
// output blockIdx.x * 16 + g of input row blockIdx.y.
__global__ void __launch_bounds__(256) matmul_f32(const float* __restrict__ x, const float* __restrict__ w,
                                                  const float* __restrict__ bias, float* __restrict__ y, int in,
                                                  int out, int accumulate) {
  const int j = threadIdx.x & 15;
  const int o = blockIdx.x * 16 + (threadIdx.x >> 4);
  const int r = blockIdx.y;
  const bool live = o < out;
  const float* xr = x + static_cast<std::size_t>(r) * in;
  const float* wr = w + static_cast<std::size_t>(live ? o : 0) * in;
  const int nfull = in / 16;
  float lane = 0.0f;
#pragma unroll 4
  for (int c = 0; c < nfull; ++c) lane = __builtin_fmaf(xr[16 * c + j], wr[16 * c + j], lane);
  lane = add_row_shl<8>(lane);
  lane = add_row_shl<4>(lane);
  lane = add_row_shl<2>(lane);
  lane = add_row_shl<1>(lane);
  if (j == 0 && live) {
    const float d = lane + ref_dot_rest(xr + 16 * nfull, wr + 16 * nfull, in - 16 * nfull);
    const float v = d + (bias != nullptr ? bias[o] : 0.0f);
    float* dst = y + static_cast<std::size_t>(r) * out + o;
    *dst = accumulate ? *dst + v : v;
  }
}

// dst[i] = rows ids[i] of w (the fp32 embedding gather).
__global__ void __launch_bounds__(256) gather_rows_f32(const float* __restrict__ w, const std::int32_t* __restrict__ ids,
                                                       std::size_t n, int in, float* __restrict__ dst) {
  const std::size_t e = static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n * static_cast<std::size_t>(in)) return;
  const std::size_t i = e / in;
  const int k = static_cast<int>(e % in);
  dst[e] = w[static_cast<std::size_t>(ids[i]) * in + k];
}

}  // namespace

int launch_matmul_f32(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y,
                      hipStream_t s, bool accumulate) {
  LLMI_REQUIRE(rows <= 65535, "matmul (f32): at most 65535 input rows per call");
  const dim3 grid(static_cast<unsigned>(ceil_div(m.out, 16)), static_cast<unsigned>(rows));
  matmul_f32<<<grid, 256, 0, s>>>(x, reinterpret_cast<const float*>(m.codes), bias, y, static_cast<int>(m.in),
                                  static_cast<int>(m.out), accumulate ? 1 : 0);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int launch_gather_f32(const DeviceMatrix& m, const std::int32_t* ids, std::size_t n, float* dst, hipStream_t s) {
  const std::size_t total = n * m.in;
  if (total == 0) return LLMI_OK;
  gather_rows_f32<<<static_cast<unsigned>(ceil_div(total, 256)), 256, 0, s>>>(
      reinterpret_cast<const float*>(m.codes), ids, n, static_cast<int>(m.in), dst);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

}  // namespace llmi_hip
