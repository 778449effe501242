// Prefill GEMM on the matrix cores (bf16 MFMA, fp32 accumulate) for gfx950.
//
// Reference: the prefill calls of quant::matmul (src/model/quant.cpp:119-153)
// with rows = T tokens (transformer.cpp:245-291).  y[t][o] = sum_k x[t][k] *
// code[o][k] * scale[o][k/32] (+ bias[o]).  Here x and the dequantized weights
// are rounded to bf16 and the products summed in fp32 by v_mfma_f32_16x16x32_bf16,
// so y differs from the reference by bf16 rounding (relative error ~1e-3;
// the tested bound is max|dy| <= 2e-2 * max|y|).  The exact path for the
// same shapes is llmi_hip_matmul_dev.
//
// One workgroup computes a 128 (tokens) x 128 (outputs) tile of y; its 4
// wavefronts each own a 64 x 64 quarter (4 x 4 MFMA tiles of 16 x 16).  Per
// K-step of 64 (two quantization blocks) every thread loads 32 activations
// (fp32) and 32 weight codes (one row of one block) from HBM into registers,
// converts them to bf16 (weights: code * scale) and stores them to LDS
// ([row][k], k contiguous, rows padded by 16 bytes so that the 16-byte
// operand reads of 8 consecutive lanes hit distinct banks).  The loads of the
// next K-step are issued before the MFMAs of the current one.
//
// Products are launched as groups (one kernel for many products; a single
// product is passed by value): workgroup w first maps to a work index so that consecutive work items -- the token
// tiles sharing one weight tile -- run on the same XCD (workgroups are
// dealt to the 8 XCDs round-robin), then finds its product through a
// work -> product map.
#include <algorithm>
#include <vector>

#include "common.hpp"

namespace llmi_hip {

namespace {

#define GMEM __attribute__((address_space(1)))

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kLdsRow = kBK + 8;  // bf16 per LDS row (16 bytes of padding)
constexpr int kXcds = 8;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ std::uint32_t pack_bf16(float a, float b) {
  const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(std::uint32_t, v);
}

__device__ __forceinline__ int sbyte(std::uint32_t w, int i) {
  return static_cast<int>(__builtin_amdgcn_sbfe(w, i * 8, 8));
}
__device__ __forceinline__ int snib(std::uint32_t w, int i) {
  return static_cast<int>(__builtin_amdgcn_sbfe(w ^ 0x88888888u, i * 4, 4));
}

template <int TYPE>
__global__ void __launch_bounds__(256) qgemm_mfma(const GemmProblem* __restrict__ probs,
                                                  const std::uint32_t* __restrict__ work_prob, int total,
                                                  GemmProblem one) {
  __shared__ __attribute__((aligned(16))) std::uint16_t xs[kBM * kLdsRow];
  __shared__ __attribute__((aligned(16))) std::uint16_t ws[kBN * kLdsRow];

  // Work index: workgroup w runs on XCD w % 8; give each XCD a contiguous
  // range of work items.
  const int w = blockIdx.x;
  const int per = total / kXcds, extra = total % kXcds;
  const int xcd = w % kXcds, slot = w / kXcds;
  const int work = xcd * per + min(xcd, extra) + slot;
  // A single product comes by value (no table); a group through the map.
  GemmProblem p = one;
  if (probs != nullptr) p = probs[__builtin_amdgcn_readfirstlane(static_cast<int>(work_prob[work]))];
  const int local = work - p.first_wg;
  const int mt = local % p.mtiles, nt = local / p.mtiles;
  const int m0 = mt * kBM, n0 = nt * kBN;
  const int M = p.rows, K = p.in, N = p.out, nblk = p.nblk;
  const GMEM float* x = (const GMEM float*)p.x;
  const GMEM u32x4* codes = (const GMEM u32x4*)p.codes;
  const GMEM float* scales = (const GMEM float*)p.scales;

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  // Staging map: thread t loads row t/2 of the tile, K half t%2 (32 values).
  const int lr = t >> 1, lh = t & 1;
  const int xm = m0 + lr;
  const int wn = n0 + lr;
  const int wtile = wn / kTileRows, wlane = wn % kTileRows;
  const bool xrow_ok = xm < M;
  const bool wrow_ok = wtile < p.ntiles;
  const bool xvec = (K & 3) == 0;

  float xv[32];
  std::uint32_t wc[8];
  float wscale = 0.0f;

  auto gload = [&](int k0) {
    const int kb = k0 + lh * 32;
    if (xrow_ok && xvec && kb + 32 <= K) {
      const GMEM f32x4* src = (const GMEM f32x4*)(x + static_cast<std::size_t>(xm) * K + kb);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const f32x4 v = src[i];
        xv[4 * i] = v.x;
        xv[4 * i + 1] = v.y;
        xv[4 * i + 2] = v.z;
        xv[4 * i + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 32; ++i)
        xv[i] = (xrow_ok && kb + i < K) ? x[static_cast<std::size_t>(xm) * K + kb + i] : 0.0f;
    }
    const int b = k0 / kBlock + lh;
    if (wrow_ok && b < nblk) {
      const std::size_t slot = static_cast<std::size_t>(wtile) * nblk + b;
      if (TYPE == LLMI_TYPE_Q8_0) {
        const u32x4 c0 = codes[(slot * 2 + 0) * kTileRows + wlane];
        const u32x4 c1 = codes[(slot * 2 + 1) * kTileRows + wlane];
        wc[0] = c0.x; wc[1] = c0.y; wc[2] = c0.z; wc[3] = c0.w;
        wc[4] = c1.x; wc[5] = c1.y; wc[6] = c1.z; wc[7] = c1.w;
      } else {
        const u32x4 c0 = codes[slot * kTileRows + wlane];
        wc[0] = c0.x; wc[1] = c0.y; wc[2] = c0.z; wc[3] = c0.w;
      }
      wscale = scales[slot * kTileRows + wlane];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) wc[i] = 0;
      wscale = 0.0f;
    }
  };

  auto lstore = [&]() {
    uint4* xd = reinterpret_cast<uint4*>(xs + lr * kLdsRow + lh * 32);
    uint4* wd = reinterpret_cast<uint4*>(ws + lr * kLdsRow + lh * 32);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint4 v;
      v.x = pack_bf16(xv[8 * q + 0], xv[8 * q + 1]);
      v.y = pack_bf16(xv[8 * q + 2], xv[8 * q + 3]);
      v.z = pack_bf16(xv[8 * q + 4], xv[8 * q + 5]);
      v.w = pack_bf16(xv[8 * q + 6], xv[8 * q + 7]);
      xd[q] = v;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float c[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int e = 8 * q + i;
        c[i] = static_cast<float>(TYPE == LLMI_TYPE_Q8_0 ? sbyte(wc[e >> 2], e & 3) : snib(wc[e >> 3], e & 7)) *
               wscale;
      }
      uint4 v;
      v.x = pack_bf16(c[0], c[1]);
      v.y = pack_bf16(c[2], c[3]);
      v.z = pack_bf16(c[4], c[5]);
      v.w = pack_bf16(c[6], c[7]);
      wd[q] = v;
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const int wm0 = (wave >> 1) * 64, wn0 = (wave & 1) * 64;
  const int arow = lane & 15, akoff = (lane >> 4) * 8;

  gload(0);
  for (int k0 = 0; k0 < K; k0 += kBK) {
    lstore();
    __syncthreads();
    if (k0 + kBK < K) gload(k0 + kBK);
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      bf16x8 a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a[i] = *reinterpret_cast<const bf16x8*>(xs + (wm0 + 16 * i + arow) * kLdsRow + kk + akoff);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        b[j] = *reinterpret_cast<const bf16x8*>(ws + (wn0 + 16 * j + arow) * kLdsRow + kk + akoff);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  // acc[i][j][q]: token m0 + wm0 + 16i + 4*(lane/16) + q, output n0 + wn0 + 16j + lane%16.
  GMEM float* y = (GMEM float*)p.y;
  const GMEM float* bias = (const GMEM float*)p.bias;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + wn0 + 16 * j + (lane & 15);
    if (n >= N) continue;
    const float add = bias != nullptr ? bias[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = m0 + wm0 + 16 * i + 4 * (lane >> 4) + q;
        if (m < M) y[static_cast<std::size_t>(m) * N + n] = acc[i][j][q] + add;
      }
  }
}

}  // namespace

int plan_gemm_group(const GroupEntry* entries, std::size_t count, GemmPlan* plan) {
  *plan = GemmPlan{};
  for (int type : {LLMI_TYPE_Q8_0, LLMI_TYPE_Q4_0}) {
    GemmLaunch l;
    l.type = type;
    l.prob_offset = plan->probs.size();
    l.map_offset = plan->work_prob.size();
    std::size_t wg = 0, nprob = 0;
    for (std::size_t i = 0; i < count; ++i) {
      const GroupEntry& e = entries[i];
      LLMI_REQUIRE(e.m != nullptr, "gemm: null weight");
      LLMI_REQUIRE(e.x != nullptr && e.y != nullptr, "gemm: null x or y");
      const DeviceMatrix& m = *e.m;
      LLMI_REQUIRE(m.in > 0 && m.in <= 0x7FFFFFFFu && m.out <= 0x7FFFFFFFu, "gemm: bad shape");
      LLMI_REQUIRE(e.rows <= 0x7FFFFFFFu, "gemm: too many rows");
      if (m.type != type || e.rows == 0 || m.out == 0) continue;
      GemmProblem p{};
      p.codes = m.codes;
      p.scales = m.scales;
      p.x = e.x;
      p.bias = e.bias;
      p.y = e.y;
      p.rows = static_cast<int>(e.rows);
      p.in = static_cast<int>(m.in);
      p.out = static_cast<int>(m.out);
      p.nblk = static_cast<int>(m.nblk);
      p.ntiles = static_cast<int>(m.ntiles);
      p.mtiles = static_cast<int>(ceil_div(e.rows, kBM));
      const std::size_t ntiles_n = ceil_div(m.out, kBN);
      p.first_wg = static_cast<int>(wg);
      const std::size_t wgs = static_cast<std::size_t>(p.mtiles) * ntiles_n;
      wg += wgs;
      LLMI_REQUIRE(wg <= 0x7FFFFFFFu, "gemm: too many workgroups");
      plan->work_prob.insert(plan->work_prob.end(), wgs, static_cast<std::uint32_t>(nprob));
      plan->probs.push_back(p);
      ++nprob;
    }
    if (nprob == 0) continue;
    l.total_wgs = static_cast<int>(wg);
    plan->launches.push_back(l);
  }
  return LLMI_OK;
}

int launch_gemm(const GemmProblem* probs_dev, const std::uint32_t* map_dev, const GemmLaunch& l, hipStream_t s,
                const GemmProblem* one) {
  if (l.total_wgs == 0) return LLMI_OK;
  const GemmProblem* probs = one != nullptr ? nullptr : probs_dev + l.prob_offset;
  const std::uint32_t* map = one != nullptr ? nullptr : map_dev + l.map_offset;
  const GemmProblem single = one != nullptr ? *one : GemmProblem{};
  if (l.type == LLMI_TYPE_Q8_0)
    qgemm_mfma<LLMI_TYPE_Q8_0><<<l.total_wgs, 256, 0, s>>>(probs, map, l.total_wgs, single);
  else
    qgemm_mfma<LLMI_TYPE_Q4_0><<<l.total_wgs, 256, 0, s>>>(probs, map, l.total_wgs, single);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

}  // namespace llmi_hip
