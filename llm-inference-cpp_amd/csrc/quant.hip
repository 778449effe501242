// Block quantizer (fp32 -> Q8_0 / Q4_0), the planar <-> tiled re-layout, and
// the row dequantizer (embedding gather) for gfx950.
//
// The quantizer restates src/model/quant.cpp:36-102 one 32-weight block per
// thread: the block scan, the scale and every code are computed exactly as
// the reference computes them (IEEE fp32 divide for the scale, IEEE fp64
// divide and round-half-away-from-zero for the codes), so the packed bytes
// are bit-identical.  Load-time work: it reads each weight once (4 B) and
// writes 0.625 / 1.125 B, so it is HBM-bound.
#include "common.hpp"

namespace llmi_hip {
namespace {

// C lround: round half away from zero.  |q| <= 128 here (|v| <= amax), so
// q - trunc(q) is exact.
__device__ __forceinline__ int round_half_away(double q) {
  const double t = trunc(q);
  const double frac = q - t;
  double r = t;
  if (frac >= 0.5) r = t + 1.0;
  if (frac <= -0.5) r = t - 1.0;
  return static_cast<int>(r);
}

template <int TYPE>
__global__ void __launch_bounds__(256) quantize_blocks(const float* __restrict__ w, std::size_t out, int in, int nblk,
                                                       std::uint8_t* __restrict__ pdata, float* __restrict__ pscales,
                                                       std::uint8_t* __restrict__ tcodes,
                                                       float* __restrict__ tscales) {
  const std::size_t gid = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= out * static_cast<std::size_t>(nblk)) return;
  const std::size_t r = gid / nblk;
  const int b = static_cast<int>(gid % nblk);
  const int first = b * kBlock;
  const int n = min(kBlock, in - first);
  const float* src = w + r * static_cast<std::size_t>(in) + first;

  float v[kBlock];
#pragma unroll
  for (int i = 0; i < kBlock; ++i) v[i] = i < n ? src[i] : 0.0f;

  // quant.cpp:54-62: strict '>' keeps the first index of the largest |v|.
  float peak = 0.0f, peak_signed = 0.0f;
#pragma unroll
  for (int i = 0; i < kBlock; ++i) {
    const float mag = fabsf(v[i]);
    if (i < n && mag > peak) {
      peak = mag;
      peak_signed = v[i];
    }
  }
  float d = TYPE == LLMI_TYPE_Q4_0 ? peak_signed / -8.0f : peak / 127.0f;  // quant.cpp:63-80
  if (d == 0.0f) d = 1.0f;                                                  // quant.cpp:81
  const int hi = TYPE == LLMI_TYPE_Q4_0 ? 7 : 127;
  const int lo = TYPE == LLMI_TYPE_Q4_0 ? -8 : -127;

  // Codes, packed into 32-bit words in the reference's byte order.
  constexpr int kWords = TYPE == LLMI_TYPE_Q4_0 ? 4 : 8;
  std::uint32_t word[kWords];
#pragma unroll
  for (int k = 0; k < kWords; ++k) word[k] = 0u;
#pragma unroll
  for (int i = 0; i < kBlock; ++i) {
    if (i < n) {
      int q = round_half_away(static_cast<double>(v[i]) / static_cast<double>(d));  // quant.cpp:85
      q = min(max(q, lo), hi);
      if (TYPE == LLMI_TYPE_Q8_0) {
        word[i / 4] |= (static_cast<std::uint32_t>(q) & 0xFFu) << (8 * (i % 4));
      } else {
        word[i / 8] |= static_cast<std::uint32_t>(q + 8) << (4 * (i % 8));
      }
    }
  }

  if (pdata != nullptr) {
    const std::size_t rb = TYPE == LLMI_TYPE_Q4_0 ? (static_cast<std::size_t>(in) + 1) / 2 : static_cast<std::size_t>(in);
    std::uint8_t* dst = pdata + r * rb + (TYPE == LLMI_TYPE_Q4_0 ? first / 2 : first);
    const int nbytes = TYPE == LLMI_TYPE_Q4_0 ? (n + 1) / 2 : n;
#pragma unroll
    for (int j = 0; j < (TYPE == LLMI_TYPE_Q4_0 ? 16 : 32); ++j)
      if (j < nbytes) dst[j] = static_cast<std::uint8_t>(word[j / 4] >> (8 * (j % 4)));
    pscales[r * nblk + b] = d;
  }
  if (tcodes != nullptr) {
    const std::size_t tile = r / kTileRows;
    const int lane = static_cast<int>(r % kTileRows);
    const std::size_t slot = tile * nblk + b;
    if (TYPE == LLMI_TYPE_Q4_0) {
      reinterpret_cast<uint4*>(tcodes)[slot * kTileRows + lane] = make_uint4(word[0], word[1], word[2], word[3]);
    } else {
      uint4* dst = reinterpret_cast<uint4*>(tcodes);
      dst[(slot * 2 + 0) * kTileRows + lane] = make_uint4(word[0], word[1], word[2], word[3]);
      dst[(slot * 2 + 1) * kTileRows + lane] = make_uint4(word[4], word[5], word[6], word[7]);
    }
    tscales[slot * kTileRows + lane] = d;
  }
}

// Planar (reference) layout -> tiled device layout, one block per thread.
template <int TYPE>
__global__ void __launch_bounds__(256) planar_to_tiled(const std::uint8_t* __restrict__ pdata,
                                                       const float* __restrict__ pscales, std::size_t out, int in,
                                                       int nblk, std::uint8_t* __restrict__ tcodes,
                                                       float* __restrict__ tscales) {
  const std::size_t gid = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= out * static_cast<std::size_t>(nblk)) return;
  const std::size_t r = gid / nblk;
  const int b = static_cast<int>(gid % nblk);
  const int first = b * kBlock;
  const int n = min(kBlock, in - first);
  const std::size_t rb = TYPE == LLMI_TYPE_Q4_0 ? (static_cast<std::size_t>(in) + 1) / 2 : static_cast<std::size_t>(in);
  const std::uint8_t* src = pdata + r * rb + (TYPE == LLMI_TYPE_Q4_0 ? first / 2 : first);
  const int nbytes = TYPE == LLMI_TYPE_Q4_0 ? (n + 1) / 2 : n;
  constexpr int kBytes = TYPE == LLMI_TYPE_Q4_0 ? 16 : 32;
  std::uint32_t word[kBytes / 4];
#pragma unroll
  for (int k = 0; k < kBytes / 4; ++k) word[k] = 0u;
#pragma unroll
  for (int j = 0; j < kBytes; ++j)
    if (j < nbytes) word[j / 4] |= static_cast<std::uint32_t>(src[j]) << (8 * (j % 4));
  const std::size_t tile = r / kTileRows;
  const int lane = static_cast<int>(r % kTileRows);
  const std::size_t slot = tile * nblk + b;
  uint4* dst = reinterpret_cast<uint4*>(tcodes);
  if (TYPE == LLMI_TYPE_Q4_0) {
    dst[slot * kTileRows + lane] = make_uint4(word[0], word[1], word[2], word[3]);
  } else {
    dst[(slot * 2 + 0) * kTileRows + lane] = make_uint4(word[0], word[1], word[2], word[3]);
    dst[(slot * 2 + 1) * kTileRows + lane] = make_uint4(word[4], word[5], word[6], word[7]);
  }
  tscales[slot * kTileRows + lane] = pscales[r * nblk + b];
}

// IEEE binary16 -> binary32, exactly, as integer operations (src/model/
// safetensors.cpp:249-273 maps the same way: subnormals normalised, the
// infinities and NaNs keep their payload bits unchanged).
__device__ __forceinline__ float half_bits_to_float(std::uint32_t h) {
  const std::uint32_t sign = (h & 0x8000u) << 16;
  const std::uint32_t e = (h >> 10) & 0x1Fu;
  const std::uint32_t m = h & 0x3FFu;
  std::uint32_t bits;
  if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else {
      const int top = 31 - __builtin_clz(m);  // leading one of the mantissa, 0..9: value 2^(top - 24) * 1.f
      bits = sign | (static_cast<std::uint32_t>(top + 103) << 23) | ((m << (23 - top)) & 0x7FFFFFu);
    }
  } else if (e == 0x1F) {
    bits = sign | 0x7F800000u | (m << 13);
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  return __uint_as_float(bits);
}

// GGUF (ggml) blocks -> tiled device layout, one block per thread
// (gguf.cpp:577-640, to_quantized).  A ggml block is {fp16 d; codes}:
// Q8_0 34 bytes, its 32 signed codes in element order (copied as they are);
// Q4_0 18 bytes, byte j holding element j in the low nibble and element
// j + 16 in the high nibble, re-packed here into this library's pairs of
// neighbours (byte k: element 2k low, 2k + 1 high).  Blocks start 2-byte
// aligned (both sizes are even), so they are read as 16-bit words.
template <int TYPE>
__global__ void __launch_bounds__(256) gguf_to_tiled(const std::uint16_t* __restrict__ raw, std::size_t out, int nblk,
                                                     std::uint8_t* __restrict__ tcodes,
                                                     float* __restrict__ tscales) {
  const std::size_t gid = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= out * static_cast<std::size_t>(nblk)) return;
  const std::size_t r = gid / nblk;
  const int b = static_cast<int>(gid % nblk);
  constexpr int kHalfwords = TYPE == LLMI_TYPE_Q4_0 ? 9 : 17;
  const std::uint16_t* src = raw + gid * kHalfwords;
  std::uint32_t word[TYPE == LLMI_TYPE_Q4_0 ? 4 : 8];
  if (TYPE == LLMI_TYPE_Q8_0) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      word[k] = static_cast<std::uint32_t>(src[1 + 2 * k]) | (static_cast<std::uint32_t>(src[2 + 2 * k]) << 16);
  } else {
    std::uint8_t q[16];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      q[2 * k] = static_cast<std::uint8_t>(src[1 + k] & 0xFFu);
      q[2 * k + 1] = static_cast<std::uint8_t>(src[1 + k] >> 8);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) word[k] = 0u;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int e0 = 2 * k, e1 = 2 * k + 1;  // elements of engine byte k
      const std::uint32_t n0 = e0 < 16 ? (q[e0] & 0xFu) : (q[e0 - 16] >> 4);
      const std::uint32_t n1 = e1 < 16 ? (q[e1] & 0xFu) : (q[e1 - 16] >> 4);
      word[k / 4] |= (n0 | (n1 << 4)) << (8 * (k % 4));
    }
  }
  const std::size_t tile = r / kTileRows;
  const int lane = static_cast<int>(r % kTileRows);
  const std::size_t slot = tile * nblk + b;
  uint4* dst = reinterpret_cast<uint4*>(tcodes);
  if (TYPE == LLMI_TYPE_Q4_0) {
    dst[slot * kTileRows + lane] = make_uint4(word[0], word[1], word[2], word[3]);
  } else {
    dst[(slot * 2 + 0) * kTileRows + lane] = make_uint4(word[0], word[1], word[2], word[3]);
    dst[(slot * 2 + 1) * kTileRows + lane] = make_uint4(word[4], word[5], word[6], word[7]);
  }
  tscales[slot * kTileRows + lane] = half_bits_to_float(src[0]);
}

// Tiled device layout -> planar (reference) layout, one block per thread.
template <int TYPE>
__global__ void __launch_bounds__(256) tiled_to_planar(const std::uint8_t* __restrict__ tcodes,
                                                       const float* __restrict__ tscales, std::size_t out, int in,
                                                       int nblk, std::uint8_t* __restrict__ pdata,
                                                       float* __restrict__ pscales) {
  const std::size_t gid = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (gid >= out * static_cast<std::size_t>(nblk)) return;
  const std::size_t r = gid / nblk;
  const int b = static_cast<int>(gid % nblk);
  const int first = b * kBlock;
  const int n = min(kBlock, in - first);
  const std::size_t tile = r / kTileRows;
  const int lane = static_cast<int>(r % kTileRows);
  const std::size_t slot = tile * nblk + b;
  const uint4* src = reinterpret_cast<const uint4*>(tcodes);
  std::uint32_t word[8];
  uint4 a = TYPE == LLMI_TYPE_Q4_0 ? src[slot * kTileRows + lane] : src[(slot * 2 + 0) * kTileRows + lane];
  word[0] = a.x; word[1] = a.y; word[2] = a.z; word[3] = a.w;
  if (TYPE == LLMI_TYPE_Q8_0) {
    const uint4 c = src[(slot * 2 + 1) * kTileRows + lane];
    word[4] = c.x; word[5] = c.y; word[6] = c.z; word[7] = c.w;
  }
  const std::size_t rb = TYPE == LLMI_TYPE_Q4_0 ? (static_cast<std::size_t>(in) + 1) / 2 : static_cast<std::size_t>(in);
  std::uint8_t* dst = pdata + r * rb + (TYPE == LLMI_TYPE_Q4_0 ? first / 2 : first);
  const int nbytes = TYPE == LLMI_TYPE_Q4_0 ? (n + 1) / 2 : n;
#pragma unroll
  for (int j = 0; j < (TYPE == LLMI_TYPE_Q4_0 ? 16 : 32); ++j)
    if (j < nbytes) dst[j] = static_cast<std::uint8_t>(word[j / 4] >> (8 * (j % 4)));
  pscales[r * nblk + b] = tscales[slot * kTileRows + lane];
}

// quant.cpp:104-117 on the tiled layout: dst[t][k] = code * scale (one
// rounding), for token t's row ids[t].  grid.y = token.
template <int TYPE>
__global__ void __launch_bounds__(256) dequantize_rows(const std::uint8_t* __restrict__ tcodes,
                                                       const float* __restrict__ tscales, int in, int nblk,
                                                       const std::int32_t* __restrict__ ids,
                                                       float* __restrict__ dst) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= in) return;
  const std::size_t row = static_cast<std::size_t>(ids[blockIdx.y]);
  const std::size_t tile = row / kTileRows;
  const int lane = static_cast<int>(row % kTileRows);
  const int b = k / kBlock;
  const int i = k % kBlock;
  const std::size_t slot = tile * nblk + b;
  float code;
  if (TYPE == LLMI_TYPE_Q4_0) {
    const std::uint8_t byte = tcodes[(slot * kTileRows + lane) * 16 + i / 2];
    const int nib = (i & 1) ? (byte >> 4) : (byte & 0xF);
    code = static_cast<float>(nib - 8);
  } else {
    const std::uint8_t byte = tcodes[((slot * 2 + i / 16) * kTileRows + lane) * 16 + (i % 16)];
    code = static_cast<float>(static_cast<std::int8_t>(byte));
  }
  dst[static_cast<std::size_t>(blockIdx.y) * in + k] = code * tscales[slot * kTileRows + lane];
}

unsigned grid_for(std::size_t work, unsigned threads) { return static_cast<unsigned>(ceil_div(work, threads)); }

}  // namespace

int launch_quantize(const float* w, std::size_t out, std::size_t in, int type, std::uint8_t* planar_data,
                    float* planar_scales, DeviceMatrix* tiled, hipStream_t s) {
  const int nblk = static_cast<int>(ceil_div(in, kBlock));
  const std::size_t work = out * static_cast<std::size_t>(nblk);
  if (work == 0) return LLMI_OK;
  std::uint8_t* tc = tiled != nullptr ? tiled->codes : nullptr;
  float* ts = tiled != nullptr ? tiled->scales : nullptr;
  const unsigned g = grid_for(work, 256);
  if (type == LLMI_TYPE_Q8_0) {
    quantize_blocks<LLMI_TYPE_Q8_0><<<g, 256, 0, s>>>(w, out, static_cast<int>(in), nblk, planar_data, planar_scales, tc, ts);
  } else {
    quantize_blocks<LLMI_TYPE_Q4_0><<<g, 256, 0, s>>>(w, out, static_cast<int>(in), nblk, planar_data, planar_scales, tc, ts);
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int launch_relayout_to_tiled(const std::uint8_t* pdata, const float* pscales, const DeviceMatrix& m, hipStream_t s) {
  const std::size_t work = m.out * m.nblk;
  if (work == 0) return LLMI_OK;
  const unsigned g = grid_for(work, 256);
  if (m.type == LLMI_TYPE_Q8_0) {
    planar_to_tiled<LLMI_TYPE_Q8_0><<<g, 256, 0, s>>>(pdata, pscales, m.out, static_cast<int>(m.in), static_cast<int>(m.nblk), m.codes, m.scales);
  } else {
    planar_to_tiled<LLMI_TYPE_Q4_0><<<g, 256, 0, s>>>(pdata, pscales, m.out, static_cast<int>(m.in), static_cast<int>(m.nblk), m.codes, m.scales);
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int launch_gguf_to_tiled(const void* raw, const DeviceMatrix& m, hipStream_t s) {
  const std::size_t work = m.out * m.nblk;
  if (work == 0) return LLMI_OK;
  const unsigned g = grid_for(work, 256);
  const auto* src = static_cast<const std::uint16_t*>(raw);
  if (m.type == LLMI_TYPE_Q8_0) {
    gguf_to_tiled<LLMI_TYPE_Q8_0><<<g, 256, 0, s>>>(src, m.out, static_cast<int>(m.nblk), m.codes, m.scales);
  } else {
    gguf_to_tiled<LLMI_TYPE_Q4_0><<<g, 256, 0, s>>>(src, m.out, static_cast<int>(m.nblk), m.codes, m.scales);
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int launch_relayout_to_planar(const DeviceMatrix& m, std::uint8_t* pdata, float* pscales, hipStream_t s) {
  const std::size_t work = m.out * m.nblk;
  if (work == 0) return LLMI_OK;
  const unsigned g = grid_for(work, 256);
  if (m.type == LLMI_TYPE_Q8_0) {
    tiled_to_planar<LLMI_TYPE_Q8_0><<<g, 256, 0, s>>>(m.codes, m.scales, m.out, static_cast<int>(m.in), static_cast<int>(m.nblk), pdata, pscales);
  } else {
    tiled_to_planar<LLMI_TYPE_Q4_0><<<g, 256, 0, s>>>(m.codes, m.scales, m.out, static_cast<int>(m.in), static_cast<int>(m.nblk), pdata, pscales);
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int launch_dequantize_rows(const DeviceMatrix& m, const std::int32_t* ids, std::size_t n, float* dst, hipStream_t s) {
  if (m.type == LLMI_TYPE_F32) return launch_gather_f32(m, ids, n, dst, s);
  if (n == 0 || m.in == 0) return LLMI_OK;
  LLMI_REQUIRE(n <= 65535, "dequantize_rows: at most 65535 rows per call");
  const dim3 g(grid_for(m.in, 256), static_cast<unsigned>(n));
  if (m.type == LLMI_TYPE_Q8_0) {
    dequantize_rows<LLMI_TYPE_Q8_0><<<g, 256, 0, s>>>(m.codes, m.scales, static_cast<int>(m.in), static_cast<int>(m.nblk), ids, dst);
  } else {
    dequantize_rows<LLMI_TYPE_Q4_0><<<g, 256, 0, s>>>(m.codes, m.scales, static_cast<int>(m.in), static_cast<int>(m.nblk), ids, dst);
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

}  // namespace llmi_hip
