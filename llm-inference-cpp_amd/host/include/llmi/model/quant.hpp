// llmi::quant on the MI355X: the interface of the reference's
// include/llmi/model/quant.hpp:15-65 (names, types, argument meaning and the
// QuantizedMatrix layout are the reference's so callers compile unchanged),
// computed by libllmi_hip.so.  quantize() runs the bit-exact GPU quantizer;
// dequantize_row() and matmul() upload the host matrix for the call and run
// the GPU kernels -- callers that reuse a matrix should hold an llmi::Weight,
// which keeps it resident in HBM.  HIP failures throw std::runtime_error
// (the reference's versions cannot fail).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string_view>
#include <vector>

namespace llmi::quant {

inline constexpr std::size_t kBlockSize = 32;

enum class Type : std::uint8_t { F32, Q8_0, Q4_0 };

std::string_view type_name(Type t);

// out x in matrix of 32-weight blocks: Q8_0 int8 codes (data: out*in bytes)
// or Q4_0 +8-biased nibbles, two per byte by row-global index (data:
// out*ceil(in/2) bytes); one fp32 scale per block (out*ceil(in/32)).
struct QuantizedMatrix {
  Type type = Type::F32;
  std::size_t out = 0;
  std::size_t in = 0;
  std::size_t blocks_per_row = 0;
  std::vector<float> scales;
  std::vector<std::uint8_t> data;

  [[nodiscard]] bool empty() const { return out == 0 || in == 0; }
  [[nodiscard]] std::size_t byte_size() const { return data.size() + scales.size() * sizeof(float); }
};

QuantizedMatrix quantize(const float* w, std::size_t out, std::size_t in, Type type);
void dequantize_row(const QuantizedMatrix& m, std::size_t row, float* dst);
void matmul(const float* x, std::size_t rows, std::size_t in, const QuantizedMatrix& w, std::size_t out,
            const float* bias, float* y);

// Selects the GPU used by this process's quantized path (default 0; the
// first call of any function above initialises it otherwise).
void use_device(int device);

}  // namespace llmi::quant
