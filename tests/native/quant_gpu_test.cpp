// The reference's tests/quant_test.cpp cases, run against the GPU drop-in
// (llmi::quant and llmi::Weight of libllmi_gpu.so), plus bit-exact checks
// against the CPU oracle (oracle/liboracle.so).
#include <algorithm>

#include "check.hpp"
#include "llmi/model/quant.hpp"
#include "llmi/model/weight.hpp"
#include "llmi_hip.h"

extern "C" {
void oracle_quantize(const float* w, std::size_t out, std::size_t in, int type, std::uint8_t* data, float* scales);
void oracle_matmul(const float* x, std::size_t rows, std::size_t in, const std::uint8_t* data, const float* scales,
                   int type, std::size_t out, const float* bias, float* y, int threads);
}

using namespace llmi::quant;

namespace {
std::vector<float> random_matrix(std::size_t out, std::size_t in, unsigned seed) {
  return check::normal(seed, out * in, 0.0, 0.3);
}
int t(Type type) { return type == Type::Q8_0 ? 1 : 2; }
}  // namespace

TEST(Quant, RoundTripQ8_0StaysWithinHalfAStepOfTheOriginal) {
  for (std::size_t in : {1U, 7U, 31U, 32U, 33U, 100U}) {
    constexpr std::size_t out = 3;
    const auto w = random_matrix(out, in, 1);
    const QuantizedMatrix q = quantize(w.data(), out, in, Type::Q8_0);
    ASSERT_TRUE(q.blocks_per_row == (in + kBlockSize - 1) / kBlockSize);
    std::vector<float> row(in);
    for (std::size_t r = 0; r < out; ++r) {
      dequantize_row(q, r, row.data());
      for (std::size_t b = 0; b < q.blocks_per_row; ++b) {
        const std::size_t start = b * kBlockSize, len = std::min(kBlockSize, in - start);
        float amax = 0.0F;
        for (std::size_t i = 0; i < len; ++i) amax = std::max(amax, std::fabs(w[r * in + start + i]));
        for (std::size_t i = 0; i < len; ++i) EXPECT_NEAR(row[start + i], w[r * in + start + i], amax / 254.0F + 1e-6F);
      }
    }
  }
}

TEST(Quant, RoundTripQ4_0StaysWithinOneStepOfTheOriginal) {
  for (std::size_t in : {1U, 7U, 31U, 32U, 33U, 100U}) {
    constexpr std::size_t out = 3;
    const auto w = random_matrix(out, in, 2);
    const QuantizedMatrix q = quantize(w.data(), out, in, Type::Q4_0);
    std::vector<float> row(in);
    for (std::size_t r = 0; r < out; ++r) {
      dequantize_row(q, r, row.data());
      for (std::size_t b = 0; b < q.blocks_per_row; ++b) {
        const std::size_t start = b * kBlockSize, len = std::min(kBlockSize, in - start);
        float amax = 0.0F;
        for (std::size_t i = 0; i < len; ++i) amax = std::max(amax, std::fabs(w[r * in + start + i]));
        for (std::size_t i = 0; i < len; ++i) EXPECT_NEAR(row[start + i], w[r * in + start + i], amax / 8.0F + 1e-6F);
      }
    }
  }
}

TEST(Quant, Q4_0ExtremeValueInEachBlockRoundTripsExactly) {
  const float positive_extreme[8] = {0.9F, -0.3F, 0.1F, 0.4F, -0.5F, 0.2F, -0.1F, 0.05F};
  const float negative_extreme[8] = {-0.9F, 0.3F, 0.1F, 0.4F, -0.5F, 0.2F, -0.1F, 0.05F};
  for (const float* w : {positive_extreme, negative_extreme}) {
    const QuantizedMatrix q = quantize(w, 1, 8, Type::Q4_0);
    std::vector<float> row(8);
    dequantize_row(q, 0, row.data());
    EXPECT_EQ(row[0], w[0]);
  }
}

TEST(Quant, AllZeroBlockRoundTripsToExactlyZero) {
  constexpr std::size_t in = 40;
  std::vector<float> w(in, 0.0F);
  for (Type type : {Type::Q8_0, Type::Q4_0}) {
    const QuantizedMatrix q = quantize(w.data(), 1, in, type);
    std::vector<float> row(in);
    dequantize_row(q, 0, row.data());
    for (float v : row) EXPECT_EQ(v, 0.0F);
  }
}

TEST(Quant, ByteSizeMatchesTheDocumentedCompressionRatio) {
  constexpr std::size_t out = 100, in = 3200;
  const auto w = random_matrix(out, in, 3);
  const auto f32_bytes = static_cast<double>(out * in * sizeof(float));
  EXPECT_NEAR(f32_bytes / static_cast<double>(quantize(w.data(), out, in, Type::Q8_0).byte_size()), 3.55, 0.05);
  EXPECT_NEAR(f32_bytes / static_cast<double>(quantize(w.data(), out, in, Type::Q4_0).byte_size()), 6.4, 0.1);
}

TEST(Quant, PackedBytesAreBitExactAgainstTheOracle) {
  for (Type type : {Type::Q8_0, Type::Q4_0})
    for (std::size_t in : {1U, 7U, 33U, 576U, 4864U}) {
      const std::size_t out = 70;
      const auto w = random_matrix(out, in, 9);
      const QuantizedMatrix q = quantize(w.data(), out, in, type);
      std::vector<std::uint8_t> data(q.data.size());
      std::vector<float> scales(q.scales.size());
      oracle_quantize(w.data(), out, in, t(type), data.data(), scales.data());
      EXPECT_TRUE(data == q.data);
      EXPECT_TRUE(std::memcmp(scales.data(), q.scales.data(), scales.size() * 4) == 0);
    }
}

TEST(Quant, MatmulMatchesDequantizeThenDotProduct) {
  constexpr std::size_t rows = 3, in = 300, out = 50;
  const auto x = check::normal(4, rows * in, 0.0, 0.5);
  const auto bias = check::normal(5, out, 0.0, 0.5);
  const auto w = random_matrix(out, in, 5);
  for (Type type : {Type::Q8_0, Type::Q4_0}) {
    const QuantizedMatrix q = quantize(w.data(), out, in, type);
    std::vector<float> y(rows * out), want(rows * out);
    matmul(x.data(), rows, in, q, out, bias.data(), y.data());
    std::vector<float> row(in);
    for (std::size_t o = 0; o < out; ++o) {
      dequantize_row(q, o, row.data());
      for (std::size_t r = 0; r < rows; ++r) {
        double dot = 0;
        for (std::size_t i = 0; i < in; ++i) dot += static_cast<double>(x[r * in + i]) * row[i];
        EXPECT_NEAR(y[r * out + o], dot + bias[o], 1e-3);
      }
    }
    oracle_matmul(x.data(), rows, in, q.data.data(), q.scales.data(), t(type), out, bias.data(), want.data(), 1);
    for (std::size_t i = 0; i < y.size(); ++i) EXPECT_TRUE(check::same_bits(y[i], want[i]));
  }
}

TEST(Quant, MatmulAboveTheThreadingThresholdMatchesARowByRowReference) {
  constexpr std::size_t rows = 3, in = 300, out = 4000;
  const auto x = check::normal(6, rows * in, 0.0, 0.5);
  const auto w = random_matrix(out, in, 7);
  const QuantizedMatrix q = quantize(w.data(), out, in, Type::Q8_0);
  std::vector<float> y(rows * out), want(rows * out);
  matmul(x.data(), rows, in, q, out, nullptr, y.data());
  oracle_matmul(x.data(), rows, in, q.data.data(), q.scales.data(), 1, out, nullptr, want.data(), 1);
  for (std::size_t i = 0; i < y.size(); ++i) EXPECT_TRUE(check::same_bits(y[i], want[i]));
}

TEST(Weight, QuantizedWeightMatchesTheQuantFunctionsAndSharesDeviceMemory) {
  const std::size_t out = 1536, in = 576;
  const auto w = check::normal(11, out * in, 0.0, 0.02);
  const auto x = check::normal(12, 2 * in, 0.0, 1.0);
  for (Type type : {Type::Q8_0, Type::Q4_0}) {
    const llmi::Weight weight = llmi::Weight::quantized(w, out, in, type);
    const QuantizedMatrix q = quantize(w.data(), out, in, type);
    EXPECT_EQ(weight.byte_size(), q.byte_size());
    EXPECT_TRUE(weight.type() == type);
    std::vector<float> y(2 * out), want(2 * out);
    weight.matmul(x.data(), 2, in, out, nullptr, y.data());
    matmul(x.data(), 2, in, q, out, nullptr, want.data());
    for (std::size_t i = 0; i < y.size(); ++i) EXPECT_TRUE(check::same_bits(y[i], want[i]));
    std::vector<float> r1(in), r2(in);
    weight.row(77, in, r1.data());
    dequantize_row(q, 77, r2.data());
    EXPECT_TRUE(std::memcmp(r1.data(), r2.data(), in * 4) == 0);
    const llmi::Weight copy = weight;  // copies share the device matrix
    EXPECT_TRUE(copy.device() == weight.device());
    const llmi::Weight again = llmi::Weight::from_quantized(q);
    std::vector<float> y2(2 * out);
    again.matmul(x.data(), 2, in, out, nullptr, y2.data());
    EXPECT_TRUE(std::memcmp(y.data(), y2.data(), y.size() * 4) == 0);
  }
}

// gguf_test.cpp:389-416 and :418-453 through Weight::from_gguf (the device
// does gguf::to_quantized): one Q8_0 block (scale 1.0, codes 0..31 in order)
// and one Q4_0 block (scale 2.0, byte 0 = 0x91: element 0 nibble 1, element
// 16 nibble 9).
TEST(Weight, FromGgufMatchesTheReferenceKnownAnswers) {
  std::vector<std::uint8_t> q8 = {0x00, 0x3C};
  for (int i = 0; i < 32; ++i) q8.push_back(static_cast<std::uint8_t>(i));
  auto w8 = llmi::Weight::from_gguf(q8.data(), q8.size(), 1, 32, LLMI_GGUF_Q8_0);
  EXPECT_TRUE(w8.ok());
  std::vector<float> row(32);
  w8->row(0, 32, row.data());
  for (int i = 0; i < 32; ++i) EXPECT_TRUE(row[static_cast<std::size_t>(i)] == static_cast<float>(i));
  std::vector<std::uint8_t> q4 = {0x00, 0x40, 0x91};
  for (int i = 1; i < 16; ++i) q4.push_back(0x88);
  auto w4 = llmi::Weight::from_gguf(q4.data(), q4.size(), 1, 32, LLMI_GGUF_Q4_0);
  EXPECT_TRUE(w4.ok());
  w4->row(0, 32, row.data());
  EXPECT_TRUE(row[0] == -14.0F && row[16] == 2.0F && row[1] == 0.0F && row[17] == 0.0F);
  EXPECT_TRUE(!llmi::Weight::from_gguf(q4.data(), q4.size(), 1, 32, 0).ok());  // F32 is not Q8_0/Q4_0
}

// transformer_test.cpp:30-44 (Kernels.MatmulWithBias) through fp32 Weights:
// kernels::matmul on the GPU, from_float (shape at the first call) and
// quantized(..., F32).
TEST(Weight, Float32WeightsRunTheReferenceMatmul) {
  const std::vector<float> x = {1, 2, 3, 4, 5, 6};
  const std::vector<float> w = {1, 0, -1, 0.5F, 0.5F, 0.5F};
  const float bias[] = {10, -1};
  for (int how = 0; how < 2; ++how) {
    const llmi::Weight weight = how == 0 ? llmi::Weight::from_float(w) : llmi::Weight::quantized(w, 2, 3, Type::F32);
    float y[4];
    weight.matmul(x.data(), 2, 3, 2, bias, y);
    EXPECT_TRUE(y[0] == 1 - 3 + 10.0F && y[1] == 3 - 1.0F && y[2] == 4 - 6 + 10.0F && y[3] == 7.5F - 1);
    weight.matmul(x.data(), 2, 3, 2, nullptr, y);
    EXPECT_TRUE(y[0] == -2.0F);
    EXPECT_TRUE(weight.byte_size() == 24);
    float r[3];
    weight.row(1, 3, r);
    EXPECT_TRUE(r[0] == 0.5F && r[1] == 0.5F && r[2] == 0.5F);
  }
}
