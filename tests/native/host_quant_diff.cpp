// Differential test of the C++ host layer's quant and Weight API
// (llmi::quant::quantize / dequantize_row / matmul and llmi::Weight of
// libllmi_gpu.so, which run on the GPU) against the CPU oracle
// (oracle/liboracle.so, the restatement of src/model/quant.cpp:36-153,
// src/model/weight.cpp:9-45 and src/model/gguf.cpp:577-640): for every case
// of a table of shapes, types, value ranges and row counts, every output
// must be the oracle's bit for bit.
#include <algorithm>
#include <cstring>
#include <stdexcept>

#include "check.hpp"
#include "llmi/model/quant.hpp"
#include "llmi/model/weight.hpp"
#include "llmi_hip.h"

extern "C" {
void oracle_quantize(const float* w, std::size_t out, std::size_t in, int type, std::uint8_t* data, float* scales);
void oracle_dequantize_row(const std::uint8_t* data, const float* scales, std::size_t in, int type, std::size_t row,
                           float* dst);
void oracle_matmul(const float* x, std::size_t rows, std::size_t in, const std::uint8_t* data, const float* scales,
                   int type, std::size_t out, const float* bias, float* y, int threads);
int oracle_gguf_to_quantized(const std::uint8_t* raw, std::size_t nbytes, std::size_t out, std::size_t in, int gtype,
                             std::uint8_t* data, float* scales);
float oracle_dot(const float* a, const float* b, std::size_t n);
}

namespace q = llmi::quant;

namespace {

int abi_type(q::Type t) { return t == q::Type::Q8_0 ? LLMI_TYPE_Q8_0 : LLMI_TYPE_Q4_0; }

bool bits_equal(const float* a, const float* b, std::size_t n) { return std::memcmp(a, b, n * sizeof(float)) == 0; }

// One matrix case: shape, type, weight spread, and the input row counts to
// multiply with (decode 1..8, the exact multi-row kernels above 8).
struct MatCase {
  std::size_t out, in;
  q::Type type;
  double sd;
  std::vector<std::size_t> rows;
};

const MatCase kMatrices[] = {
    {5, 1, q::Type::Q8_0, 1.0, {1, 2}},
    {9, 19, q::Type::Q4_0, 0.5, {1, 3}},
    {64, 32, q::Type::Q8_0, 0.02, {1, 8}},
    {65, 33, q::Type::Q4_0, 0.02, {1, 5, 9}},
    {130, 200, q::Type::Q8_0, 3.0, {1, 4, 17}},
    {200, 576, q::Type::Q4_0, 0.02, {1, 8, 40}},
    {1536, 576, q::Type::Q8_0, 0.02, {1, 2}},
    {896, 4864, q::Type::Q4_0, 0.02, {1, 8}},
    {4000, 300, q::Type::Q8_0, 0.3, {3}},
};

}  // namespace

TEST(QuantDiff, PackingDequantAndProductsEqualTheOracle) {
  std::uint64_t seed = 100;
  for (const MatCase& c : kMatrices) {
    const std::vector<float> w = check::normal(++seed, c.out * c.in, 0.0, c.sd);
    const q::QuantizedMatrix m = q::quantize(w.data(), c.out, c.in, c.type);
    std::vector<std::uint8_t> data(m.data.size());
    std::vector<float> scales(m.scales.size());
    oracle_quantize(w.data(), c.out, c.in, abi_type(c.type), data.data(), scales.data());
    ASSERT_TRUE(m.out == c.out && m.in == c.in && m.type == c.type);
    EXPECT_TRUE(m.data == data);
    EXPECT_TRUE(bits_equal(m.scales.data(), scales.data(), scales.size()));
    EXPECT_EQ(m.byte_size(), data.size() + 4 * scales.size());

    std::vector<float> got(c.in), want(c.in);
    for (std::size_t r : {std::size_t{0}, c.out / 2, c.out - 1}) {
      q::dequantize_row(m, r, got.data());
      oracle_dequantize_row(data.data(), scales.data(), c.in, abi_type(c.type), r, want.data());
      EXPECT_TRUE(bits_equal(got.data(), want.data(), c.in));
    }
    // Only the row is uploaded; a row past the matrix is an error, not a read.
    bool threw = false;
    try {
      q::dequantize_row(m, c.out, got.data());
    } catch (const std::runtime_error&) {
      threw = true;
    }
    EXPECT_TRUE(threw);

    const std::vector<float> bias = check::normal(seed + 7, c.out, 0.0, 0.1);
    for (std::size_t rows : c.rows) {
      const std::vector<float> x = check::normal(seed + 11 + rows, rows * c.in, 0.0, 1.0);
      for (const float* b : {static_cast<const float*>(nullptr), bias.data()}) {
        std::vector<float> y(rows * c.out), ref(rows * c.out);
        q::matmul(x.data(), rows, c.in, m, c.out, b, y.data());
        oracle_matmul(x.data(), rows, c.in, data.data(), scales.data(), abi_type(c.type), c.out, b, ref.data(), 0);
        if (!bits_equal(y.data(), ref.data(), y.size()))
          check::report(__FILE__, __LINE__, "matmul " + std::to_string(c.out) + "x" + std::to_string(c.in) +
                                                " rows " + std::to_string(rows));
      }
    }
  }
}

// Weight is a handle to one device matrix: quantized() and from_quantized()
// give products equal to quant::matmul, row() equals dequantize_row, and
// copies share the device allocation.
TEST(QuantDiff, WeightHandlesAgreeWithTheQuantFunctions) {
  const std::size_t out = 300, in = 96;
  const std::vector<float> w = check::normal(31, out * in, 0.0, 0.05);
  const std::vector<float> x = check::normal(32, 4 * in, 0.0, 1.0);
  for (q::Type type : {q::Type::Q8_0, q::Type::Q4_0}) {
    const q::QuantizedMatrix m = q::quantize(w.data(), out, in, type);
    const llmi::Weight a = llmi::Weight::quantized(w, out, in, type);
    const llmi::Weight b = llmi::Weight::from_quantized(m);
    const llmi::Weight shared = a;
    EXPECT_TRUE(shared.device() == a.device());
    EXPECT_TRUE(a.type() == type && a.byte_size() == m.byte_size());
    std::vector<float> ya(4 * out), yb(4 * out), yq(4 * out);
    a.matmul(x.data(), 4, in, out, nullptr, ya.data());
    b.matmul(x.data(), 4, in, out, nullptr, yb.data());
    q::matmul(x.data(), 4, in, m, out, nullptr, yq.data());
    EXPECT_TRUE(bits_equal(ya.data(), yq.data(), ya.size()));
    EXPECT_TRUE(bits_equal(yb.data(), yq.data(), yb.size()));
    std::vector<float> r1(in), r2(in);
    for (std::size_t row : {std::size_t{0}, std::size_t{123}, out - 1}) {
      shared.row(row, in, r1.data());
      q::dequantize_row(m, row, r2.data());
      EXPECT_TRUE(bits_equal(r1.data(), r2.data(), in));
    }
  }
}

// GGUF blocks straight into a device Weight: the rows and products equal the
// oracle's to_quantized of the same bytes, for random fp16 scales (all
// exponent ranges, incl. subnormal) and random codes; malformed inputs fail.
TEST(QuantDiff, GgufBlocksEqualTheOracleConversion) {
  struct G {
    int gtype;
    std::size_t qbytes;
    q::Type type;
  };
  for (const G g : {G{LLMI_GGUF_Q8_0, 32, q::Type::Q8_0}, G{LLMI_GGUF_Q4_0, 16, q::Type::Q4_0}}) {
    const std::size_t out = 70, in = 160, nb = out * in / 32;
    std::vector<std::uint8_t> raw(nb * (2 + g.qbytes));
    for (std::size_t i = 0; i < raw.size(); ++i)
      raw[i] = static_cast<std::uint8_t>(check::splitmix(77 + static_cast<std::uint64_t>(g.gtype), i) & 0xFF);
    for (std::size_t b = 0; b < nb; ++b) raw[b * (2 + g.qbytes) + 1] &= 0x3F;  // finite scales, |d| < 2
    auto dev = llmi::Weight::from_gguf(raw.data(), raw.size(), out, in, g.gtype);
    ASSERT_TRUE(dev.ok());
    std::vector<std::uint8_t> data(out * llmi_hip_row_bytes(in, abi_type(g.type)));
    std::vector<float> scales(nb);
    ASSERT_TRUE(oracle_gguf_to_quantized(raw.data(), raw.size(), out, in, g.gtype, data.data(), scales.data()) == 0);
    std::vector<float> r1(in), r2(in);
    for (std::size_t row = 0; row < out; row += 23) {
      dev->row(row, in, r1.data());
      oracle_dequantize_row(data.data(), scales.data(), in, abi_type(g.type), row, r2.data());
      EXPECT_TRUE(bits_equal(r1.data(), r2.data(), in));
    }
    const std::vector<float> x = check::normal(5, in, 0.0, 1.0);
    std::vector<float> y(out), ref(out);
    dev->matmul(x.data(), 1, in, out, nullptr, y.data());
    oracle_matmul(x.data(), 1, in, data.data(), scales.data(), abi_type(g.type), out, nullptr, ref.data(), 1);
    EXPECT_TRUE(bits_equal(y.data(), ref.data(), out));
    EXPECT_FALSE(llmi::Weight::from_gguf(raw.data(), raw.size() - 1, out, in, g.gtype).ok());
    EXPECT_FALSE(llmi::Weight::from_gguf(raw.data(), raw.size(), out, in, 0).ok());
  }
}

// fp32 weights (Weight::from_float / quantized(..., F32)) multiply with the
// reference's dot arithmetic: each output is the oracle's dot(x_r, w_o) plus
// the bias, bit for bit, over lengths that end on every tail residue.
TEST(QuantDiff, Float32WeightsEqualTheOracleDot) {
  for (std::size_t in : {1U, 15U, 16U, 17U, 40U, 129U}) {
    const std::size_t out = 37, rows = 3;
    const std::vector<float> w = check::normal(in, out * in, 0.0, 0.3);
    const std::vector<float> x = check::normal(in + 1, rows * in, 0.0, 1.0);
    const std::vector<float> bias = check::normal(in + 2, out, 0.0, 1.0);
    const llmi::Weight a = llmi::Weight::quantized(w, out, in, q::Type::F32);
    std::vector<float> y(rows * out);
    a.matmul(x.data(), rows, in, out, bias.data(), y.data());
    for (std::size_t r = 0; r < rows; ++r)
      for (std::size_t o = 0; o < out; ++o) {
        const float want = oracle_dot(x.data() + r * in, w.data() + o * in, in) + bias[o];
        EXPECT_TRUE(check::same_bits(y[r * out + o], want));
      }
    EXPECT_EQ(a.byte_size(), out * in * 4);
  }
}
