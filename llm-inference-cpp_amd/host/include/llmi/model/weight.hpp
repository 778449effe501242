// llmi::Weight on the MI355X: the interface of the reference's
// include/llmi/model/weight.hpp:18-39.  A quantized Weight lives in HBM (the
// GPU quantizer packs it straight into the device layout); copies share the
// device matrix, which is freed with the last copy.  matmul() and row() take
// and return host memory like the reference's and return with the result
// complete.  Type::F32 weights (from_float(), quantized() with F32) run the
// reference's kernels::matmul arithmetic on the GPU, bit for bit.
#pragma once

#include <cstddef>
#include <memory>
#include <vector>

#include "llmi/model/quant.hpp"
#include "llmi/util/result.hpp"

struct llmi_hip_weight;

namespace llmi {

class Weight {
 public:
  Weight() = default;
  static Weight from_float(std::vector<float> w);
  static Weight quantized(const std::vector<float>& w, std::size_t out, std::size_t in, quant::Type type);
  // A Weight of an already quantized matrix (e.g. from a GGUF file).
  static Weight from_quantized(const quant::QuantizedMatrix& m);
  // gguf::to_quantized (src/model/gguf.cpp:577-640) done on the device: the
  // raw bytes of a GGUF Q8_0 / Q4_0 tensor (gguf_type 8 / 2, the values of
  // gguf::TensorType) of shape [out][in] go to HBM as they are and are
  // converted there.  Fails where to_quantized fails (type, shape, size).
  static Result<Weight> from_gguf(const void* raw, std::size_t nbytes, std::size_t out, std::size_t in,
                                  int gguf_type);

  [[nodiscard]] bool empty() const;
  [[nodiscard]] std::size_t byte_size() const;
  [[nodiscard]] quant::Type type() const { return type_; }

  void matmul(const float* x, std::size_t rows, std::size_t in, std::size_t out, const float* bias, float* y) const;
  void row(std::size_t index, std::size_t in, float* dst) const;

  // The device matrix, for device-pointer callers (llmi_hip_matmul_dev).
  [[nodiscard]] const llmi_hip_weight* device() const { return dev_.get(); }

 private:
  void upload_f32(std::size_t in) const;  // from_float's matrix, once its shape is known

  quant::Type type_ = quant::Type::F32;
  mutable std::size_t out_ = 0, in_ = 0;
  mutable std::shared_ptr<llmi_hip_weight> dev_;
  mutable std::shared_ptr<const std::vector<float>> pending_;
};

}  // namespace llmi
