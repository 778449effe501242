// llmi::Weight on the GPU (the reference's src/model/weight.cpp interface).
#include "llmi/model/weight.hpp"

#include <stdexcept>
#include <string>

#include "llmi_hip.h"

namespace llmi::quant {
void init_for_host_api();
}

namespace llmi {

namespace {
void check(int rc, const char* what) {
  if (rc != LLMI_OK) throw std::runtime_error(std::string(what) + ": " + llmi_hip_last_error());
}
std::shared_ptr<llmi_hip_weight> own(llmi_hip_weight* w) {
  return std::shared_ptr<llmi_hip_weight>(w, [](llmi_hip_weight* p) { llmi_hip_weight_free(p); });
}
int abi_type(quant::Type t) {
  if (t == quant::Type::Q8_0) return LLMI_TYPE_Q8_0;
  if (t == quant::Type::Q4_0) return LLMI_TYPE_Q4_0;
  return LLMI_TYPE_F32;
}
}  // namespace

// weight.cpp:9-14: the fp32 matrix is kept as it is.  Its shape arrives with
// the first matmul()/row() call, which uploads it (row-major [out][in]).
Weight Weight::from_float(std::vector<float> w) {
  quant::init_for_host_api();
  Weight weight;
  weight.type_ = quant::Type::F32;
  weight.pending_ = std::make_shared<const std::vector<float>>(std::move(w));
  return weight;
}

void Weight::upload_f32(std::size_t in) const {
  if (dev_ != nullptr || pending_ == nullptr) return;
  if (in == 0 || pending_->size() % in != 0) throw std::invalid_argument("Weight: fp32 size is not a multiple of in");
  llmi_hip_weight* h = nullptr;
  check(llmi_hip_weight_quantize(pending_->data(), pending_->size() / in, in, LLMI_TYPE_F32, &h),
        "llmi_hip_weight_quantize");
  dev_ = own(h);
  out_ = pending_->size() / in;
  in_ = in;
  pending_.reset();
}

Weight Weight::quantized(const std::vector<float>& w, std::size_t out, std::size_t in, quant::Type type) {
  quant::init_for_host_api();
  Weight weight;
  weight.type_ = type;
  weight.out_ = out;
  weight.in_ = in;
  llmi_hip_weight* h = nullptr;
  check(llmi_hip_weight_quantize(w.data(), out, in, abi_type(type), &h), "llmi_hip_weight_quantize");
  weight.dev_ = own(h);
  return weight;
}

Weight Weight::from_quantized(const quant::QuantizedMatrix& m) {
  quant::init_for_host_api();
  Weight weight;
  weight.type_ = m.type;
  weight.out_ = m.out;
  weight.in_ = m.in;
  llmi_hip_weight* h = nullptr;
  check(llmi_hip_weight_upload(m.data.data(), m.scales.data(), m.out, m.in, abi_type(m.type), &h),
        "llmi_hip_weight_upload");
  weight.dev_ = own(h);
  return weight;
}

Result<Weight> Weight::from_gguf(const void* raw, std::size_t nbytes, std::size_t out, std::size_t in,
                                 int gguf_type) {
  quant::init_for_host_api();
  llmi_hip_weight* h = nullptr;
  if (llmi_hip_weight_from_gguf(raw, nbytes, out, in, gguf_type, &h) != LLMI_OK)
    return fail(std::string("gguf: to_quantized: ") + llmi_hip_last_error());
  Weight weight;
  weight.type_ = gguf_type == LLMI_GGUF_Q8_0 ? quant::Type::Q8_0 : quant::Type::Q4_0;
  weight.out_ = out;
  weight.in_ = in;
  weight.dev_ = own(h);
  return weight;
}

bool Weight::empty() const {
  if (pending_ != nullptr) return pending_->empty();
  return dev_ == nullptr || out_ == 0 || in_ == 0;
}

std::size_t Weight::byte_size() const {
  if (pending_ != nullptr) return pending_->size() * sizeof(float);  // weight.cpp:26-28
  if (dev_ == nullptr) return 0;
  std::size_t bytes = 0;
  llmi_hip_weight_info(dev_.get(), nullptr, nullptr, nullptr, &bytes);
  return bytes;
}

void Weight::matmul(const float* x, std::size_t rows, std::size_t in, std::size_t out, const float* bias,
                    float* y) const {
  upload_f32(in);
  if (dev_ == nullptr) throw std::logic_error("Weight::matmul on an empty weight");
  check(llmi_hip_matmul(dev_.get(), x, rows, in, out, bias, y), "llmi_hip_matmul");
}

void Weight::row(std::size_t index, std::size_t in, float* dst) const {
  upload_f32(in);
  if (dev_ == nullptr) throw std::logic_error("Weight::row on an empty weight");
  check(llmi_hip_dequantize_row(dev_.get(), index, dst), "llmi_hip_dequantize_row");
}

}  // namespace llmi
