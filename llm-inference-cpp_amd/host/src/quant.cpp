// llmi::quant on the GPU (the reference's src/model/quant.cpp interface).
#include "llmi/model/quant.hpp"

#include <mutex>
#include <stdexcept>
#include <string>

#include "llmi_hip.h"

namespace llmi::quant {

namespace {
std::once_flag g_once;
int g_device = 0;

void ensure_init() {
  std::call_once(g_once, [] {
    if (llmi_hip_init(g_device) != LLMI_OK) throw std::runtime_error(std::string("llmi_hip_init: ") + llmi_hip_last_error());
  });
}

void check(int rc, const char* what) {
  if (rc != LLMI_OK) throw std::runtime_error(std::string(what) + ": " + llmi_hip_last_error());
}

int abi_type(Type t) {
  switch (t) {
    case Type::Q8_0: return LLMI_TYPE_Q8_0;
    case Type::Q4_0: return LLMI_TYPE_Q4_0;
    default: throw std::invalid_argument("quant: type must be Q8_0 or Q4_0");
  }
}

struct Uploaded {
  llmi_hip_weight* w = nullptr;
  ~Uploaded() { llmi_hip_weight_free(w); }
};

void upload(const QuantizedMatrix& m, Uploaded& u) {
  ensure_init();
  check(llmi_hip_weight_upload(m.data.data(), m.scales.data(), m.out, m.in, abi_type(m.type), &u.w),
        "llmi_hip_weight_upload");
}
}  // namespace

void use_device(int device) { g_device = device; }

std::string_view type_name(Type t) {
  switch (t) {
    case Type::F32: return "f32";
    case Type::Q8_0: return "q8_0";
    case Type::Q4_0: return "q4_0";
  }
  return "unknown";
}

QuantizedMatrix quantize(const float* w, std::size_t out, std::size_t in, Type type) {
  ensure_init();
  QuantizedMatrix m;
  m.type = type;
  m.out = out;
  m.in = in;
  m.blocks_per_row = (in + kBlockSize - 1) / kBlockSize;
  m.scales.assign(out * m.blocks_per_row, 0.0F);
  m.data.assign(out * llmi_hip_row_bytes(in, abi_type(type)), 0);
  if (out > 0 && in > 0) check(llmi_hip_quantize(w, out, in, abi_type(type), m.data.data(), m.scales.data()), "llmi_hip_quantize");
  return m;
}

// Only the row travels to the device, as a one-row matrix: a loop over the
// rows of a large matrix then moves each row once, not the whole matrix per
// row.
void dequantize_row(const QuantizedMatrix& m, std::size_t row, float* dst) {
  ensure_init();
  if (row >= m.out) throw std::runtime_error("llmi_hip_dequantize_row: dequantize_row: row out of range");
  const std::size_t rb = llmi_hip_row_bytes(m.in, abi_type(m.type));
  Uploaded u;
  check(llmi_hip_weight_upload(m.data.data() + row * rb, m.scales.data() + row * m.blocks_per_row, 1, m.in,
                               abi_type(m.type), &u.w),
        "llmi_hip_weight_upload");
  check(llmi_hip_dequantize_row(u.w, 0, dst), "llmi_hip_dequantize_row");
}

void matmul(const float* x, std::size_t rows, std::size_t in, const QuantizedMatrix& w, std::size_t out,
            const float* bias, float* y) {
  Uploaded u;
  upload(w, u);
  check(llmi_hip_matmul(u.w, x, rows, in, out, bias, y), "llmi_hip_matmul");
}

// Used by weight.cpp and transformer.cpp.
void init_for_host_api() { ensure_init(); }

}  // namespace llmi::quant
