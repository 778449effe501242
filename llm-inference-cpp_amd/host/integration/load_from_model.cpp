// Transformer::load(const Model&, quant::Type) -- the reference's signature
// (include/llmi/model/transformer.hpp:58) -- for builds inside the reference
// engine: compile with -DLLMI_GPU_WITH_REFERENCE_MODEL and both include
// directories (this repository's host/include first).  It reads every tensor
// of the reference's Model (safetensors, F32/F16/BF16) as fp32 the way the
// reference's own load does (transformer.cpp:12-18) and hands them to the
// GPU model.
#include <string>
#include <vector>

#include "llmi/model/model.hpp"
#include "llmi/model/safetensors.hpp"
#include "llmi/model/transformer.hpp"

namespace llmi {

Result<Transformer> Transformer::load(const Model& model, quant::Type weight_type) {
  const SafetensorsFile& w = model.weights();
  const TensorReader read = [&w](const std::string& name) -> Result<std::vector<float>> {
    const TensorInfo* t = w.find(name);
    if (t == nullptr) return fail("load: missing tensor " + name);
    const auto raw = w.data(*t);
    std::vector<float> out(static_cast<std::size_t>(t->numel()));
    for (std::size_t i = 0; i < out.size(); ++i) out[i] = read_float(raw, t->dtype, i);
    return out;
  };
  return load(model.config(), read, weight_type);
}

}  // namespace llmi
