// ============================================================================
// TEST INFRASTRUCTURE ONLY.
//
// A C ABI over the reference's own quantized-weight path, compiled together
// with the reference sources where they lie (/root/reference/src/...) into
// oracle/_ref/libllmi_ref.so by oracle/Makefile.  The golden-fixture script
// (tests/golden/gen_golden.py) and the oracle tests call it to pin the CPU
// restatement (oracle/oracle.cpp) against the real reference, and bench.py
// may time it as the CPU baseline.  No reference source is copied: this file
// only includes the reference's public headers and calls its functions.
// ============================================================================

#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../include/llmi_hip.h"
#include "llmi/model/gguf.hpp"
#include "llmi/model/kernels.hpp"
#include "llmi/model/model.hpp"
#include "llmi/model/quant.hpp"
#include "llmi/model/safetensors.hpp"
#include "llmi/model/sampling.hpp"
#include "llmi/model/transformer.hpp"
#include "llmi/util/thread_pool.hpp"

namespace {

thread_local std::string g_err;

llmi::quant::QuantizedMatrix wrap(const std::uint8_t* data, const float* scales, std::size_t out, std::size_t in,
                                  int type) {
  llmi::quant::QuantizedMatrix m;
  m.type = static_cast<llmi::quant::Type>(type);
  m.out = out;
  m.in = in;
  m.blocks_per_row = (in + llmi::quant::kBlockSize - 1) / llmi::quant::kBlockSize;
  const std::size_t rb = type == LLMI_TYPE_Q4_0 ? (in + 1) / 2 : in;
  m.data.assign(data, data + out * rb);
  m.scales.assign(scales, scales + out * m.blocks_per_row);
  return m;
}

struct RefModel {
  std::vector<std::byte> bytes;  // the in-memory safetensors file (must outlive the Model)
  std::unique_ptr<llmi::Transformer> tf;
  std::unique_ptr<llmi::KVCache> cache;
  std::uint32_t vocab = 0;
};

// The tensor manifest of src/model/model.cpp:135-162, rebuilt from the
// reference's own expected_tensors().
std::string config_json(const llmi_model_config& c) {
  char buf[1024];
  std::snprintf(buf, sizeof buf,
                "{\"architectures\": [\"%s\"], \"vocab_size\": %u, \"hidden_size\": %u, \"intermediate_size\": %u, "
                "\"num_hidden_layers\": %u, \"num_attention_heads\": %u, \"num_key_value_heads\": %u, "
                "\"max_position_embeddings\": %u, \"rms_norm_eps\": %.17g, \"rope_theta\": %.17g, "
                "\"tie_word_embeddings\": %s, \"attention_bias\": %s, \"hidden_act\": \"silu\"}",
                c.arch == 1 ? "Qwen2ForCausalLM" : "LlamaForCausalLM", c.vocab_size, c.hidden_size,
                c.intermediate_size, c.num_layers, c.num_heads, c.num_kv_heads, c.max_position_embeddings,
                c.rms_norm_eps, c.rope_theta, c.tie_word_embeddings ? "true" : "false",
                c.qkv_bias ? "true" : "false");
  return buf;
}

}  // namespace

extern "C" {

const char* ref_last_error() { return g_err.c_str(); }

int ref_pool_workers() { return static_cast<int>(llmi::util::ThreadPool::shared().num_workers()); }

void ref_quantize(const float* w, std::size_t out, std::size_t in, int type, std::uint8_t* data, float* scales) {
  const auto m = llmi::quant::quantize(w, out, in, static_cast<llmi::quant::Type>(type));
  std::memcpy(data, m.data.data(), m.data.size());
  std::memcpy(scales, m.scales.data(), m.scales.size() * sizeof(float));
}

void ref_dequantize_row(const std::uint8_t* data, const float* scales, std::size_t out, std::size_t in, int type,
                        std::size_t row, float* dst) {
  llmi::quant::dequantize_row(wrap(data, scales, out, in, type), row, dst);
}

void ref_matmul(const float* x, std::size_t rows, std::size_t in, const std::uint8_t* data, const float* scales,
                int type, std::size_t out, const float* bias, float* y) {
  const auto m = wrap(data, scales, out, in, type);
  llmi::quant::matmul(x, rows, in, m, out, bias, y);
}

// A QuantizedMatrix kept alive between calls, so timing loops measure
// quant::matmul alone.
void* ref_qmatrix_create(const std::uint8_t* data, const float* scales, std::size_t out, std::size_t in, int type) {
  return new llmi::quant::QuantizedMatrix(wrap(data, scales, out, in, type));
}
void ref_qmatrix_free(void* m) { delete static_cast<llmi::quant::QuantizedMatrix*>(m); }
void ref_qmatrix_matmul(void* m, const float* x, std::size_t rows, const float* bias, float* y) {
  const auto& q = *static_cast<llmi::quant::QuantizedMatrix*>(m);
  llmi::quant::matmul(x, rows, q.in, q, q.out, bias, y);
}

float ref_dot(const float* a, const float* b, std::size_t n) { return llmi::kernels::dot(a, b, n); }
void ref_rmsnorm(const float* x, const float* w, std::size_t n, float eps, float* y) { llmi::kernels::rmsnorm(x, w, n, eps, y); }
void ref_rope(float* v, std::size_t hd, std::size_t pos, const float* inv_freq) { llmi::kernels::rope(v, hd, pos, inv_freq); }
void ref_softmax(float* x, std::size_t n) { llmi::kernels::softmax(x, n); }
float ref_silu(float v) { return llmi::kernels::silu(v); }
std::size_t ref_argmax(const float* x, std::size_t n) { return llmi::argmax(x, n); }

// sampling.cpp: the reference's own filtering, and `count` successive sample()
// calls on one std::mt19937_64(seed).  targets[c] receives the number call c
// draws (read from a copy of the generator taken just before the call), or
// -1 where temperature <= 0 draws nothing.
void ref_sampling_probabilities(const float* logits, std::size_t n, float temperature, std::size_t top_k, float top_p,
                                float* out) {
  const llmi::SamplingConfig cfg{temperature, top_k, top_p};
  const std::vector<float> p = llmi::sampling_probabilities(logits, n, cfg);
  std::memcpy(out, p.data(), n * sizeof(float));
}
void ref_sample_sequence(const float* logits, std::size_t n, float temperature, std::size_t top_k, float top_p,
                         std::uint64_t seed, std::size_t count, std::int32_t* ids, double* targets) {
  const llmi::SamplingConfig cfg{temperature, top_k, top_p};
  std::mt19937_64 rng(seed);
  for (std::size_t c = 0; c < count; ++c) {
    std::mt19937_64 peek = rng;
    std::uniform_real_distribution<double> u(0.0, 1.0);
    targets[c] = temperature <= 0.0F ? -1.0 : u(peek);
    ids[c] = llmi::sample(logits, n, cfg, rng);
  }
}

// tensors: fp32 arrays in expected_tensors() order.
void* ref_model_create(const llmi_model_config* cfg, const float* const* tensors, int type) {
  auto parsed = llmi::parse_config(config_json(*cfg));
  if (!parsed) {
    g_err = parsed.error();
    return nullptr;
  }
  const auto list = llmi::expected_tensors(*parsed);
  std::string header = "{";
  std::uint64_t offset = 0;
  std::vector<std::uint64_t> sizes;
  for (std::size_t i = 0; i < list.size(); ++i) {
    std::uint64_t n = 1;
    std::string shape;
    for (std::size_t d = 0; d < list[i].shape.size(); ++d) {
      n *= list[i].shape[d];
      shape += (d != 0 ? "," : "") + std::to_string(list[i].shape[d]);
    }
    sizes.push_back(n);
    header += (i != 0 ? "," : "") + std::string("\"") + list[i].name + "\":{\"dtype\":\"F32\",\"shape\":[" + shape +
              "],\"data_offsets\":[" + std::to_string(offset) + "," + std::to_string(offset + n * 4) + "]}";
    offset += n * 4;
  }
  header += "}";
  auto rm = std::make_unique<RefModel>();
  rm->bytes.resize(8 + header.size() + offset);
  for (int k = 0; k < 8; ++k) rm->bytes[static_cast<std::size_t>(k)] = std::byte((header.size() >> (8U * k)) & 0xFFU);
  std::memcpy(rm->bytes.data() + 8, header.data(), header.size());
  std::size_t at = 8 + header.size();
  for (std::size_t i = 0; i < list.size(); ++i) {
    std::memcpy(rm->bytes.data() + at, tensors[i], sizes[i] * 4);
    at += sizes[i] * 4;
  }
  auto st = llmi::SafetensorsFile::parse(rm->bytes);
  if (!st) {
    g_err = st.error();
    return nullptr;
  }
  auto model = llmi::Model::from_parts(*parsed, std::move(st.value()));
  if (!model) {
    g_err = model.error();
    return nullptr;
  }
  auto tf = llmi::Transformer::load(*model, static_cast<llmi::quant::Type>(type));
  if (!tf) {
    g_err = tf.error();
    return nullptr;
  }
  rm->tf = std::make_unique<llmi::Transformer>(std::move(tf.value()));
  rm->vocab = cfg->vocab_size;
  // The quantized Transformer no longer reads the safetensors bytes.
  std::vector<std::byte>().swap(rm->bytes);
  return rm.release();
}

void ref_model_free(void* m) { delete static_cast<RefModel*>(m); }

std::size_t ref_model_weight_bytes(void* m) { return static_cast<RefModel*>(m)->tf->weight_bytes(); }

int ref_model_new_cache(void* m, std::size_t max_len) {
  auto* rm = static_cast<RefModel*>(m);
  auto c = rm->tf->new_cache(max_len);
  if (!c) {
    g_err = c.error();
    return 1;
  }
  rm->cache = std::make_unique<llmi::KVCache>(std::move(c.value()));
  return 0;
}

std::size_t ref_model_cache_length(void* m) {
  auto* rm = static_cast<RefModel*>(m);
  return rm->cache ? rm->cache->length() : 0;
}

int ref_model_forward_cached(void* m, const std::int32_t* tokens, std::size_t n, int all_positions, float* logits) {
  auto* rm = static_cast<RefModel*>(m);
  if (!rm->cache) {
    g_err = "no cache";
    return 1;
  }
  auto r = rm->tf->forward_cached(std::vector<llmi::TokenId>(tokens, tokens + n), *rm->cache, all_positions != 0);
  if (!r) {
    g_err = r.error();
    return 1;
  }
  std::memcpy(logits, r->data(), r->size() * sizeof(float));
  return 0;
}

int ref_model_forward(void* m, const std::int32_t* tokens, std::size_t n, int all_positions, float* logits) {
  auto* rm = static_cast<RefModel*>(m);
  auto r = rm->tf->forward(std::vector<llmi::TokenId>(tokens, tokens + n), all_positions != 0);
  if (!r) {
    g_err = r.error();
    return 1;
  }
  std::memcpy(logits, r->data(), r->size() * sizeof(float));
  return 0;
}

// transformer.cpp:308-327, step by step so the top-1/top-2 margin of every
// step can be recorded (ids are exactly generate_greedy_cached's).
int ref_generate_greedy_cached(void* m, const std::int32_t* prompt, std::size_t n, std::size_t max_new,
                               std::int32_t* ids, float* margins) {
  auto* rm = static_cast<RefModel*>(m);
  if (ref_model_new_cache(m, n + max_new) != 0) return 1;
  std::vector<float> logits(rm->vocab);
  if (ref_model_forward_cached(m, prompt, n, 0, logits.data()) != 0) return 1;
  for (std::size_t step = 0; step < max_new; ++step) {
    const std::size_t best = llmi::argmax(logits.data(), logits.size());
    float second = -INFINITY;
    for (std::size_t i = 0; i < logits.size(); ++i)
      if (i != best && logits[i] > second) second = logits[i];
    ids[step] = static_cast<std::int32_t>(best);
    if (margins != nullptr) margins[step] = logits[best] - second;
    if (step + 1 == max_new) break;
    const std::int32_t next = ids[step];
    if (ref_model_forward_cached(m, &next, 1, 0, logits.data()) != 0) return 1;
  }
  return 0;
}

// The reference's gguf::to_quantized (gguf.cpp:577-640) on one tensor "w"
// of type gtype and shape [out][in], given its raw blocks: a minimal GGUF v3
// image (no metadata, one tensor at offset 0, default alignment 32) is
// parsed with GGUFFile::parse and converted.  Returns 0, or 1 with the
// reference's error message.
int ref_gguf_to_quantized(const std::uint8_t* raw, std::size_t nbytes, std::size_t out, std::size_t in, int gtype,
                          std::uint8_t* data, float* scales) {
  std::vector<std::byte> img;
  const auto put = [&](std::uint64_t v, int n) {
    for (int k = 0; k < n; ++k) img.push_back(static_cast<std::byte>((v >> (8 * k)) & 0xFFU));
  };
  for (char c : {'G', 'G', 'U', 'F'}) img.push_back(static_cast<std::byte>(c));
  put(3, 4);           // version
  put(1, 8);           // tensors
  put(0, 8);           // metadata entries
  put(1, 8);           // name length
  img.push_back(static_cast<std::byte>('w'));
  put(2, 4);           // dimensions, fastest first
  put(in, 8);
  put(out, 8);
  put(static_cast<std::uint64_t>(gtype), 4);
  put(0, 8);           // offset in the data section
  while (img.size() % 32 != 0) img.push_back(std::byte{0});
  for (std::size_t i = 0; i < nbytes; ++i) img.push_back(static_cast<std::byte>(raw[i]));
  auto f = llmi::gguf::GGUFFile::parse(img);
  if (!f) {
    g_err = f.error();
    return 1;
  }
  const auto* t = f->find("w");
  if (t == nullptr) {
    g_err = "tensor w not found";
    return 1;
  }
  auto m = llmi::gguf::to_quantized(*f, *t, out, in);
  if (!m) {
    g_err = m.error();
    return 1;
  }
  std::memcpy(data, m->data.data(), m->data.size());
  std::memcpy(scales, m->scales.data(), m->scales.size() * sizeof(float));
  return 0;
}

}  // extern "C"
