// ============================================================================
// TEST INFRASTRUCTURE ONLY -- not part of the product.
//
// CPU restatement of llm-inference-cpp's quantized-weight path, used as the
// parity oracle by tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg.  Nothing in llm-inference-cpp_amd/ links, loads or calls
// this file.
//
// Every function cites the reference source it restates.  The reference is
// built with `-O3 -mavx2 -mfma` (g++, C++20), which contracts a*b+c into a
// single fused multiply-add; the restatement writes those contractions out
// with std::fma, so its bits do not depend on the flags it is compiled with.
// The contraction pattern was read from x86 assembly of the reference built
// in this container (quant.cpp, kernels.cpp, transformer.cpp).
//
// Parity pins (tests/test_oracle.py):
//   quantize / dequantize_row / matmul: golden vectors from the compiled
//     reference (tests/golden), the reference's own known-answer tests
//     (quant_test.cpp:85-112, gguf_test.cpp:389-453 codes), round-trip bounds
//     and an fp64 brute-force dot product.
//   dot / rmsnorm / rope / softmax / silu: golden vectors from the compiled
//     reference plus the reference's own kernel tests
//     (transformer_test.cpp:15-144).
//   forward_cached / generate_greedy_cached: golden logits and greedy ids of
//     the compiled reference on synthetic models.
//   sampling_probabilities / sample_with_target / draw_uniform: the compiled
//     reference's sampling_probabilities and sample() (same generator seed),
//     its own sampling tests (sampling_test.cpp), a plain double softmax, the
//     standard's mt19937_64 known answer and the uniform mapping's closed form
//     (tests/test_oracle_sampling.py).
// ============================================================================

#include <algorithm>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "../include/llmi_hip.h"

namespace oracle {

constexpr std::size_t kBlock = 32;                // quant.hpp:15
constexpr std::size_t kMinWorkForThreading = 200000;  // quant.cpp:16, kernels.cpp:32

enum : int { kF32 = 0, kQ8 = 1, kQ4 = 2 };  // quant.hpp:17

std::size_t row_bytes(std::size_t in, int type) { return type == kQ4 ? (in + 1) / 2 : in; }  // quant.cpp:18-20

// ---------------------------------------------------------------- thread pool
// Restates util::ThreadPool (thread_pool.cpp:7-85): hardware_concurrency()-1
// persistent workers plus the calling thread, [0,n) cut into workers+1
// contiguous chunks of ceil(n/slots), run inline when n < min_total_work or
// when there are no workers.  Only the CPU-baseline timing depends on it; the
// arithmetic of every chunk is the same as the serial loop.
class Pool {
 public:
  explicit Pool(std::size_t workers) {
    for (std::size_t i = 0; i < workers; ++i) threads_.emplace_back([this, i] { loop(i); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> g(mu_);
      quit_ = true;
    }
    go_.notify_all();
    for (auto& t : threads_) t.join();
  }
  std::size_t workers() const { return threads_.size(); }

  void parallel_for(std::size_t n, std::size_t min_work, const std::function<void(std::size_t, std::size_t)>& fn) {
    if (n == 0) return;
    if (threads_.empty() || n < min_work) {
      fn(0, n);
      return;
    }
    const std::size_t slots = threads_.size() + 1;
    const std::size_t chunk = (n + slots - 1) / slots;
    {
      std::lock_guard<std::mutex> g(mu_);
      spans_.clear();
      for (std::size_t s = 0; s < threads_.size(); ++s) spans_.emplace_back(std::min(s * chunk, n), std::min((s + 1) * chunk, n));
      job_ = &fn;
      left_ = threads_.size();
      ++epoch_;
    }
    go_.notify_all();
    const std::size_t s = threads_.size();
    fn(std::min(s * chunk, n), std::min((s + 1) * chunk, n));
    std::unique_lock<std::mutex> lk(mu_);
    done_.wait(lk, [&] { return left_ == 0; });
  }

 private:
  void loop(std::size_t me) {
    std::size_t seen = 0;
    for (;;) {
      std::pair<std::size_t, std::size_t> span;
      const std::function<void(std::size_t, std::size_t)>* job = nullptr;
      {
        std::unique_lock<std::mutex> lk(mu_);
        go_.wait(lk, [&] { return quit_ || epoch_ != seen; });
        if (quit_) return;
        seen = epoch_;
        span = spans_[me];
        job = job_;
      }
      (*job)(span.first, span.second);
      std::lock_guard<std::mutex> g(mu_);
      if (--left_ == 0) done_.notify_one();
    }
  }

  std::vector<std::thread> threads_;
  std::mutex mu_;
  std::condition_variable go_, done_;
  std::vector<std::pair<std::size_t, std::size_t>> spans_;
  const std::function<void(std::size_t, std::size_t)>* job_ = nullptr;
  std::size_t epoch_ = 0, left_ = 0;
  bool quit_ = false;
};

std::unique_ptr<Pool>& pool_slot() {
  static std::unique_ptr<Pool> pool;
  return pool;
}

Pool& shared_pool() {  // thread_pool.cpp:7-15 (size overridable for timing)
  auto& p = pool_slot();
  if (!p) {
    const unsigned hw = std::thread::hardware_concurrency();
    p = std::make_unique<Pool>(hw > 1 ? static_cast<std::size_t>(hw) - 1 : std::size_t{0});
  }
  return *p;
}

Pool& serial_pool() {
  static Pool pool(0);
  return pool;
}

// ------------------------------------------------------------------- quant
// quant.cpp:36-102.  Per 32-weight block: amax and the signed value at the
// FIRST index reaching it (strict >), Q8 scale amax/127, Q4 scale
// extreme/-8, an all-zero block gets scale 1, codes are
// clamp(lround(double(v)/double(scale))), Q4 nibbles carry +8 and pack two
// per byte by row-global index (even index in the low nibble).
void quantize(const float* w, std::size_t out, std::size_t in, int type, std::uint8_t* data, float* scales) {
  const std::size_t nb = (in + kBlock - 1) / kBlock;
  const std::size_t rb = row_bytes(in, type);
  std::memset(data, 0, out * rb);
  const int hi = type == kQ4 ? 7 : 127;
  const int lo = type == kQ4 ? -8 : -127;
  for (std::size_t r = 0; r < out; ++r) {
    const float* src = w + r * in;
    std::uint8_t* dst = data + r * rb;
    for (std::size_t b = 0; b < nb; ++b) {
      const std::size_t first = b * kBlock;
      const std::size_t n = std::min(kBlock, in - first);
      float peak = 0.0F;
      float peak_signed = 0.0F;
      for (std::size_t i = 0; i < n; ++i) {
        const float mag = std::fabs(src[first + i]);
        if (mag > peak) {
          peak = mag;
          peak_signed = src[first + i];
        }
      }
      float d = type == kQ4 ? peak_signed / -8.0F : peak / 127.0F;
      if (d == 0.0F) d = 1.0F;
      scales[r * nb + b] = d;
      for (std::size_t i = 0; i < n; ++i) {
        const std::size_t k = first + i;
        int q = static_cast<int>(std::lround(static_cast<double>(src[k]) / static_cast<double>(d)));
        q = std::min(std::max(q, lo), hi);
        if (type == kQ8) {
          dst[k] = static_cast<std::uint8_t>(static_cast<std::int8_t>(q));
        } else {
          const std::uint8_t nib = static_cast<std::uint8_t>(q + 8);
          dst[k / 2] = (k % 2 == 0) ? static_cast<std::uint8_t>((dst[k / 2] & 0xF0U) | nib)
                                    : static_cast<std::uint8_t>((dst[k / 2] & 0x0FU) | (nib << 4U));
        }
      }
    }
  }
}

inline float code_at(const std::uint8_t* row, std::size_t k, int type) {
  if (type == kQ8) return static_cast<float>(static_cast<std::int8_t>(row[k]));
  const std::uint8_t byte = row[k / 2];
  const int nib = (k % 2 == 0) ? (byte & 0x0F) : (byte >> 4);
  return static_cast<float>(nib - 8);
}

// quant.cpp:104-117: dst[k] = code_k * scale[k/32], one rounding.
void dequantize_row(const std::uint8_t* data, const float* scales, std::size_t in, int type, std::size_t row, float* dst) {
  const std::size_t nb = (in + kBlock - 1) / kBlock;
  const std::uint8_t* q = data + row * row_bytes(in, type);
  for (std::size_t k = 0; k < in; ++k) dst[k] = code_at(q, k, type) * scales[row * nb + k / kBlock];
}

// quant.cpp:119-153: per output o and input row r, per block a sequential
// fused chain block_sum = fma(x_k, code_k, block_sum), then the sequential
// chain acc = fma(block_sum, scale_b, acc), then y = acc + bias[o].
void matmul(const float* x, std::size_t rows, std::size_t in, const std::uint8_t* data, const float* scales, int type,
            std::size_t out, const float* bias, float* y, Pool& pool) {
  const std::size_t nb = (in + kBlock - 1) / kBlock;
  const std::size_t rb = row_bytes(in, type);
  auto body = [&](std::size_t o0, std::size_t o1) {
    for (std::size_t o = o0; o < o1; ++o) {
      const std::uint8_t* q = data + o * rb;
      const float* s = scales + o * nb;
      const float add = bias != nullptr ? bias[o] : 0.0F;
      for (std::size_t r = 0; r < rows; ++r) {
        const float* xr = x + r * in;
        float acc = 0.0F;
        for (std::size_t b = 0; b < nb; ++b) {
          const std::size_t first = b * kBlock;
          const std::size_t n = std::min(kBlock, in - first);
          float part = 0.0F;
          for (std::size_t i = 0; i < n; ++i) part = std::fma(xr[first + i], code_at(q, first + i, type), part);
          acc = std::fma(part, s[b], acc);
        }
        y[r * out + o] = acc + add;
      }
    }
  };
  pool.parallel_for(out, kMinWorkForThreading / std::max<std::size_t>(rows * in, 1), body);
}

// ----------------------------------------------------------------- kernels
// kernels.cpp:41-50 (dot_scalar): 8 accumulators, fused chains, fixed tree.
// The compiler vectorizes the final `tail` loop (fewer than 8 elements): when
// 4 or more remain, the first 4 products are rounded on their own and added
// in order, and only the last 1-3 elements are fused.
float dot_tail(const float* a, const float* b, std::size_t n) {
  float acc[8] = {};
  std::size_t i = 0;
  for (; i + 8 <= n; i += 8)
    for (std::size_t k = 0; k < 8; ++k) acc[k] = std::fma(a[i + k], b[i + k], acc[k]);
  float tail = 0.0F;
  if (n - i >= 4) {
    for (std::size_t k = 0; k < 4; ++k) {
      const float p = a[i + k] * b[i + k];
      tail = tail + p;
    }
    i += 4;
  }
  for (; i < n; ++i) tail = std::fma(a[i], b[i], tail);
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7])) + tail;
}

// kernels.cpp:56-74 (the AVX2 build): 16 fused lanes over 16-element chunks,
// then (lane j + lane j+8), (+4), (+2), (+1), then + dot_scalar(rest).
float dot(const float* a, const float* b, std::size_t n) {
  float lane[16] = {};
  std::size_t i = 0;
  for (; i + 16 <= n; i += 16)
    for (std::size_t j = 0; j < 16; ++j) lane[j] = std::fma(a[i + j], b[i + j], lane[j]);
  float s8[8], s4[4];
  for (int j = 0; j < 8; ++j) s8[j] = lane[j] + lane[j + 8];
  for (int j = 0; j < 4; ++j) s4[j] = s8[j] + s8[j + 4];
  const float t0 = s4[0] + s4[2];
  const float t1 = s4[1] + s4[3];
  return (t0 + t1) + dot_tail(a + i, b + i, n - i);
}

// kernels.cpp:115-120: sum of squares in double (fused, exact squares),
// scale rounded to float once, y = w * (x * scale).
void rmsnorm(const float* x, const float* w, std::size_t n, float eps, float* y) {
  double ss = 0.0;
  for (std::size_t i = 0; i < n; ++i) ss = std::fma(static_cast<double>(x[i]), static_cast<double>(x[i]), ss);
  const float scale = static_cast<float>(1.0 / std::sqrt(ss / static_cast<double>(n) + static_cast<double>(eps)));
  for (std::size_t i = 0; i < n; ++i) y[i] = w[i] * (x[i] * scale);
}

// kernels.cpp:122-134: float angle pos*inv_freq[i], sincosf, rotate-half with
// the contraction the compiler emits: v[i] = fma(a, c, -(b*s)),
// v[i+half] = fma(b, c, a*s).
void rope(float* v, std::size_t hd, std::size_t pos, const float* inv_freq) {
  const std::size_t half = hd / 2;
  for (std::size_t i = 0; i < half; ++i) {
    const float angle = static_cast<float>(pos) * inv_freq[i];
    float s = 0.0F, c = 0.0F;
    sincosf(angle, &s, &c);
    const float a = v[i];
    const float b = v[i + half];
    v[i] = std::fma(a, c, -(b * s));
    v[i + half] = std::fma(b, c, a * s);
  }
}

// kernels.cpp:136-146: float max, float expf, double running sum,
// x *= float(1/sum).
void softmax(float* x, std::size_t n) {
  if (n == 0) return;
  float mx = x[0];
  for (std::size_t i = 1; i < n; ++i)
    if (mx < x[i]) mx = x[i];
  double sum = 0.0;
  for (std::size_t i = 0; i < n; ++i) {
    x[i] = expf(x[i] - mx);
    sum += static_cast<double>(x[i]);
  }
  const float inv = static_cast<float>(1.0 / sum);
  for (std::size_t i = 0; i < n; ++i) x[i] *= inv;
}

float silu(float v) { return v / (1.0F + expf(-v)); }  // kernels.cpp:148

std::size_t argmax(const float* x, std::size_t n) {  // transformer.cpp:22-24: first maximum
  std::size_t best = 0;
  for (std::size_t i = 1; i < n; ++i)
    if (x[best] < x[i]) best = i;
  return best;
}

// ---------------------------------------------------------------- sampling
// src/model/sampling.cpp:11-58 (sampling_probabilities).  temperature <= 0:
// all mass on the first maximum.  Otherwise: each logit divided by the
// temperature in float, kernels::softmax, the entries ranked by probability
// (descending; equal probabilities keep index order, as std::stable_sort
// does), top-k, then the top-p nucleus -- the shortest prefix of the ranking
// whose double running sum reaches double(top_p), at least one entry -- and
// the kept entries divided by their double sum taken in ranking order.
std::vector<float> sampling_probabilities(const float* logits, std::size_t n, float temperature, std::size_t top_k,
                                          float top_p) {
  std::vector<float> out(n, 0.0F);
  if (temperature <= 0.0F) {
    out[argmax(logits, n)] = 1.0F;
    return out;
  }
  std::vector<float> p(n);
  for (std::size_t i = 0; i < n; ++i) p[i] = logits[i] / temperature;
  softmax(p.data(), n);
  std::vector<std::size_t> rank(n);
  for (std::size_t i = 0; i < n; ++i) rank[i] = i;
  std::stable_sort(rank.begin(), rank.end(), [&p](std::size_t a, std::size_t b) { return p[a] > p[b]; });
  const std::size_t k = top_k == 0 || top_k > n ? n : top_k;
  std::size_t keep = k;
  if (top_p < 1.0F) {
    double run = 0.0;
    for (std::size_t j = 0; j < k; ++j) {
      run += static_cast<double>(p[rank[j]]);
      if (run >= static_cast<double>(top_p)) {
        keep = j + 1;
        break;
      }
    }
    if (keep == 0) keep = 1;
  }
  double total = 0.0;
  for (std::size_t j = 0; j < keep; ++j) {
    out[rank[j]] = p[rank[j]];
    total += static_cast<double>(p[rank[j]]);
  }
  if (total > 0.0)
    for (float& v : out) v = static_cast<float>(static_cast<double>(v) / total);
  return out;
}

// sampling.cpp:60-77 (sample) with its random number given: target is what
// std::uniform_real_distribution<double>(0, 1) drew from the caller's
// generator.  The first index whose double running sum (in index order) of
// the filtered probabilities reaches target; else the last nonzero entry;
// else the first maximum.  temperature <= 0 draws nothing: the first maximum.
std::size_t sample_with_target(const float* logits, std::size_t n, float temperature, std::size_t top_k, float top_p,
                               double target) {
  if (temperature <= 0.0F) return argmax(logits, n);
  const std::vector<float> f = sampling_probabilities(logits, n, temperature, top_k, top_p);
  double run = 0.0;
  for (std::size_t i = 0; i < n; ++i) {
    run += static_cast<double>(f[i]);
    if (run >= target) return i;
  }
  for (std::size_t i = n; i-- > 0;)
    if (f[i] > 0.0F) return i;
  return argmax(logits, n);
}

// ------------------------------------------------------------------- model
struct Mat {  // weight.hpp:18-39: fp32 or block-quantized
  int type = kF32;
  std::size_t out = 0, in = 0;
  std::vector<float> f32, scales;
  std::vector<std::uint8_t> q;

  void set(const float* w, std::size_t o, std::size_t i, int t) {
    type = t;
    out = o;
    in = i;
    if (t == kF32) {
      f32.assign(w, w + o * i);
    } else {
      q.resize(o * row_bytes(i, t));
      scales.resize(o * ((i + kBlock - 1) / kBlock));
      quantize(w, o, i, t, q.data(), scales.data());
    }
  }
  // weight.cpp:30-37: quantized -> quant::matmul; fp32 -> kernels::matmul
  // (kernels.cpp:97-113: y = dot(x_r, w_o) + bias).
  void mm(const float* x, std::size_t rows, const float* bias, float* y, Pool& pool) const {
    if (type != kF32) {
      matmul(x, rows, in, q.data(), scales.data(), type, out, bias, y, pool);
      return;
    }
    auto body = [&](std::size_t o0, std::size_t o1) {
      for (std::size_t o = o0; o < o1; ++o) {
        const float add = bias != nullptr ? bias[o] : 0.0F;
        for (std::size_t r = 0; r < rows; ++r) y[r * out + o] = dot(x + r * in, f32.data() + o * in, in) + add;
      }
    };
    pool.parallel_for(out, kMinWorkForThreading / std::max<std::size_t>(rows * in, 1), body);
  }
  void row(std::size_t idx, float* dst) const {  // weight.cpp:39-45
    if (type == kF32) {
      std::copy_n(f32.data() + idx * in, in, dst);
    } else {
      dequantize_row(q.data(), scales.data(), in, type, idx, dst);
    }
  }
};

struct Layer {
  std::vector<float> attn_norm, bq, bk, bv, mlp_norm;
  Mat wq, wk, wv, wo, gate, up, down;
};

struct Model {
  llmi_model_config c{};
  Mat embed, lm_head;
  std::vector<float> final_norm, inv_freq;
  std::vector<Layer> layers;
  // KVCache (transformer.hpp:29-45): head-major [layer][kv_head][cap][hd].
  std::size_t cap = 0, len = 0;
  std::vector<std::vector<float>> kc, vc;
  bool threaded = true;
  std::string err;
};

// transformer.cpp:26-67 (load) with tensors in model.cpp:135-162 order.
Model* create(const llmi_model_config* cfg, const float* const* t, int type) {
  auto m = std::make_unique<Model>();
  m->c = *cfg;
  const auto& c = m->c;
  const std::size_t H = c.hidden_size, hd = H / c.num_heads, Q = c.num_heads * hd, KV = c.num_kv_heads * hd,
                    F = c.intermediate_size, V = c.vocab_size;
  std::size_t k = 0;
  m->embed.set(t[k++], V, H, type);
  m->layers.resize(c.num_layers);
  for (auto& l : m->layers) {
    l.attn_norm.assign(t[k], t[k] + H);
    ++k;
    l.wq.set(t[k++], Q, H, type);
    l.wk.set(t[k++], KV, H, type);
    l.wv.set(t[k++], KV, H, type);
    if (c.qkv_bias) {
      l.bq.assign(t[k], t[k] + Q);
      ++k;
      l.bk.assign(t[k], t[k] + KV);
      ++k;
      l.bv.assign(t[k], t[k] + KV);
      ++k;
    }
    l.wo.set(t[k++], H, Q, type);
    l.mlp_norm.assign(t[k], t[k] + H);
    ++k;
    l.gate.set(t[k++], F, H, type);
    l.up.set(t[k++], F, H, type);
    l.down.set(t[k++], H, F, type);
  }
  m->final_norm.assign(t[k], t[k] + H);
  ++k;
  if (!c.tie_word_embeddings) m->lm_head.set(t[k++], V, H, type);
  m->inv_freq.resize(hd / 2);
  for (std::size_t i = 0; i < hd / 2; ++i) {
    const float e = static_cast<float>(2 * i) / static_cast<float>(hd);
    m->inv_freq[i] = 1.0F / std::pow(static_cast<float>(c.rope_theta), e);
  }
  return m.release();
}

// transformer.cpp:182-190
bool new_cache(Model& m, std::size_t max_len) {
  m.cap = std::min<std::size_t>(max_len, m.c.max_position_embeddings);
  m.len = 0;
  if (m.cap == 0) {
    m.err = "new_cache: max_len must be positive";
    return false;
  }
  const std::size_t per = static_cast<std::size_t>(m.c.num_kv_heads) * (m.c.hidden_size / m.c.num_heads);
  m.kc.assign(m.c.num_layers, std::vector<float>(m.cap * per));
  m.vc.assign(m.c.num_layers, std::vector<float>(m.cap * per));
  return true;
}

// transformer.cpp:192-306
bool forward_cached(Model& m, const std::int32_t* tokens, std::size_t T, bool all_positions, float* logits) {
  const auto& c = m.c;
  const std::size_t H = c.hidden_size, nh = c.num_heads, nkv = c.num_kv_heads, hd = H / nh, group = nh / nkv,
                    F = c.intermediate_size, V = c.vocab_size;
  const float eps = static_cast<float>(c.rms_norm_eps);
  Pool& pool = m.threaded ? shared_pool() : serial_pool();
  if (T == 0) return m.err = "forward_cached: no tokens", false;
  if (m.kc.size() != c.num_layers) return m.err = "forward_cached: cache was not created by this model", false;
  const std::size_t base = m.len;
  if (base + T > m.cap) return m.err = "forward_cached: cache is full", false;
  if (base + T > c.max_position_embeddings) return m.err = "forward_cached: sequence longer than the model's context", false;
  for (std::size_t t = 0; t < T; ++t)
    if (tokens[t] < 0 || static_cast<std::size_t>(tokens[t]) >= V)
      return m.err = "forward_cached: token id " + std::to_string(tokens[t]) + " out of range", false;

  std::vector<float> x(T * H), h(T * H), q(T * nh * hd), att(T * nh * hd), proj(T * H), g(T * F), u(T * F),
      sc(base + T), kn(T * nkv * hd), vn(T * nkv * hd);
  for (std::size_t t = 0; t < T; ++t) m.embed.row(static_cast<std::size_t>(tokens[t]), x.data() + t * H);
  const std::size_t cap = m.cap;
  const float scale = 1.0F / std::sqrt(static_cast<float>(hd));
  for (std::size_t li = 0; li < m.layers.size(); ++li) {
    const Layer& l = m.layers[li];
    float* kcache = m.kc[li].data();
    float* vcache = m.vc[li].data();
    for (std::size_t t = 0; t < T; ++t) rmsnorm(x.data() + t * H, l.attn_norm.data(), H, eps, h.data() + t * H);
    l.wq.mm(h.data(), T, l.bq.empty() ? nullptr : l.bq.data(), q.data(), pool);
    l.wk.mm(h.data(), T, l.bk.empty() ? nullptr : l.bk.data(), kn.data(), pool);
    l.wv.mm(h.data(), T, l.bv.empty() ? nullptr : l.bv.data(), vn.data(), pool);
    for (std::size_t t = 0; t < T; ++t) {
      for (std::size_t hh = 0; hh < nh; ++hh) rope(q.data() + (t * nh + hh) * hd, hd, base + t, m.inv_freq.data());
      for (std::size_t hh = 0; hh < nkv; ++hh) rope(kn.data() + (t * nkv + hh) * hd, hd, base + t, m.inv_freq.data());
    }
    for (std::size_t t = 0; t < T; ++t)
      for (std::size_t kvh = 0; kvh < nkv; ++kvh) {
        std::copy_n(kn.data() + (t * nkv + kvh) * hd, hd, kcache + (kvh * cap + base + t) * hd);
        std::copy_n(vn.data() + (t * nkv + kvh) * hd, hd, vcache + (kvh * cap + base + t) * hd);
      }
    for (std::size_t hh = 0; hh < nh; ++hh) {
      const std::size_t kvh = hh / group;
      const float* kh = kcache + kvh * cap * hd;
      const float* vh = vcache + kvh * cap * hd;
      for (std::size_t t = 0; t < T; ++t) {
        const std::size_t pos = base + t;
        const float* qv = q.data() + (t * nh + hh) * hd;
        for (std::size_t s = 0; s <= pos; ++s) sc[s] = dot(qv, kh + s * hd, hd) * scale;
        softmax(sc.data(), pos + 1);
        float* o = att.data() + (t * nh + hh) * hd;
        std::fill_n(o, hd, 0.0F);
        for (std::size_t s = 0; s <= pos; ++s)
          for (std::size_t i = 0; i < hd; ++i) o[i] = std::fma(sc[s], vh[s * hd + i], o[i]);
      }
    }
    l.wo.mm(att.data(), T, nullptr, proj.data(), pool);
    for (std::size_t i = 0; i < T * H; ++i) x[i] += proj[i];
    for (std::size_t t = 0; t < T; ++t) rmsnorm(x.data() + t * H, l.mlp_norm.data(), H, eps, h.data() + t * H);
    l.gate.mm(h.data(), T, nullptr, g.data(), pool);
    l.up.mm(h.data(), T, nullptr, u.data(), pool);
    for (std::size_t i = 0; i < T * F; ++i) g[i] = silu(g[i]) * u[i];
    l.down.mm(g.data(), T, nullptr, proj.data(), pool);
    for (std::size_t i = 0; i < T * H; ++i) x[i] += proj[i];
  }
  m.len = base + T;
  for (std::size_t t = 0; t < T; ++t) rmsnorm(x.data() + t * H, m.final_norm.data(), H, eps, h.data() + t * H);
  const Mat& head = m.c.tie_word_embeddings ? m.embed : m.lm_head;
  const std::size_t first = all_positions ? 0 : T - 1;
  head.mm(h.data() + first * H, T - first, nullptr, logits, pool);
  return true;
}

// ------------------------------------------------------------ GGUF blocks
// src/model/safetensors.cpp:249-273 (half_to_float): IEEE binary16 ->
// binary32; zero keeps its sign, subnormals are normalised, infinities and
// NaNs keep their payload bits.
float half_to_float(std::uint16_t h) {
  const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000U) << 16U;
  const std::uint32_t e = (h >> 10U) & 0x1FU;
  std::uint32_t m = h & 0x3FFU;
  std::uint32_t bits = sign;
  if (e == 0x1FU) {
    bits |= 0x7F800000U | (m << 13U);
  } else if (e != 0) {
    bits |= ((e + 112U) << 23U) | (m << 13U);
  } else if (m != 0) {
    // value m * 2^-24: shift the leading one up to bit 10.
    std::uint32_t exp32 = 113;  // biased exponent of 2^-14
    while ((m & 0x400U) == 0) {
      m <<= 1U;
      --exp32;
    }
    bits |= (exp32 << 23U) | ((m & 0x3FFU) << 13U);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// src/model/gguf.cpp:577-640 (to_quantized), the checks in its order, then
// each ggml block {fp16 d; codes} into the engine layout: the scale through
// half_to_float; Q8_0 codes in order; Q4_0 byte j of the block holds element
// j (low nibble) and element j + 16 (high nibble), and each element's nibble
// (code + 8) goes to the engine's neighbour pairs (even element low nibble).
// gtype: GGUF tensor type (2 = Q4_0, 8 = Q8_0).  Returns false with a
// message on the reference's failure cases.
bool gguf_to_quantized(const std::uint8_t* raw, std::size_t nbytes, std::size_t out, std::size_t in, int gtype,
                       std::uint8_t* data, float* scales, std::string* err) {
  int type = 0;
  std::size_t qbytes = 0;
  if (gtype == 8) {
    type = kQ8;
    qbytes = kBlock;
  } else if (gtype == 2) {
    type = kQ4;
    qbytes = kBlock / 2;
  } else {
    *err = "not Q8_0/Q4_0";
    return false;
  }
  if (out == 0 || in == 0) {
    *err = "out*in does not match its element count";
    return false;
  }
  if (in % kBlock != 0) {
    *err = "in is not a multiple of the block size";
    return false;
  }
  const std::size_t bpr = in / kBlock, bb = 2 + qbytes;
  if (nbytes != out * bpr * bb) {
    *err = "unexpected byte size for its declared shape";
    return false;
  }
  const std::size_t rb = row_bytes(in, type);
  std::memset(data, 0, out * rb);
  for (std::size_t r = 0; r < out; ++r) {
    for (std::size_t b = 0; b < bpr; ++b) {
      const std::uint8_t* blk = raw + (r * bpr + b) * bb;
      scales[r * bpr + b] = half_to_float(static_cast<std::uint16_t>(blk[0] | (blk[1] << 8U)));
      std::uint8_t* row = data + r * rb;
      if (type == kQ8) {
        std::memcpy(row + b * kBlock, blk + 2, kBlock);
        continue;
      }
      for (std::size_t e = 0; e < kBlock; ++e) {
        const std::uint8_t byte = blk[2 + (e % 16)];
        const std::uint8_t nib = e < 16 ? (byte & 0x0FU) : static_cast<std::uint8_t>(byte >> 4U);
        const std::size_t idx = b * kBlock + e;
        row[idx / 2] |= static_cast<std::uint8_t>(idx % 2 == 0 ? nib : nib << 4U);
      }
    }
  }
  return true;
}

}  // namespace oracle

namespace {
thread_local std::string g_err;
}

extern "C" {

const char* oracle_last_error() { return g_err.c_str(); }
int oracle_gguf_to_quantized(const std::uint8_t* raw, std::size_t nbytes, std::size_t out, std::size_t in, int gtype,
                             std::uint8_t* data, float* scales) {
  return oracle::gguf_to_quantized(raw, nbytes, out, in, gtype, data, scales, &g_err) ? 0 : 1;
}
std::size_t oracle_row_bytes(std::size_t in, int type) { return oracle::row_bytes(in, type); }

void oracle_quantize(const float* w, std::size_t out, std::size_t in, int type, std::uint8_t* data, float* scales) {
  oracle::quantize(w, out, in, type, data, scales);
}
void oracle_dequantize_row(const std::uint8_t* data, const float* scales, std::size_t in, int type, std::size_t row,
                           float* dst) {
  oracle::dequantize_row(data, scales, in, type, row, dst);
}
// threads: 0 -> the reference's default pool (hardware_concurrency()-1 workers
// plus the caller); 1 -> the calling thread only.
void oracle_matmul(const float* x, std::size_t rows, std::size_t in, const std::uint8_t* data, const float* scales,
                   int type, std::size_t out, const float* bias, float* y, int threads) {
  oracle::matmul(x, rows, in, data, scales, type, out, bias, y, threads == 1 ? oracle::serial_pool() : oracle::shared_pool());
}
int oracle_pool_workers() { return static_cast<int>(oracle::shared_pool().workers()); }
// Replaces the shared pool by one with `workers` worker threads (plus the
// calling thread), e.g. to match the host cores granted to the process.
void oracle_set_pool_workers(int workers) {
  oracle::pool_slot() = std::make_unique<oracle::Pool>(static_cast<std::size_t>(workers < 0 ? 0 : workers));
}
float oracle_dot(const float* a, const float* b, std::size_t n) { return oracle::dot(a, b, n); }
void oracle_rmsnorm(const float* x, const float* w, std::size_t n, float eps, float* y) { oracle::rmsnorm(x, w, n, eps, y); }
void oracle_rope(float* v, std::size_t hd, std::size_t pos, const float* inv_freq) { oracle::rope(v, hd, pos, inv_freq); }
void oracle_softmax(float* x, std::size_t n) { oracle::softmax(x, n); }
float oracle_silu(float v) { return oracle::silu(v); }
std::size_t oracle_argmax(const float* x, std::size_t n) { return oracle::argmax(x, n); }

// n >= 1 (the reference indexes an empty vector otherwise).
void oracle_sampling_probabilities(const float* logits, std::size_t n, float temperature, std::size_t top_k,
                                   float top_p, float* out) {
  const std::vector<float> f = oracle::sampling_probabilities(logits, n, temperature, top_k, top_p);
  std::memcpy(out, f.data(), n * sizeof(float));
}
std::size_t oracle_sample_target(const float* logits, std::size_t n, float temperature, std::size_t top_k, float top_p,
                                 double target) {
  return oracle::sample_with_target(logits, n, temperature, top_k, top_p, target);
}
// The numbers sample() draws (sampling.cpp:64-65): `count` successive
// std::uniform_real_distribution<double>(0, 1) draws from
// std::mt19937_64(seed) -- the standard library's generator and mapping, as
// the reference's build uses them.
void oracle_draw_uniform(std::uint64_t seed, std::size_t count, double* out) {
  std::mt19937_64 rng(seed);
  std::uniform_real_distribution<double> u(0.0, 1.0);
  for (std::size_t i = 0; i < count; ++i) out[i] = u(rng);
}

void* oracle_model_create(const llmi_model_config* cfg, const float* const* tensors, int type) {
  return oracle::create(cfg, tensors, type);
}
void oracle_model_free(void* m) { delete static_cast<oracle::Model*>(m); }
void oracle_model_set_threaded(void* m, int on) { static_cast<oracle::Model*>(m)->threaded = on != 0; }
int oracle_model_new_cache(void* m, std::size_t max_len) {
  auto* mm = static_cast<oracle::Model*>(m);
  if (!oracle::new_cache(*mm, max_len)) {
    g_err = mm->err;
    return 1;
  }
  return 0;
}
std::size_t oracle_model_cache_length(void* m) { return static_cast<oracle::Model*>(m)->len; }
int oracle_model_forward_cached(void* m, const std::int32_t* tokens, std::size_t n, int all_positions, float* logits) {
  auto* mm = static_cast<oracle::Model*>(m);
  if (!oracle::forward_cached(*mm, tokens, n, all_positions != 0, logits)) {
    g_err = mm->err;
    return 1;
  }
  return 0;
}

// transformer.cpp:308-327 with no stop ids; margins[i] = top1 - top2 logit of
// the step that produced ids[i] (the reference's crosscheck_forward.py
// reports the same quantity when ids diverge).
int oracle_generate_greedy_cached(void* m, const std::int32_t* prompt, std::size_t n, std::size_t max_new,
                                  std::int32_t* ids, float* margins) {
  auto* mm = static_cast<oracle::Model*>(m);
  const std::size_t V = mm->c.vocab_size;
  if (!oracle::new_cache(*mm, n + max_new)) return g_err = mm->err, 1;
  std::vector<float> logits(V);
  if (!oracle::forward_cached(*mm, prompt, n, false, logits.data())) return g_err = mm->err, 1;
  for (std::size_t step = 0; step < max_new; ++step) {
    const std::size_t best = oracle::argmax(logits.data(), V);
    float second = -INFINITY;
    for (std::size_t i = 0; i < V; ++i)
      if (i != best && logits[i] > second) second = logits[i];
    ids[step] = static_cast<std::int32_t>(best);
    if (margins != nullptr) margins[step] = logits[best] - second;
    if (step + 1 == max_new) break;
    const std::int32_t next = ids[step];
    if (!oracle::forward_cached(*mm, &next, 1, false, logits.data())) return g_err = mm->err, 1;
  }
  return 0;
}

}  // extern "C"
