/*
 * llmi_hip.h -- C ABI of the MI355X (gfx950) quantized-weight path.
 *
 * Every entry point replaces one function of llm-inference-cpp's
 * quantized-weight path; the reference interface each one stands in for is
 * cited beside it (paths relative to the reference repository root).  Plain
 * pointers and sizes only: host pointers unless the name ends in _dev, in
 * which case the pointers are device pointers and the work is queued on
 * `stream` (a hipStream_t; NULL means the library's own stream) without a
 * host synchronisation.
 *
 * Errors: every function returns LLMI_OK (0) or a non-zero LLMI_ERR_* code
 * and leaves a message for llmi_hip_last_error() on the calling thread.  The
 * reference's quant functions have no error channel (they return void and
 * assume valid shapes); here bad shapes, unsupported types and HIP failures
 * are reported instead of being undefined behaviour.
 *
 * Threading: like the reference (include/llmi/util/thread_pool.hpp:18-21,
 * src/server/server.cpp:44-49) calls are not reentrant; serialise them.
 */
#ifndef LLMI_HIP_H
#define LLMI_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  LLMI_OK = 0,
  LLMI_ERR_ARG = 1,   /* bad shape, type, pointer or token id */
  LLMI_ERR_HIP = 2,   /* HIP runtime failure (allocation, launch, copy) */
  LLMI_ERR_STATE = 3, /* not initialised, cache full, cache from another model */
};

/* Weight storage types; the values of llmi::quant::Type
 * (include/llmi/model/quant.hpp:17). */
enum { LLMI_TYPE_F32 = 0, LLMI_TYPE_Q8_0 = 1, LLMI_TYPE_Q4_0 = 2 };

/* Weights per quantization block (include/llmi/model/quant.hpp:15). */
#define LLMI_BLOCK_SIZE 32

/* GGUF tensor types accepted by llmi_hip_weight_from_gguf: the values of
 * llmi::gguf::TensorType (include/llmi/model/gguf.hpp:26-34). */
enum { LLMI_GGUF_Q4_0 = 2, LLMI_GGUF_Q8_0 = 8 };

/* Model hyper-parameters: the fields of llmi::ModelConfig
 * (include/llmi/model/model.hpp:21-36) that the forward pass reads.
 * head_dim = hidden_size / num_heads (src/model/model.cpp:100-105). */
typedef struct llmi_model_config {
  int32_t arch; /* 0 = Llama, 1 = Qwen2 (model.hpp:16) */
  uint32_t vocab_size;
  uint32_t hidden_size;
  uint32_t intermediate_size;
  uint32_t num_layers;
  uint32_t num_heads;
  uint32_t num_kv_heads;
  uint32_t max_position_embeddings;
  double rms_norm_eps;
  double rope_theta;
  int32_t tie_word_embeddings;
  int32_t qkv_bias;
} llmi_model_config;

typedef struct llmi_hip_weight llmi_hip_weight; /* device-resident packed matrix */

/* ----------------------------------------------------------------- runtime */

/* Selects the GPU and creates the library stream.  Must precede every other
 * call except llmi_hip_last_error and llmi_hip_version. */
int llmi_hip_init(int device);
/* Releases the library stream.  Weights stay valid until freed. */
int llmi_hip_shutdown(void);
const char* llmi_hip_last_error(void);
const char* llmi_hip_version(void);
/* The library's stream (hipStream_t), for callers that queue their own work. */
void* llmi_hip_stream(void);
int llmi_hip_synchronize(void);

/* Plain device memory and copies, for callers without an allocator of
 * their own (tests, bench.py).  Copies are synchronous. */
int llmi_hip_malloc(void** ptr, size_t bytes);
int llmi_hip_free(void* ptr);
int llmi_hip_memcpy_h2d(void* dst_dev, const void* src, size_t bytes);
int llmi_hip_memcpy_d2h(void* dst, const void* src_dev, size_t bytes);
/* Device-to-device copy queued on `stream` (a plain copy kernel). */
int llmi_hip_memcpy_d2d(void* dst_dev, const void* src_dev, size_t bytes, void* stream);
int llmi_hip_memset_dev(void* dst_dev, int value, size_t bytes);

/* HIP events on `stream` (NULL = library stream), for kernel timing. */
int llmi_hip_event_create(void** ev);
int llmi_hip_event_destroy(void* ev);
int llmi_hip_event_record(void* ev, void* stream);
int llmi_hip_event_elapsed_ms(void* start, void* stop, float* ms);

/* Captures the work queued on the library stream between begin and end into
 * a HIP graph (hipStreamBeginCapture / hipGraphInstantiate), for callers
 * that replay a fixed sequence of _dev calls (a decode step, a benchmark
 * pass) without per-launch host overhead.  Only _dev entry points may be
 * called while capturing; the captured kernels allocate and clear nothing. */
int llmi_hip_graph_begin(void);
int llmi_hip_graph_end(void** graph);
int llmi_hip_graph_launch(void* graph);
int llmi_hip_graph_destroy(void* graph);

/* Fills dst_dev[i] = float32(mean + std * z_{offset+i}) from the deterministic
 * "synth-v1" stream `seed` (the same values llm-inference-cpp_amd/synth.py
 * produces on the host).  Test and benchmark input generation only. */
int llmi_hip_synth_normal_dev(float* dst_dev, size_t n, uint64_t seed, uint64_t offset, double mean, double stdev,
                              void* stream);

/* ------------------------------------------------------- block quantizer */

/* Bytes of packed codes per row: in (Q8_0) or ceil(in/2) (Q4_0)
 * (src/model/quant.cpp:18-20). */
size_t llmi_hip_row_bytes(size_t in, int type);

/* Replaces llmi::quant::quantize (include/llmi/model/quant.hpp:51,
 * src/model/quant.cpp:36-102), computed on the GPU.  w is the out x in
 * row-major fp32 matrix; data (out * row_bytes) and scales
 * (out * ceil(in/32)) receive the reference's planar layout
 * (QuantizedMatrix::data / ::scales, quant.hpp:38-48), bit-exact. */
int llmi_hip_quantize(const float* w, size_t out, size_t in, int type, uint8_t* data, float* scales);
int llmi_hip_quantize_dev(const float* w_dev, size_t out, size_t in, int type, uint8_t* data_dev, float* scales_dev,
                          void* stream);

/* ------------------------------------------------ device-resident weights */

/* Uploads a QuantizedMatrix (planar data + scales, as produced by
 * quant::quantize) and re-lays it out for the GPU kernels.  Stands in for the
 * storage of llmi::Weight (include/llmi/model/weight.hpp:18-39,
 * src/model/weight.cpp:16-22). */
int llmi_hip_weight_upload(const uint8_t* data, const float* scales, size_t out, size_t in, int type,
                           llmi_hip_weight** weight);
/* Weight::quantized (src/model/weight.cpp:16-22): quantizes an fp32 matrix on
 * the GPU straight into the device layout.  w is a host pointer.  With
 * LLMI_TYPE_F32 the matrix is kept as fp32 (Weight::from_float,
 * weight.cpp:9-14) and products run kernels::matmul (kernels.cpp:97-113):
 * y = dot(x_r, w_o) + bias with the reference's dot arithmetic, bit-exact. */
int llmi_hip_weight_quantize(const float* w, size_t out, size_t in, int type, llmi_hip_weight** weight);
int llmi_hip_weight_quantize_dev(const float* w_dev, size_t out, size_t in, int type, llmi_hip_weight** weight);
int llmi_hip_weight_free(llmi_hip_weight* weight);
/* Replaces llmi::gguf::to_quantized (include/llmi/model/gguf.hpp:184,
 * src/model/gguf.cpp:577-640) followed by the upload: `blocks` (host) is a
 * GGUF tensor's raw data, nbytes long, out rows of in/32 ggml blocks
 * ({fp16 d; codes}, 34 bytes for Q8_0, 18 for Q4_0).  The device converts
 * each block into the layout llmi_hip_weight_upload produces from the
 * reference's own QuantizedMatrix (fp16 scale -> fp32 exactly; Q4_0's
 * halves-of-the-block nibble pairing re-packed into neighbour pairs), so
 * downloading the result gives to_quantized's data and scales bit for bit.
 * Fails (LLMI_ERR_ARG) where to_quantized fails: a type other than Q8_0 /
 * Q4_0, an empty shape, in not a multiple of 32, or nbytes not matching the
 * shape. */
int llmi_hip_weight_from_gguf(const void* blocks, size_t nbytes, size_t out, size_t in, int gguf_type,
                              llmi_hip_weight** weight);
/* Copies the weight back into the reference's planar layout (an fp32 weight:
 * its out x in floats into data, scales untouched). */
int llmi_hip_weight_download(const llmi_hip_weight* weight, uint8_t* data, float* scales);
/* Shape/type queries; byte_size is QuantizedMatrix::byte_size
 * (quant.hpp:47): packed code bytes + 4 * number of scales. */
int llmi_hip_weight_info(const llmi_hip_weight* weight, size_t* out, size_t* in, int* type, size_t* byte_size);
/* Device footprint of the re-laid-out matrix (codes + scales, with padding). */
size_t llmi_hip_weight_device_bytes(const llmi_hip_weight* weight);

/* Replaces llmi::quant::dequantize_row (quant.hpp:54, quant.cpp:104-117) and
 * the embedding gather Weight::row (weight.cpp:39-45): dst[k] =
 * code[row][k] * scale[row][k/32], one rounding, bit-exact. */
int llmi_hip_dequantize_row(const llmi_hip_weight* weight, size_t row, float* dst);
/* Gathers rows ids_dev[0..n) into dst_dev (n x in).  Ids must be in range. */
int llmi_hip_dequantize_rows_dev(const llmi_hip_weight* weight, const int32_t* ids_dev, size_t n, float* dst_dev,
                                 void* stream);

/* Replaces llmi::quant::matmul (quant.hpp:64-65, quant.cpp:119-153) and
 * Weight::matmul (weight.cpp:30-37): y[r*out + o] = sum_i x[r*in + i] *
 * dequantized(w[o][i]) (+ bias[o]), for r < rows.  The arithmetic is the
 * reference's, operation for operation (per 32-block a fused chain over the
 * block, then a fused chain over the blocks, then + bias), so y is bit-exact.
 * in and out must equal the weight's shape; bias may be NULL.
 * llmi_hip_matmul takes host pointers and returns with y complete. */
int llmi_hip_matmul(const llmi_hip_weight* weight, const float* x, size_t rows, size_t in, size_t out,
                    const float* bias, float* y);
int llmi_hip_matmul_dev(const llmi_hip_weight* weight, const float* x_dev, size_t rows, const float* bias_dev,
                        float* y_dev, void* stream);

/* A fixed list of independent products launched as ONE kernel: for each i,
 * y_dev[i] = quant::matmul(x_dev[i], rows[i], w[i]) (+ bias_dev[i]) exactly
 * as llmi_hip_matmul_dev would compute it (quant.cpp:119-153, bit-identical),
 * for callers that issue many small matmuls back to back (the per-layer
 * Weight::matmul calls of transformer.cpp:245-304 when their inputs are
 * ready together).  rows[i] is 1..8 (NULL: all 1); bias_dev may be NULL (no
 * biases) or hold NULL entries.  Every weight must have in <= ~10k.  The
 * group keeps the pointers, not the data: launch it whenever the inputs are
 * in place.  Products must not write memory another product of the group
 * reads.  llmi_hip_group_launch queues the kernel on `stream` (capturable in
 * a graph). */
typedef struct llmi_hip_group llmi_hip_group;
int llmi_hip_group_create(const llmi_hip_weight* const* w, const float* const* x_dev, const size_t* rows,
                          const float* const* bias_dev, float* const* y_dev, size_t count, llmi_hip_group** out);
int llmi_hip_group_launch(const llmi_hip_group* group, void* stream);
void llmi_hip_group_free(llmi_hip_group* group);

/* Tolerance mode, Q4_0: quant::matmul (quant.cpp:119-153) for batch 1..8
 * with the products summed on the matrix cores in another order than the
 * reference's chains.  NOT bit-exact: |y - y_ref| <= 1e-4 * max|y_ref| (the
 * fp32-accumulate tolerance of the path's contract; measured ~1e-6), with
 * finite x below ~3e38.  The codes enter as exact bf16 values, x as two bf16
 * parts (16 significant bits), sums in fp32.  Same arguments and meaning as
 * llmi_hip_matmul_dev (rows 1..8, in <= ~14k); llmi_hip_tol_group_* run a
 * list of such products as one launch, as llmi_hip_group_* do for the exact
 * kernel.  The exact
 * entry points stay the default everywhere: the model's decode and the
 * reference-signature layer never take this one. */
typedef struct llmi_hip_tol_group llmi_hip_tol_group;
int llmi_hip_matmul_tol_dev(const llmi_hip_weight* weight, const float* x_dev, size_t rows, const float* bias_dev,
                            float* y_dev, void* stream);
int llmi_hip_tol_group_create(const llmi_hip_weight* const* w, const float* const* x_dev, const size_t* rows,
                              const float* const* bias_dev, float* const* y_dev, size_t count,
                              llmi_hip_tol_group** out);
int llmi_hip_tol_group_launch(const llmi_hip_tol_group* group, void* stream);
void llmi_hip_tol_group_free(llmi_hip_tol_group* group);

/* Prefill GEMM on the matrix cores: quant::matmul (quant.cpp:119-153) as the
 * reference's prefill calls it with rows = T tokens (transformer.cpp:245-291),
 * computed with x and the dequantized weights rounded to bf16 and fp32
 * accumulation (bf16 MFMA).  NOT bit-exact: |y - y_ref| <= 2e-2 * max|y_ref|
 * (typically ~1e-3).  Use llmi_hip_matmul_dev where the reference's exact
 * results are needed.  Any rows >= 1; efficient for rows >= 64.
 * llmi_hip_gemm_group_* run a list of such products as one launch (per
 * weight type), e.g. the q/k/v or gate/up products of a layer.  A launch of
 * fewer than 256 output tiles (128 x 256) splits the K of products with
 * more than 1536 inputs over several workgroups and sums their fp32 partials
 * in a second kernel, so a product's results can differ in the last bits
 * between a launch that splits it and one that does not. */
int llmi_hip_matmul_mfma_dev(const llmi_hip_weight* weight, const float* x_dev, size_t rows, const float* bias_dev,
                             float* y_dev, void* stream);
/* llmi_hip_matmul_mfma_dev for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same kernels and results,
 * bit for bit; the GEMM's scratch -- the bf16 copy of x and, for a product
 * whose K is split over several workgroups (more than 1536 inputs on fewer
 * than 256 output tiles of 128 x 256, as llmi_hip_matmul_mfma_dev splits
 * it), its fp32 partial sums -- lives in a
 * fixed per-GPU array set up by llmi_hip_init instead of a buffer the
 * library grows, so the call makes no allocation.  Limit: 2 * rows * (in
 * rounded up to 64), rounded up to 256, plus 4 * rows * out * kchunks when K
 * is split, at most LLMI_MFMA_NOALLOC_SCRATCH_BYTES (LLMI_ERR_ARG beyond).
 * With nk = ceil(in / 64) and tiles = ceil(rows / 128) * ceil(out / 256), K
 * is split when nk > 24, tiles < 256 and k = min(256 / tiles, nk / 8)
 * (integer quotients) is at least 2, into kchunks = ceil(nk / ceil(nk / k))
 * chunks; e.g. 512 rows of 896 x 4864 take 9 chunks and need 21.5 MB.  Calls
 * that overlap on one GPU (e.g. on two streams) share that array and race. */
#define LLMI_MFMA_NOALLOC_SCRATCH_BYTES 33554432
int llmi_hip_matmul_mfma_noalloc_dev(const llmi_hip_weight* weight, const float* x_dev, size_t rows,
                                     const float* bias_dev, float* y_dev, void* stream);
typedef struct llmi_hip_gemm_group llmi_hip_gemm_group;
int llmi_hip_gemm_group_create(const llmi_hip_weight* const* w, const float* const* x_dev, const size_t* rows,
                               const float* const* bias_dev, float* const* y_dev, size_t count,
                               llmi_hip_gemm_group** out);
int llmi_hip_gemm_group_launch(const llmi_hip_gemm_group* group, void* stream);
void llmi_hip_gemm_group_free(llmi_hip_gemm_group* group);

/* ------------------------------------------------- glue kernels (device) */
/* Device counterparts of llmi::kernels (include/llmi/model/kernels.hpp:13-32)
 * and llmi::argmax (transformer.hpp:120), bit-identical to the reference.
 * All pointers are device pointers. */

/* kernels::dot (kernels.cpp:41-95, the AVX2 build's summation order):
 * out[i] = dot(a, b, lens[i]) for i < count. */
int llmi_hip_dot_dev(const float* a, const float* b, const int32_t* lens, size_t count, float* out, void* stream);
/* kernels::rmsnorm (kernels.cpp:115-120) on each of `rows` rows of length n. */
int llmi_hip_rmsnorm_dev(const float* x, const float* w, size_t rows, size_t n, float eps, float* y, void* stream);
/* kernels::softmax (kernels.cpp:136-146), in place on each row. */
int llmi_hip_softmax_dev(float* x, size_t rows, size_t n, void* stream);
/* kernels::silu (kernels.cpp:148), in place. */
int llmi_hip_silu_dev(float* x, size_t n, void* stream);
/* argmax (transformer.cpp:22-24): index of the first maximum of x[0..n). */
int llmi_hip_argmax_dev(const float* x, size_t n, int32_t* out, void* stream);

/* ------------------------------------------------------------- the model */

typedef struct llmi_hip_model llmi_hip_model; /* device-resident quantized decoder */
typedef struct llmi_hip_cache llmi_hip_cache; /* device KV cache of one sequence */

/* Replaces llmi::Transformer::load(model, F32 | Q8_0 | Q4_0)
 * (include/llmi/model/transformer.hpp:58, src/model/transformer.cpp:26-67):
 * quantizes every matrix (embedding, q/k/v/o, gate/up/down, untied lm_head)
 * on the GPU, or keeps them fp32 with LLMI_TYPE_F32; RMSNorm weights and
 * q/k/v biases stay fp32.  `tensors` holds
 * one fp32 array per tensor in the reference's expected_tensors() order
 * (src/model/model.cpp:135-162): embed; per layer input_layernorm, q, k, v,
 * [q_bias, k_bias, v_bias], o, post_attention_layernorm, gate, up, down;
 * final norm; [lm_head when untied].  _dev: the arrays are device pointers. */
int llmi_hip_model_create(const llmi_model_config* cfg, const float* const* tensors, int type, llmi_hip_model** model);
int llmi_hip_model_create_dev(const llmi_model_config* cfg, const float* const* tensors_dev, int type,
                              llmi_hip_model** model);
int llmi_hip_model_free(llmi_hip_model* model);
/* Transformer::weight_bytes (transformer.cpp:69-76). */
size_t llmi_hip_model_weight_bytes(const llmi_hip_model* model);

/* Transformer::new_cache (transformer.cpp:182-190): capacity
 * min(max_len, max_position_embeddings) positions, head-major fp32 K/V. */
int llmi_hip_model_new_cache(llmi_hip_model* model, size_t max_len, llmi_hip_cache** cache);
int llmi_hip_cache_free(llmi_hip_cache* cache);
/* KVCache::length / capacity / reset (transformer.hpp:29-45). */
size_t llmi_hip_cache_length(const llmi_hip_cache* cache);
size_t llmi_hip_cache_capacity(const llmi_hip_cache* cache);
int llmi_hip_cache_reset(llmi_hip_cache* cache);

/* Transformer::forward_cached (transformer.cpp:192-306): runs `n` new tokens
 * through the model, appends their K/V to `cache`, and writes the logits of
 * the last token (vocab floats) or of every new token (n x vocab) when
 * all_positions is set.  Bit-identical to the reference's logits.  Errors
 * (no tokens, id out of range, cache full or from another model) carry the
 * reference's messages. */
int llmi_hip_model_forward_cached(llmi_hip_model* model, llmi_hip_cache* cache, const int32_t* tokens, size_t n,
                                  int all_positions, float* logits);
/* forward_cached filling the reference's ForwardTrace (transformer.hpp:14-19,
 * transformer.cpp:218-221, :294, :299): states (host, NULL to skip) receives
 * (num_layers + 2) x n x hidden_size floats -- the token embeddings, the
 * output of every layer, then the final RMSNorm of every new token. */
int llmi_hip_model_forward_cached_trace(llmi_hip_model* model, llmi_hip_cache* cache, const int32_t* tokens,
                                        size_t n, int all_positions, float* logits, float* states);

/* Transformer::forward (transformer.cpp:78-166): the whole sequence without a
 * caller's cache (the model's own is reused and reset), logits of the last
 * token or of every token; states as for forward_cached_trace (NULL to
 * skip).  Bit-identical to forward_cached on a fresh cache, as the
 * reference's own test holds (tests/transformer_test.cpp:322-339); errors
 * carry forward's messages ("forward: ..."). */
int llmi_hip_model_forward(llmi_hip_model* model, const int32_t* tokens, size_t n, int all_positions, float* logits,
                           float* states);

/* Transformer::generate_greedy_cached (transformer.cpp:308-327): prefill,
 * then up to max_new greedy tokens (first maximum), stopping after a token in
 * stop_ids.  Writes *n_ids ids to `ids` (room for max_new). */
int llmi_hip_model_generate_greedy(llmi_hip_model* model, const int32_t* prompt, size_t n, size_t max_new,
                                   const int32_t* stop_ids, size_t n_stop, int32_t* ids, size_t* n_ids);
/* The scoring loop of llmi-perplexity on one chunk
 * (apps/llmi-perplexity/main.cpp:146-168): Transformer::forward(chunk,
 * all_positions = true) (transformer.cpp:78-166; here through a fresh cache,
 * bit-identical by the reference's own test), then for every position t in
 * [t_start, n - 1): nll[t - t_start] = -(logit_t[chunk[t + 1]] - lse_t),
 * lse_t = log(sum_v exp(double(logit_t[v] - max_t))) + max_t.  The caller
 * sums nll in order, as the app does.  Positions before t_start are still
 * run (they are the later positions' context) but not scored.  mode:
 *   LLMI_SCORE_EXACT      the reference's arithmetic throughout (logits bit-
 *                         identical; the double sum is taken as a tree, so
 *                         nll agrees to ~1e-15 relative);
 *   LLMI_SCORE_MFMA_HEAD  the lm_head on the bf16-MFMA GEMM (logits within
 *                         2e-2 of max|logit|, so each nll within 4e-2 of it);
 *   LLMI_SCORE_MFMA       every linear layer and the lm_head on the bf16-MFMA
 *                         GEMM (the fast perplexity path; not bit-exact). */
enum { LLMI_SCORE_EXACT = 0, LLMI_SCORE_MFMA_HEAD = 1, LLMI_SCORE_MFMA = 2 };
int llmi_hip_model_chunk_nll(llmi_hip_model* model, const int32_t* tokens, size_t n, size_t t_start, int mode,
                             double* nll);
/* ---------------------------------------------------------- token sampling */

/* SamplingConfig (include/llmi/model/sampling.hpp:20-24). */
typedef struct llmi_hip_sampling {
  float temperature; /* <= 0: the first maximum, nothing drawn (sampling.cpp:61) */
  size_t top_k;      /* 0 (or > n): no top-k filter */
  float top_p;       /* >= 1: no nucleus filter */
} llmi_hip_sampling;

/* llmi::sample (include/llmi/model/sampling.hpp:39, src/model/sampling.cpp:
 * 60-77) with its random number given: `target` is the number sample() draws
 * from the caller's generator, std::uniform_real_distribution<double>(0, 1)
 * on std::mt19937_64, once per call when temperature > 0 (no draw, and
 * `target` unused, otherwise).  *id is the reference's index for the same
 * logits, configuration and draw, bit for bit.  Logits may be -inf (masked
 * entries); NaN, or +inf after the division by temperature, are rejected
 * (LLMI_ERR_ARG: the reference's ranking is undefined there); every entry
 * -inf gives index 0, as the reference's fallback to argmax does.
 * _dev: logits in device memory, queued on `stream` (NULL = the library's),
 * synchronous (the index returns to the host).  n >= 1. */
int llmi_hip_sample(const float* logits, size_t n, const llmi_hip_sampling* cfg, double target, int32_t* id);
int llmi_hip_sample_dev(const float* logits, size_t n, const llmi_hip_sampling* cfg, double target, int32_t* id,
                        void* stream);
/* llmi::sampling_probabilities (sampling.hpp:32, sampling.cpp:11-58): the
 * filtered, renormalised distribution (host pointers), bit for bit. */
int llmi_hip_sampling_probabilities(const float* logits, size_t n, const llmi_hip_sampling* cfg, float* probs);
/* Testing aids, no counterpart in the reference: force every double sum of a
 * sample call onto its sequential pass (same results, slower), and report
 * which sums of the last call took the sequential pass (bit 0 softmax sum,
 * 1 top-p sum, 2 running sum of the draw, 3 renormalisation sum, 4 all of
 * the top-p sum, renormalisation sum and draw over the top-k select's
 * k <= 64 ranked values, which always run sequentially). */
int llmi_hip_sampling_set_exact_only(int on);
int llmi_hip_sampling_last_paths(int* paths);

/* One serving step on the device: forward_cached of `tokens` (transformer.cpp:
 * 192-306) and sample() on the last position's logits, which never leave HBM
 * (the loop of src/server/server.cpp:109-195 and llmi-chat, one call per
 * token).  `target` as for llmi_hip_sample. */
int llmi_hip_model_forward_sample(llmi_hip_model* model, llmi_hip_cache* cache, const int32_t* tokens, size_t n,
                                  const llmi_hip_sampling* cfg, double target, int32_t* id);
/* generate_greedy_cached with sample() in place of argmax: prefill, then up to
 * max_new sampled tokens, targets[i] being the draw of step i (room for
 * max_new; the caller draws them from its generator in order), stopping after
 * a token in stop_ids.  Timing as for generate_greedy (last_timing). */
int llmi_hip_model_generate_sampled(llmi_hip_model* model, const int32_t* prompt, size_t n, size_t max_new,
                                    const llmi_hip_sampling* cfg, const double* targets, const int32_t* stop_ids,
                                    size_t n_stop, int32_t* ids, size_t* n_ids);

/* GPU time of the last generate_greedy / generate_sampled call: the prompt
 * prefill and the decode loop (HIP events; the reference's llmi-generate --json reports the
 * same split as wall-clock seconds, apps/llmi-generate/main.cpp:329-345). */
int llmi_hip_model_last_timing(const llmi_hip_model* model, double* prefill_ms, double* decode_ms);

/* Of the last generate_sampled call: how many of its steps were redrawn with
 * a host read-back of their own.  With temperature > 0 the steps are queued
 * on the device in windows and read back once per window; a queued draw that
 * its bounds leave undecided (a target on a running sum) sends the run back
 * to that step, which is redrawn exactly before queueing resumes.  0 when
 * every step ran queued.  Diagnostic: no counterpart in the reference. */
int llmi_hip_model_last_redraws(const llmi_hip_model* model, size_t* steps);

/* The arithmetic of the model's one-token decode steps (forward_cached with
 * one token, generate_greedy / generate_sampled after the prompt).
 * LLMI_DECODE_EXACT (the default): the reference's operations in its order,
 * logits bit-identical to transformer.cpp:192-306.  LLMI_DECODE_TOLERANCE:
 * attention split over position chunks (at most 16 per head), each chunk's
 * softmax taken against its own maximum with the hardware exponential, the
 * chunks merged in the o_proj product's staging, and every matmul split
 * over K into one-wavefront workgroups whose partial sums meet by atomic
 * adds; logits within the path's floating-point tolerance of the exact
 * ones, neither bit-identical nor reproducible bit for bit.  Applies to
 * head_dim 64 / 128 with at most 16 query heads per KV head and row counts
 * of q, k, v, gate and up that are multiples of 64 (other models keep the
 * exact step); the prompt's prefill is exact in both modes.
 * No counterpart in the reference (whose decode is exact by construction):
 * a speed option for callers that accept the tolerance. */
enum { LLMI_DECODE_EXACT = 0, LLMI_DECODE_TOLERANCE = 1 };
int llmi_hip_model_set_decode_mode(llmi_hip_model* model, int mode);

/* Whether generate_greedy replays its tolerance-mode steps (no stop ids, at
 * least 8 new tokens) from one captured HIP graph -- the step's positions
 * and output slot read from device memory, one host launch per token
 * instead of ~5 per layer -- (enable != 0, the default) or launches every
 * kernel of every step (0; e.g. under profilers that do not follow graphs).
 * The same kernels and results either way.  No counterpart in the
 * reference: a launch-overhead option. */
int llmi_hip_model_set_decode_graph(llmi_hip_model* model, int enable);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* LLMI_HIP_H */
