// Shared definitions of the gfx950 quantized-weight library: error channel,
// the device weight layout, and launch helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/llmi_hip.h"

namespace llmi_hip {

constexpr int kBlock = LLMI_BLOCK_SIZE;  // weights per quantization block
constexpr int kTileRows = 64;            // output rows per wavefront tile (one row per lane)

// Thread-local last error (llmi_hip_last_error).
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

hipStream_t library_stream();
bool initialised();
std::size_t max_lds_per_block();  // bytes of LDS one workgroup may allocate
inline hipStream_t pick(void* s) { return s != nullptr ? static_cast<hipStream_t>(s) : library_stream(); }

#define LLMI_TRY_HIP(expr)                                                                        \
  do {                                                                                            \
    const hipError_t err_ = (expr);                                                               \
    if (err_ != hipSuccess) return ::llmi_hip::fail(LLMI_ERR_HIP, std::string(#expr) + ": " + hipGetErrorString(err_)); \
  } while (0)

#define LLMI_REQUIRE(cond, msg)                                   \
  do {                                                            \
    if (!(cond)) return ::llmi_hip::fail(LLMI_ERR_ARG, (msg));    \
  } while (0)

#define LLMI_REQUIRE_INIT()                                                                   \
  do {                                                                                        \
    if (!::llmi_hip::initialised()) return ::llmi_hip::fail(LLMI_ERR_STATE, "llmi_hip_init has not been called"); \
  } while (0)

inline std::size_t ceil_div(std::size_t a, std::size_t b) { return (a + b - 1) / b; }
inline std::size_t row_bytes(std::size_t in, int type) {
  return type == LLMI_TYPE_Q4_0 ? (in + 1) / 2 : type == LLMI_TYPE_F32 ? 4 * in : in;
}

// Device layout of a packed matrix ("tiled"): rows are grouped in tiles of 64
// (lane l of a wavefront owns row tile*64 + l).  For each tile and each
// 32-weight block b the 64 rows' codes sit next to each other, so one
// wavefront reads a block of 64 rows with fully coalesced 16-byte loads:
//   Q4_0: codes[((tile*nblk + b)*64 + lane)*16 + j], j = 0..15, holding the
//         block's elements in the reference's nibble order (element 2j in the
//         low nibble of byte j, 2j+1 in the high nibble, +8 bias).
//   Q8_0: codes[(((tile*nblk + b)*2 + h)*64 + lane)*16 + j] = int8 code of
//         element 16h + j of the block.
//   scales[(tile*nblk + b)*64 + lane] = the block's fp32 scale.
// Rows past `out` in the last tile and elements past `in` in the last block
// are zero bytes.  A block is 16 (Q4_0) or 32 (Q8_0) code bytes plus 4 scale
// bytes, the reference's 0.625 / 1.125 bytes per weight.
struct DeviceMatrix {
  int type = 0;
  std::size_t out = 0, in = 0, nblk = 0, ntiles = 0;
  std::uint8_t* codes = nullptr;
  float* scales = nullptr;
  std::size_t code_bytes = 0, scale_bytes = 0;
};

// How a 16-row tile stages its activations in LDS (GroupProblem::prologue):
// kPlain x; kRmsNorm w * (x * scale), the reference's RMSNorm of x
// (kernels.cpp:115-120) with pw = w; kSiluUp silu(x) * pw, the reference's
// SiLU times up (transformer.cpp:290, kernels.cpp:148).  Either one is the
// same arithmetic as the separate glue kernel it replaces.
// kAttnCombine (the tolerance-mode decode's split products only, see
// SplitProduct): the attention output assembled from per-chunk partial
// softmax states (attn_part_1); pw points to the partials (layout at
// kAttnMaxChunks).
enum { kPlain = 0, kRmsNorm = 1, kSiluUp = 2, kAttnCombine = 3 };

// Partial attention states of the tolerance-mode decode, per query head h
// and position chunk c < kAttnMaxChunks, in one buffer of
// kAttnMaxChunks * nh * (hd + 2) floats: o[h][c][hd] (the chunk's
// unnormalised P.V), then m[h][c] (the chunk's score maximum), then
// l[h][c] (its sum of exp(score - m)).
constexpr int kAttnMaxChunks = 16;
constexpr int kAttnChunkUnit = 64;  // chunks are whole multiples of this many positions
// Positions per chunk for npos positions: the fewest multiples of
// kAttnChunkUnit that give at most kAttnMaxChunks chunks.
__host__ __device__ inline int attn_chunk_len(int npos) {
  const int units = (npos + kAttnChunkUnit - 1) / kAttnChunkUnit;
  return kAttnChunkUnit * ((units + kAttnMaxChunks - 1) / kAttnMaxChunks);
}

// One product of a grouped launch (qgemv_group), as the kernel reads it.
struct GroupProblem {
  static constexpr int kNarrow = 16;  // kind: 16-row tiles, batch 1; else the row chunk R (1, 2, 4, 8)
  const std::uint8_t* codes;
  const float* scales;
  const float* x;
  const float* bias;
  float* y;
  const float* pw;  // prologue operand (RMSNorm weight, the up vector or the attention partials)
  float eps;        // RMSNorm epsilon
  int type, kind, in, nblk, out, rows, ntiles, bpw, accumulate, first_wg, prologue;
};

// One product y = W x (+ bias) (y += ... with accumulate), rows 1..8, as the
// caller describes it; a prologue (batch 1 only) transforms x first.
struct GroupEntry {
  const DeviceMatrix* m;
  const float* x;
  const float* bias;
  float* y;
  std::size_t rows;
  bool accumulate;
  int prologue = kPlain;
  const float* pw = nullptr;
  float eps = 0.0f;
};
// One kernel launch of a group: the products of weight type `type` and row
// chunk `rchunk` (GroupProblem::kNarrow: the 16-row tiles), at
// probs[prob_offset...], workgroup w running product wg_prob[map_offset + w].
struct GroupLaunch {
  int type = 0, rchunk = 1, waves = 1, total_wgs = 0, nprob = 0;
  std::size_t lds = 0, prob_offset = 0, map_offset = 0;
};
struct GroupPlan {
  std::vector<GroupProblem> probs;
  std::vector<std::uint32_t> wg_prob;
  std::vector<GroupLaunch> launches;
};
int plan_group(const GroupEntry* entries, std::size_t count, GroupPlan* plan);
int launch_group(const GroupProblem* probs_dev, const std::uint32_t* map_dev, const GroupLaunch& l, hipStream_t s);

// A planned group resident on the device (its table and workgroup map).
struct DeviceGroup {
  void* table = nullptr;
  const GroupProblem* probs = nullptr;
  const std::uint32_t* map = nullptr;
  std::vector<GroupLaunch> launches;
  std::vector<GroupProblem> host_probs;  // the table's host copy (few-product launches pass them by value)
  int build(const GroupEntry* entries, std::size_t count);
  int launch(hipStream_t s) const;
  void release();
};

// One product of a grouped bf16-MFMA GEMM launch (qgemm_mfma).  xb: the
// activations converted to bf16, [rows][ldx] (ldx = in rounded up to 64).
struct GemmProblem {
  const std::uint8_t* codes;
  const float* scales;
  const std::uint16_t* xb;
  const float* xf;  // the fp32 activations, read directly by launches with GemmLaunch::f32x
  const float* bias;
  float* y;
  int rows, in, ldx, out, nblk, ntiles, mtiles, first_wg, input;
  int accumulate;  // y += acc + bias (the residual update), else y = acc + bias
  // Split K: kchunks workgroups per output tile, each over kpc K-steps of 64,
  // write fp32 partial tiles to part ([kchunks][rows][out]); gemm_reduce then
  // sums them in chunk order and applies bias / accumulate.  kchunks == 1:
  // the workgroup writes y itself.
  int kchunks, kpc;
  float* part;
};
// K chunks of a product with `in` inputs on a GEMM launch of `launch_tiles`
// output tiles (128 x 256), `split_tiles` of them belonging to products of
// more than 24 K-steps of 64.  A launch of fewer tiles than the 256 CUs
// splits the K of those long products over as many workgroups (chunks of at
// least 8 steps) as the CUs its short products leave free, so the long K
// loops of a few workgroups are not the launch's critical path; launches
// with enough tiles are not split (partial sums would only add traffic).
// The split changes the fp32 summation order, so a product's bits depend on
// whether and how its launch splits it.
int gemm_kchunks(std::size_t in, std::size_t launch_tiles, std::size_t split_tiles);
// K-steps per chunk for kchunks chunks (every chunk non-empty).
int gemm_kpc(std::size_t in, int kchunks);
std::size_t gemm_tiles(std::size_t rows, std::size_t out);
// Tiles of a product that the K split may apply to (0 for short K).
std::size_t gemm_split_tiles(std::size_t rows, std::size_t in, std::size_t out);
// A distinct fp32 activation matrix of a GEMM group and where its bf16 copy
// lives in the group's scratch (element offset).
struct GemmInput {
  const float* x = nullptr;
  std::size_t rows = 0, in = 0, ldx = 0, offset = 0;
};
struct GemmLaunch {
  int type = 0, total_wgs = 0;
  std::size_t prob_offset = 0, map_offset = 0;
  // The GEMM reads the fp32 activations itself and rounds them to bf16 as it
  // stages them (every product's K a multiple of 64, rows 16-byte aligned):
  // no conversion launch, no bf16 copy.
  bool f32x = false;
};
struct GemmPlan {
  std::vector<GemmProblem> probs;
  std::vector<std::uint32_t> work_prob;
  std::vector<GemmLaunch> launches;
  std::vector<GemmInput> inputs;
  std::size_t scratch_elems = 0;  // bf16 elements of scratch the inputs need
  std::vector<std::size_t> part_off;  // per problem: float offset of its partials (split problems)
  std::size_t part_floats = 0;        // fp32 partials the split problems need
  bool f32x = false;                  // the launches read fp32 activations (GemmLaunch::f32x)
};
// Bytes of a plan's scratch: the bf16 inputs, then (256-byte aligned) the
// fp32 partials.
std::size_t gemm_scratch_bytes(const GemmPlan& plan);
int plan_gemm_group(const GroupEntry* entries, std::size_t count, GemmPlan* plan);
// One product on the bf16-MFMA GEMM, with the library's bf16 staging buffer
// (grown on demand, outside any graph capture).
// Up to kGemmFew products (GroupEntry, batch rows each) on the bf16-MFMA
// GEMM as one conversion launch, one GEMM launch per weight type (products
// by value) and the split products' reductions; scratch from the library's
// grow-only GEMM workspace.
int launch_gemm_entries(const GroupEntry* e, std::size_t n, hipStream_t s);
int launch_gemm_single(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y,
                       hipStream_t s, bool accumulate = false);
// The allocation-free single-product GEMM (llmi_hip_matmul_mfma_noalloc_dev):
// noalloc_setup records, with `device` current, the device address of its
// file-scope scratch array (once per device, from llmi_hip_init);
// launch_gemm_noalloc runs launch_gemm_single's kernels with x's bf16 copy
// in that array.
int noalloc_setup(int device);
int launch_gemm_noalloc(int device, const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias,
                        float* y, hipStream_t s);
// Points every problem at its input's bf16 copy inside `scratch` and its
// partials after them (gemm_scratch_bytes bytes in all).
void bind_gemm_scratch(GemmPlan* plan, std::uint16_t* scratch);
// The reduction of every split problem of a plan (after its GEMM launches).
int launch_gemm_reduces(const GemmPlan& plan, hipStream_t s);
// Queues the fp32 -> bf16 conversion of every input into `scratch`.
int launch_gemm_inputs(const GemmPlan& plan, std::uint16_t* scratch, hipStream_t s);
// one != nullptr: launch the single product *one (plan of one entry) without
// a device table.
// Up to kGemmFew products of one launch passed by value (no device table).
constexpr int kGemmFew = 3;
struct GemmFew {
  GemmProblem p[kGemmFew];
  int count;
};
// probs_dev / map_dev: a launch's device tables; or one != nullptr: the
// launch's nfew (1..kGemmFew) products by value.
int launch_gemm(const GemmProblem* probs_dev, const std::uint32_t* map_dev, const GemmLaunch& l, hipStream_t s,
                const GemmProblem* one = nullptr, int nfew = 1);

inline std::size_t block_code_bytes(int type) { return type == LLMI_TYPE_Q4_0 ? 16 : 32; }

// Kernel launchers (implemented next to their kernels).
int launch_quantize(const float* w, std::size_t out, std::size_t in, int type, std::uint8_t* planar_data,
                    float* planar_scales, DeviceMatrix* tiled, hipStream_t s);
int launch_relayout_to_tiled(const std::uint8_t* planar_data, const float* planar_scales, const DeviceMatrix& m,
                             hipStream_t s);
int launch_relayout_to_planar(const DeviceMatrix& m, std::uint8_t* planar_data, float* planar_scales, hipStream_t s);
// fp32 weights (type LLMI_TYPE_F32: codes holds the row-major [out][in]
// floats, no scales): kernels::matmul and the row gather (f32.hip).
int launch_matmul_f32(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y,
                      hipStream_t s, bool accumulate);
int launch_gather_f32(const DeviceMatrix& m, const std::int32_t* ids, std::size_t n, float* dst, hipStream_t s);
// GGUF (ggml) Q8_0 / Q4_0 blocks of m's shape (device memory) -> m.
int launch_gguf_to_tiled(const void* raw, const DeviceMatrix& m, hipStream_t s);
int launch_dequantize_rows(const DeviceMatrix& m, const std::int32_t* ids, std::size_t n, float* dst, hipStream_t s);
// accumulate: y[r][o] = y[r][o] + (acc + bias) -- the reference's
// `proj = W x; x += proj` residual update (transformer.cpp:283-284, :291-292)
// done in the GEMV's epilogue with the same two roundings.
int launch_matmul(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y, hipStream_t s,
                  bool accumulate = false);
// Products of one weight type and input size sharing x and rows (the
// prefill's q/k/v, gate/up): one split-block launch over all their tiles
// when each would take the split-block product, else one launch each.
// RoPE tables (cos_t / sin_t: [position][32], head size 64), the first
// position of the launch's rows, and one layer's K / V cache ([head][cap][64]).
struct RopeCache {
  const float* cos_t = nullptr;
  const float* sin_t = nullptr;
  float* kc = nullptr;
  float* vc = nullptr;
  int base = 0, cap = 0;
};
enum SharedEpilogue { kStorePlain = 0, kStoreRope = 1, kStoreRopeCache = 2, kStoreCache = 3 };
// With rope (and roped) given and three products of head size 64 grouped,
// q is RoPE'd in place, k RoPE'd into rope->kc and v copied into rope->vc at
// positions base + row, and *roped is set; otherwise the caller applies RoPE.
int launch_matmul_shared(const DeviceMatrix* const* ms, const float* const* biases, float* const* ys, int count,
                         const float* x, std::size_t rows, hipStream_t s, const RopeCache* rope = nullptr,
                         bool* roped = nullptr);
// The prefill's MLP gate and up projections fused with silu(gate) * up into
// y, when both would take the split-block product (rows > 8, few tiles, one
// quantized type and shape); *fused reports whether it ran (else nothing was
// launched and the caller takes the unfused path).
int launch_gate_up_silu(const DeviceMatrix& gate, const DeviceMatrix& up, const float* x, std::size_t rows,
                        float* y, hipStream_t s, bool* fused);
// The tolerance-mode one-token step's products (gemv.hip): y += W x' split
// over K into about kSplitTarget workgroups of one wavefront, each adding
// its partial sums to y with atomic adds (so y must hold the residual, or
// zeros, beforehand; the bias is added by the first split).  x' is x under
// `prologue`: kRmsNorm (pw = the norm weight), kSiluUp (pw = up) or
// kAttnCombine (pw = x = the attention partials, comb_hd = head_dim).  zero
// (may be null): nzero floats the launch clears besides, for a product
// later in the step that accumulates into them.  Within a split the sums
// are the exact kernels'; the splits land in no fixed order, so results are
// within the fp32-accumulate tolerance and not reproducible bit for bit.
struct SplitProduct {
  const DeviceMatrix* m = nullptr;
  const float* x = nullptr;
  const float* pw = nullptr;
  const float* bias = nullptr;
  float* y = nullptr;
  int prologue = kPlain;
  float eps = 0.0f;
  int comb_hd = 0;
  float* zero = nullptr;
  int nzero = 0;
  int bps = 0, splits = 0;  // set by plan_split: blocks per split, splits per 64-row tile
};
int plan_split(SplitProduct* p);
// comb_nch: kAttnCombine's chunk count; npos_dev (may be null): the
// positions of the step in device memory (a step replayed from a graph),
// comb_nch then being the chunk length and the count taken on the device.
int launch_split(const SplitProduct& p, hipStream_t s, int comb_nch = 0, const int* npos_dev = nullptr);
// Frees the sampling workspace (llmi_hip_shutdown; the stream is idle).
void release_sampling_workspace();
// Frees the tolerance-mode product's split activations (likewise).
void release_tol_workspace();

// sample() on device logits (sampling.hip); *id_host receives the index and
// `also` (device, may be null) too, on the stream.
int sample_device(const float* logits, std::size_t n, const llmi_hip_sampling& cfg, double target,
                  std::int32_t* id_host, std::int32_t* also, hipStream_t s);
// One draw's outcome, written on the device: id (-1 when undecided) and
// state (bit 0: decided; bits 1..: the logits' NaN / +inf / all -inf flags).
struct SampleLog {
  std::int32_t id;
  std::int32_t state;
};
// sample_device without the host read-back (temperature > 0): the index goes
// to `also` and *log; an undecided log entry must be redrawn by sample_device.
int sample_device_async(const float* logits, std::size_t n, const llmi_hip_sampling& cfg, double target,
                        std::int32_t* also, SampleLog* log, hipStream_t s);

int launch_synth_normal(float* dst, std::size_t n, std::uint64_t seed, std::uint64_t offset, double mean, double stdev,
                        hipStream_t s);

}  // namespace llmi_hip

struct llmi_hip_weight {
  llmi_hip::DeviceMatrix m;
};
