// The C ABI (include/llmi_hip.h): runtime state, error channel, device
// memory helpers and the quantized-weight entry points.
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"

namespace llmi_hip {

namespace {
thread_local std::string t_error;
int g_device = -1;
hipStream_t g_stream = nullptr;
std::size_t g_max_lds = 64 * 1024;

// A scoped device allocation used by the host-pointer entry points.
struct DevBuf {
  void* p = nullptr;
  ~DevBuf() {
    if (p != nullptr) (void)hipFree(p);
  }
  int alloc(std::size_t bytes) {
    if (bytes == 0) return LLMI_OK;
    LLMI_TRY_HIP(hipMalloc(&p, bytes));
    return LLMI_OK;
  }
  template <typename T>
  T* as() const {
    return static_cast<T*>(p);
  }
};

// The single-product GEMM's bf16 copy of x: grown when a call needs more (the
// stream is drained first, since queued work may still read the old one).
struct Scratch {
  void* p = nullptr;
  std::size_t bytes = 0;
  int reserve(std::size_t need, hipStream_t s) {
    if (need <= bytes) return LLMI_OK;
    LLMI_TRY_HIP(hipStreamSynchronize(s));
    if (p != nullptr) LLMI_TRY_HIP(hipFree(p));
    p = nullptr;
    bytes = 0;
    LLMI_TRY_HIP(hipMalloc(&p, need));
    bytes = need;
    return LLMI_OK;
  }
};
Scratch g_gemm_scratch;

int check_type(int type) {
  LLMI_REQUIRE(type == LLMI_TYPE_Q8_0 || type == LLMI_TYPE_Q4_0, "type must be LLMI_TYPE_Q8_0 or LLMI_TYPE_Q4_0");
  return LLMI_OK;
}

// Allocates a tiled device matrix (zeroed, so padding rows/elements are 0).
int alloc_matrix(std::size_t out, std::size_t in, int type, DeviceMatrix* m) {
  m->type = type;
  m->out = out;
  m->in = in;
  m->nblk = ceil_div(in, kBlock);
  m->ntiles = ceil_div(out, kTileRows);
  m->code_bytes = m->ntiles * m->nblk * kTileRows * block_code_bytes(type);
  m->scale_bytes = m->ntiles * m->nblk * kTileRows * sizeof(float);
  if (type == LLMI_TYPE_F32) {  // row-major floats, as the reference keeps them
    m->code_bytes = out * in * sizeof(float);
    m->scale_bytes = 0;
    if (m->code_bytes != 0) LLMI_TRY_HIP(hipMalloc(reinterpret_cast<void**>(&m->codes), m->code_bytes));
    return LLMI_OK;
  }
  if (m->code_bytes == 0) return LLMI_OK;
  LLMI_TRY_HIP(hipMalloc(reinterpret_cast<void**>(&m->codes), m->code_bytes));
  const hipError_t e = hipMalloc(reinterpret_cast<void**>(&m->scales), m->scale_bytes);
  if (e != hipSuccess) {
    (void)hipFree(m->codes);
    m->codes = nullptr;
    return fail(LLMI_ERR_HIP, std::string("hipMalloc(scales): ") + hipGetErrorString(e));
  }
  LLMI_TRY_HIP(hipMemsetAsync(m->codes, 0, m->code_bytes, library_stream()));
  LLMI_TRY_HIP(hipMemsetAsync(m->scales, 0, m->scale_bytes, library_stream()));
  return LLMI_OK;
}

void free_matrix(DeviceMatrix* m) {
  if (m->codes != nullptr) (void)hipFree(m->codes);
  if (m->scales != nullptr) (void)hipFree(m->scales);
  m->codes = nullptr;
  m->scales = nullptr;
}

}  // namespace

void set_error(const std::string& msg) { t_error = msg; }
int fail(int code, const std::string& msg) {
  t_error = msg;
  return code;
}
hipStream_t library_stream() { return g_stream; }
bool initialised() { return g_device >= 0; }
std::size_t max_lds_per_block() { return g_max_lds; }

}  // namespace llmi_hip

using namespace llmi_hip;

namespace llmi_hip {

int launch_gemm_entries(const GroupEntry* e, std::size_t n, hipStream_t s) {
  LLMI_REQUIRE(n >= 1 && n <= static_cast<std::size_t>(kGemmFew), "gemm: 1..3 products");
  GemmPlan plan;
  if (int rc = plan_gemm_group(e, n, &plan)) return rc;
  if (plan.launches.empty()) return LLMI_OK;
  if (int rc = g_gemm_scratch.reserve(gemm_scratch_bytes(plan), s)) return rc;
  auto* scratch = static_cast<std::uint16_t*>(g_gemm_scratch.p);
  bind_gemm_scratch(&plan, scratch);
  if (int rc = launch_gemm_inputs(plan, scratch, s)) return rc;
  for (std::size_t i = 0; i < plan.launches.size(); ++i) {
    const GemmLaunch& l = plan.launches[i];
    const std::size_t end = i + 1 < plan.launches.size() ? plan.launches[i + 1].prob_offset : plan.probs.size();
    if (int rc = launch_gemm(nullptr, nullptr, l, s, &plan.probs[l.prob_offset], static_cast<int>(end - l.prob_offset)))
      return rc;
  }
  return launch_gemm_reduces(plan, s);
}

int launch_gemm_single(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y,
                       hipStream_t s, bool accumulate) {
  if (rows == 0 || m.out == 0) return LLMI_OK;
  const GroupEntry e{&m, x, bias, y, rows, accumulate};
  return launch_gemm_entries(&e, 1, s);
}

}  // namespace llmi_hip

struct llmi_hip_group {
  DeviceGroup g;
  ~llmi_hip_group() { g.release(); }
};

struct llmi_hip_gemm_group {
  void* table = nullptr;  // device copy of the problem table, then the work -> problem map
  std::uint16_t* scratch = nullptr;  // bf16 copies of the inputs
  const GemmProblem* probs = nullptr;
  const std::uint32_t* map = nullptr;
  GemmPlan plan;
  ~llmi_hip_gemm_group() {
    if (table != nullptr) (void)hipFree(table);
    if (scratch != nullptr) (void)hipFree(scratch);
  }
};

namespace {

template <typename Plan, typename Group>
int upload_plan(const Plan& plan, const std::vector<typename decltype(Plan::probs)::value_type>& probs,
                const std::vector<std::uint32_t>& map, Group* g) {
  using Prob = typename decltype(Plan::probs)::value_type;
  const std::size_t pbytes = probs.size() * sizeof(Prob);
  const std::size_t mbytes = map.size() * sizeof(std::uint32_t);
  if (pbytes + mbytes == 0) return LLMI_OK;
  LLMI_TRY_HIP(hipMalloc(&g->table, pbytes + mbytes));
  auto* base = static_cast<std::uint8_t*>(g->table);
  LLMI_TRY_HIP(hipMemcpy(base, probs.data(), pbytes, hipMemcpyHostToDevice));
  if (mbytes > 0) LLMI_TRY_HIP(hipMemcpy(base + pbytes, map.data(), mbytes, hipMemcpyHostToDevice));
  g->probs = reinterpret_cast<const Prob*>(base);
  g->map = reinterpret_cast<const std::uint32_t*>(base + pbytes);
  (void)plan;
  return LLMI_OK;
}

int group_entries(const llmi_hip_weight* const* w, const float* const* x, const size_t* rows, const float* const* bias,
                  float* const* y, size_t count, std::size_t default_rows, std::vector<GroupEntry>* entries) {
  LLMI_REQUIRE(count == 0 || (w != nullptr && x != nullptr && y != nullptr), "group: null array");
  entries->resize(count);
  for (size_t i = 0; i < count; ++i) {
    LLMI_REQUIRE(w[i] != nullptr, "group: null weight");
    (*entries)[i] = GroupEntry{&w[i]->m, x[i], bias != nullptr ? bias[i] : nullptr, y[i],
                               rows != nullptr ? rows[i] : default_rows, false};
  }
  return LLMI_OK;
}

}  // namespace

extern "C" {

const char* llmi_hip_last_error(void) { return t_error.c_str(); }
const char* llmi_hip_version(void) { return "llmi_hip 0.1 (gfx950, exact fused-chain GEMV)"; }

int llmi_hip_init(int device) {
  int count = 0;
  LLMI_TRY_HIP(hipGetDeviceCount(&count));
  LLMI_REQUIRE(device >= 0 && device < count, "llmi_hip_init: no such device");
  if (g_device == device && g_stream != nullptr) return LLMI_OK;
  LLMI_TRY_HIP(hipSetDevice(device));
  if (g_stream != nullptr) {
    LLMI_TRY_HIP(hipStreamDestroy(g_stream));
    g_stream = nullptr;
  }
  LLMI_TRY_HIP(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
  hipDeviceProp_t prop{};
  LLMI_TRY_HIP(hipGetDeviceProperties(&prop, device));
  g_max_lds = prop.sharedMemPerBlock;
  if (int rc = noalloc_setup(device)) return rc;
  g_device = device;
  return LLMI_OK;
}

int llmi_hip_shutdown(void) {
  if (g_stream != nullptr) {
    LLMI_TRY_HIP(hipStreamSynchronize(g_stream));
    LLMI_TRY_HIP(hipStreamDestroy(g_stream));
  }
  // The library's own workspaces (model, weight and group handles belong to
  // their callers).
  release_sampling_workspace();
  release_tol_workspace();
  if (g_gemm_scratch.p != nullptr) (void)hipFree(g_gemm_scratch.p);
  g_gemm_scratch = Scratch{};
  g_stream = nullptr;
  g_device = -1;
  return LLMI_OK;
}

void* llmi_hip_stream(void) { return g_stream; }

int llmi_hip_synchronize(void) {
  LLMI_REQUIRE_INIT();
  LLMI_TRY_HIP(hipStreamSynchronize(g_stream));
  return LLMI_OK;
}

int llmi_hip_malloc(void** ptr, size_t bytes) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(ptr != nullptr, "llmi_hip_malloc: null out-pointer");
  *ptr = nullptr;
  if (bytes == 0) return LLMI_OK;
  LLMI_TRY_HIP(hipMalloc(ptr, bytes));
  return LLMI_OK;
}

int llmi_hip_free(void* ptr) {
  if (ptr != nullptr) LLMI_TRY_HIP(hipFree(ptr));
  return LLMI_OK;
}

int llmi_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
  LLMI_REQUIRE_INIT();
  if (bytes == 0) return LLMI_OK;
  LLMI_TRY_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
  LLMI_TRY_HIP(hipStreamSynchronize(g_stream));
  return LLMI_OK;
}

int llmi_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
  LLMI_REQUIRE_INIT();
  if (bytes == 0) return LLMI_OK;
  LLMI_TRY_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
  LLMI_TRY_HIP(hipStreamSynchronize(g_stream));
  return LLMI_OK;
}

int llmi_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
  LLMI_REQUIRE_INIT();
  if (bytes == 0) return LLMI_OK;
  LLMI_TRY_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, pick(stream)));
  return LLMI_OK;
}

int llmi_hip_memset_dev(void* dst, int value, size_t bytes) {
  LLMI_REQUIRE_INIT();
  if (bytes == 0) return LLMI_OK;
  LLMI_TRY_HIP(hipMemsetAsync(dst, value, bytes, g_stream));
  LLMI_TRY_HIP(hipStreamSynchronize(g_stream));
  return LLMI_OK;
}

int llmi_hip_event_create(void** ev) {
  LLMI_REQUIRE_INIT();
  hipEvent_t e = nullptr;
  LLMI_TRY_HIP(hipEventCreate(&e));
  *ev = e;
  return LLMI_OK;
}

int llmi_hip_event_destroy(void* ev) {
  if (ev != nullptr) LLMI_TRY_HIP(hipEventDestroy(static_cast<hipEvent_t>(ev)));
  return LLMI_OK;
}

int llmi_hip_event_record(void* ev, void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_TRY_HIP(hipEventRecord(static_cast<hipEvent_t>(ev), pick(stream)));
  return LLMI_OK;
}

int llmi_hip_event_elapsed_ms(void* start, void* stop, float* ms) {
  LLMI_TRY_HIP(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
  LLMI_TRY_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
  return LLMI_OK;
}

int llmi_hip_graph_begin(void) {
  LLMI_REQUIRE_INIT();
  LLMI_TRY_HIP(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal));
  return LLMI_OK;
}

int llmi_hip_graph_end(void** graph) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(graph != nullptr, "graph_end: null out-pointer");
  hipGraph_t g = nullptr;
  LLMI_TRY_HIP(hipStreamEndCapture(g_stream, &g));
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) return fail(LLMI_ERR_HIP, std::string("hipGraphInstantiate: ") + hipGetErrorString(e));
  *graph = exec;
  return LLMI_OK;
}

int llmi_hip_graph_launch(void* graph) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(graph != nullptr, "graph_launch: null graph");
  LLMI_TRY_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(graph), g_stream));
  return LLMI_OK;
}

int llmi_hip_graph_destroy(void* graph) {
  if (graph != nullptr) LLMI_TRY_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph)));
  return LLMI_OK;
}

int llmi_hip_synth_normal_dev(float* dst, size_t n, uint64_t seed, uint64_t offset, double mean, double stdev,
                              void* stream) {
  LLMI_REQUIRE_INIT();
  return launch_synth_normal(dst, n, seed, offset, mean, stdev, pick(stream));
}

size_t llmi_hip_row_bytes(size_t in, int type) { return row_bytes(in, type); }

int llmi_hip_quantize_dev(const float* w, size_t out, size_t in, int type, uint8_t* data, float* scales, void* stream) {
  LLMI_REQUIRE_INIT();
  if (const int rc = check_type(type)) return rc;
  LLMI_REQUIRE(in <= 0x7FFFFFFFu, "quantize: in too large");
  if (out == 0 || in == 0) return LLMI_OK;
  LLMI_REQUIRE(w != nullptr && data != nullptr && scales != nullptr, "quantize: null pointer");
  return launch_quantize(w, out, in, type, data, scales, nullptr, pick(stream));
}

int llmi_hip_quantize(const float* w, size_t out, size_t in, int type, uint8_t* data, float* scales) {
  LLMI_REQUIRE_INIT();
  if (const int rc = check_type(type)) return rc;
  if (out == 0 || in == 0) return LLMI_OK;
  LLMI_REQUIRE(w != nullptr && data != nullptr && scales != nullptr, "quantize: null pointer");
  const std::size_t nw = out * in, nd = out * row_bytes(in, type), ns = out * ceil_div(in, kBlock);
  DevBuf dw, dd, ds;
  if (int rc = dw.alloc(nw * sizeof(float))) return rc;
  if (int rc = dd.alloc(nd)) return rc;
  if (int rc = ds.alloc(ns * sizeof(float))) return rc;
  LLMI_TRY_HIP(hipMemcpyAsync(dw.p, w, nw * sizeof(float), hipMemcpyHostToDevice, g_stream));
  if (int rc = launch_quantize(dw.as<float>(), out, in, type, dd.as<std::uint8_t>(), ds.as<float>(), nullptr, g_stream))
    return rc;
  LLMI_TRY_HIP(hipMemcpyAsync(data, dd.p, nd, hipMemcpyDeviceToHost, g_stream));
  LLMI_TRY_HIP(hipMemcpyAsync(scales, ds.p, ns * sizeof(float), hipMemcpyDeviceToHost, g_stream));
  LLMI_TRY_HIP(hipStreamSynchronize(g_stream));
  return LLMI_OK;
}

int llmi_hip_weight_upload(const uint8_t* data, const float* scales, size_t out, size_t in, int type,
                           llmi_hip_weight** weight) {
  LLMI_REQUIRE_INIT();
  if (const int rc = check_type(type)) return rc;
  LLMI_REQUIRE(weight != nullptr, "weight_upload: null out-pointer");
  LLMI_REQUIRE(in <= 0x7FFFFFFFu, "weight_upload: in too large");
  *weight = nullptr;
  auto h = std::make_unique<llmi_hip_weight>();
  if (int rc = alloc_matrix(out, in, type, &h->m)) {
    free_matrix(&h->m);
    return rc;
  }
  const std::size_t nd = out * row_bytes(in, type), ns = out * ceil_div(in, kBlock);
  if (nd > 0) {
    DevBuf dd, ds;
    int rc = dd.alloc(nd);
    if (rc == LLMI_OK) rc = ds.alloc(ns * sizeof(float));
    if (rc == LLMI_OK && hipMemcpyAsync(dd.p, data, nd, hipMemcpyHostToDevice, g_stream) != hipSuccess) rc = fail(LLMI_ERR_HIP, "weight_upload: copy");
    if (rc == LLMI_OK && hipMemcpyAsync(ds.p, scales, ns * sizeof(float), hipMemcpyHostToDevice, g_stream) != hipSuccess) rc = fail(LLMI_ERR_HIP, "weight_upload: copy");
    if (rc == LLMI_OK) rc = launch_relayout_to_tiled(dd.as<std::uint8_t>(), ds.as<float>(), h->m, g_stream);
    if (rc == LLMI_OK && hipStreamSynchronize(g_stream) != hipSuccess) rc = fail(LLMI_ERR_HIP, "weight_upload: sync");
    if (rc != LLMI_OK) {
      free_matrix(&h->m);
      return rc;
    }
  }
  *weight = h.release();
  return LLMI_OK;
}

int llmi_hip_weight_from_gguf(const void* blocks, size_t nbytes, size_t out, size_t in, int gguf_type,
                              llmi_hip_weight** weight) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(weight != nullptr, "weight_from_gguf: null out-pointer");
  *weight = nullptr;
  int type = 0;
  std::size_t block_bytes = 0;  // the 2-byte fp16 scale + the packed codes
  switch (gguf_type) {
    case LLMI_GGUF_Q8_0:
      type = LLMI_TYPE_Q8_0;
      block_bytes = 2 + kBlock;
      break;
    case LLMI_GGUF_Q4_0:
      type = LLMI_TYPE_Q4_0;
      block_bytes = 2 + kBlock / 2;
      break;
    default:
      return fail(LLMI_ERR_ARG, "weight_from_gguf: tensor type is not Q8_0/Q4_0");
  }
  LLMI_REQUIRE(out > 0 && in > 0, "weight_from_gguf: out*in does not match its element count");
  LLMI_REQUIRE(in % kBlock == 0, "weight_from_gguf: in is not a multiple of the block size (32)");
  LLMI_REQUIRE(in <= 0x7FFFFFFFu && out <= (std::size_t{1} << 40) / in, "weight_from_gguf: shape too large");
  LLMI_REQUIRE(nbytes == out * (in / kBlock) * block_bytes,
               "weight_from_gguf: unexpected byte size for its declared shape");
  LLMI_REQUIRE(blocks != nullptr, "weight_from_gguf: null blocks");
  auto h = std::make_unique<llmi_hip_weight>();
  if (int rc = alloc_matrix(out, in, type, &h->m)) {
    free_matrix(&h->m);
    return rc;
  }
  DevBuf raw;
  int rc = raw.alloc(nbytes);
  if (rc == LLMI_OK && hipMemcpyAsync(raw.p, blocks, nbytes, hipMemcpyHostToDevice, g_stream) != hipSuccess)
    rc = fail(LLMI_ERR_HIP, "weight_from_gguf: copy");
  if (rc == LLMI_OK) rc = launch_gguf_to_tiled(raw.p, h->m, g_stream);
  if (rc == LLMI_OK && hipStreamSynchronize(g_stream) != hipSuccess) rc = fail(LLMI_ERR_HIP, "weight_from_gguf: sync");
  if (rc != LLMI_OK) {
    free_matrix(&h->m);
    return rc;
  }
  *weight = h.release();
  return LLMI_OK;
}

int llmi_hip_weight_quantize_dev(const float* w, size_t out, size_t in, int type, llmi_hip_weight** weight) {
  LLMI_REQUIRE_INIT();
  if (type != LLMI_TYPE_F32)
    if (const int rc = check_type(type)) return rc;
  LLMI_REQUIRE(weight != nullptr, "weight_quantize: null out-pointer");
  LLMI_REQUIRE(in <= 0x7FFFFFFFu, "weight_quantize: in too large");
  *weight = nullptr;
  auto h = std::make_unique<llmi_hip_weight>();
  if (int rc = alloc_matrix(out, in, type, &h->m)) {
    free_matrix(&h->m);
    return rc;
  }
  if (out > 0 && in > 0) {
    int rc = type == LLMI_TYPE_F32
                 ? (hipMemcpyAsync(h->m.codes, w, out * in * sizeof(float), hipMemcpyDeviceToDevice, g_stream) ==
                            hipSuccess
                        ? LLMI_OK
                        : fail(LLMI_ERR_HIP, "weight_quantize: copy"))
                 : launch_quantize(w, out, in, type, nullptr, nullptr, &h->m, g_stream);
    if (rc == LLMI_OK && hipStreamSynchronize(g_stream) != hipSuccess) rc = fail(LLMI_ERR_HIP, "weight_quantize: sync");
    if (rc != LLMI_OK) {
      free_matrix(&h->m);
      return rc;
    }
  }
  *weight = h.release();
  return LLMI_OK;
}

int llmi_hip_weight_quantize(const float* w, size_t out, size_t in, int type, llmi_hip_weight** weight) {
  LLMI_REQUIRE_INIT();
  if (type != LLMI_TYPE_F32)
    if (const int rc = check_type(type)) return rc;
  DevBuf dw;
  if (int rc = dw.alloc(out * in * sizeof(float))) return rc;
  if (out * in > 0) LLMI_TRY_HIP(hipMemcpyAsync(dw.p, w, out * in * sizeof(float), hipMemcpyHostToDevice, g_stream));
  return llmi_hip_weight_quantize_dev(dw.as<float>(), out, in, type, weight);
}

int llmi_hip_weight_free(llmi_hip_weight* weight) {
  if (weight == nullptr) return LLMI_OK;
  if (g_stream != nullptr) (void)hipStreamSynchronize(g_stream);
  free_matrix(&weight->m);
  delete weight;
  return LLMI_OK;
}

int llmi_hip_weight_download(const llmi_hip_weight* weight, uint8_t* data, float* scales) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(weight != nullptr, "weight_download: null weight");
  const DeviceMatrix& m = weight->m;
  const std::size_t nd = m.out * row_bytes(m.in, m.type), ns = m.out * m.nblk;
  if (nd == 0) return LLMI_OK;
  if (m.type == LLMI_TYPE_F32) {  // the floats themselves; no scales
    LLMI_TRY_HIP(hipMemcpyAsync(data, m.codes, nd, hipMemcpyDeviceToHost, g_stream));
    LLMI_TRY_HIP(hipStreamSynchronize(g_stream));
    return LLMI_OK;
  }
  DevBuf dd, ds;
  if (int rc = dd.alloc(nd)) return rc;
  if (int rc = ds.alloc(ns * sizeof(float))) return rc;
  LLMI_TRY_HIP(hipMemsetAsync(dd.p, 0, nd, g_stream));
  if (int rc = launch_relayout_to_planar(m, dd.as<std::uint8_t>(), ds.as<float>(), g_stream)) return rc;
  LLMI_TRY_HIP(hipMemcpyAsync(data, dd.p, nd, hipMemcpyDeviceToHost, g_stream));
  LLMI_TRY_HIP(hipMemcpyAsync(scales, ds.p, ns * sizeof(float), hipMemcpyDeviceToHost, g_stream));
  LLMI_TRY_HIP(hipStreamSynchronize(g_stream));
  return LLMI_OK;
}

int llmi_hip_weight_info(const llmi_hip_weight* weight, size_t* out, size_t* in, int* type, size_t* byte_size) {
  LLMI_REQUIRE(weight != nullptr, "weight_info: null weight");
  const DeviceMatrix& m = weight->m;
  if (out != nullptr) *out = m.out;
  if (in != nullptr) *in = m.in;
  if (type != nullptr) *type = m.type;
  if (byte_size != nullptr)
    *byte_size = m.out * row_bytes(m.in, m.type) + (m.type == LLMI_TYPE_F32 ? 0 : m.out * m.nblk * sizeof(float));
  return LLMI_OK;
}

size_t llmi_hip_weight_device_bytes(const llmi_hip_weight* weight) {
  return weight == nullptr ? 0 : weight->m.code_bytes + weight->m.scale_bytes;
}

int llmi_hip_dequantize_rows_dev(const llmi_hip_weight* weight, const int32_t* ids, size_t n, float* dst, void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(weight != nullptr, "dequantize_rows: null weight");
  return launch_dequantize_rows(weight->m, ids, n, dst, pick(stream));
}

int llmi_hip_dequantize_row(const llmi_hip_weight* weight, size_t row, float* dst) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(weight != nullptr, "dequantize_row: null weight");
  const DeviceMatrix& m = weight->m;
  LLMI_REQUIRE(row < m.out, "dequantize_row: row out of range");
  if (m.in == 0) return LLMI_OK;
  DevBuf did, dd;
  if (int rc = did.alloc(sizeof(std::int32_t))) return rc;
  if (int rc = dd.alloc(m.in * sizeof(float))) return rc;
  const std::int32_t id = static_cast<std::int32_t>(row);
  LLMI_TRY_HIP(hipMemcpyAsync(did.p, &id, sizeof(id), hipMemcpyHostToDevice, g_stream));
  if (int rc = launch_dequantize_rows(m, did.as<std::int32_t>(), 1, dd.as<float>(), g_stream)) return rc;
  LLMI_TRY_HIP(hipMemcpyAsync(dst, dd.p, m.in * sizeof(float), hipMemcpyDeviceToHost, g_stream));
  LLMI_TRY_HIP(hipStreamSynchronize(g_stream));
  return LLMI_OK;
}

int llmi_hip_matmul_dev(const llmi_hip_weight* weight, const float* x, size_t rows, const float* bias, float* y,
                        void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(weight != nullptr, "matmul: null weight");
  return launch_matmul(weight->m, x, rows, bias, y, pick(stream));
}

int llmi_hip_matmul(const llmi_hip_weight* weight, const float* x, size_t rows, size_t in, size_t out,
                    const float* bias, float* y) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(weight != nullptr, "matmul: null weight");
  const DeviceMatrix& m = weight->m;
  LLMI_REQUIRE(in == m.in && out == m.out, "matmul: in/out do not match the weight's shape");
  if (rows == 0 || out == 0) return LLMI_OK;
  DevBuf dx, db, dy;
  if (int rc = dx.alloc(rows * in * sizeof(float))) return rc;
  if (int rc = dy.alloc(rows * out * sizeof(float))) return rc;
  if (bias != nullptr) {
    if (int rc = db.alloc(out * sizeof(float))) return rc;
    LLMI_TRY_HIP(hipMemcpyAsync(db.p, bias, out * sizeof(float), hipMemcpyHostToDevice, g_stream));
  }
  LLMI_TRY_HIP(hipMemcpyAsync(dx.p, x, rows * in * sizeof(float), hipMemcpyHostToDevice, g_stream));
  if (int rc = launch_matmul(m, dx.as<float>(), rows, db.as<float>(), dy.as<float>(), g_stream)) return rc;
  LLMI_TRY_HIP(hipMemcpyAsync(y, dy.p, rows * out * sizeof(float), hipMemcpyDeviceToHost, g_stream));
  LLMI_TRY_HIP(hipStreamSynchronize(g_stream));
  return LLMI_OK;
}

int llmi_hip_group_create(const llmi_hip_weight* const* w, const float* const* x, const size_t* rows,
                          const float* const* bias, float* const* y, size_t count, llmi_hip_group** out) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(out != nullptr, "group: null output handle");
  *out = nullptr;
  std::vector<GroupEntry> entries;
  if (int rc = group_entries(w, x, rows, bias, y, count, 1, &entries)) return rc;
  auto g = std::make_unique<llmi_hip_group>();
  if (int rc = g->g.build(entries.data(), count)) return rc;
  *out = g.release();
  return LLMI_OK;
}

int llmi_hip_group_launch(const llmi_hip_group* g, void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(g != nullptr, "group: null group");
  return g->g.launch(pick(stream));
}

void llmi_hip_group_free(llmi_hip_group* g) { delete g; }

int llmi_hip_gemm_group_create(const llmi_hip_weight* const* w, const float* const* x, const size_t* rows,
                               const float* const* bias, float* const* y, size_t count, llmi_hip_gemm_group** out) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(out != nullptr, "gemm: null output handle");
  LLMI_REQUIRE(rows != nullptr || count == 0, "gemm: null rows");
  *out = nullptr;
  std::vector<GroupEntry> entries;
  if (int rc = group_entries(w, x, rows, bias, y, count, 0, &entries)) return rc;
  auto g = std::make_unique<llmi_hip_gemm_group>();
  if (int rc = plan_gemm_group(entries.data(), count, &g->plan)) return rc;
  if (gemm_scratch_bytes(g->plan) > 0) {
    LLMI_TRY_HIP(hipMalloc(reinterpret_cast<void**>(&g->scratch), gemm_scratch_bytes(g->plan)));
    bind_gemm_scratch(&g->plan, g->scratch);
  }
  if (int rc = upload_plan(g->plan, g->plan.probs, g->plan.work_prob, g.get())) return rc;
  *out = g.release();
  return LLMI_OK;
}

int llmi_hip_gemm_group_launch(const llmi_hip_gemm_group* g, void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(g != nullptr, "gemm: null group");
  if (int rc = launch_gemm_inputs(g->plan, g->scratch, pick(stream))) return rc;
  for (const GemmLaunch& l : g->plan.launches)
    if (int rc = launch_gemm(g->probs, g->map, l, pick(stream))) return rc;
  return launch_gemm_reduces(g->plan, pick(stream));
}

void llmi_hip_gemm_group_free(llmi_hip_gemm_group* g) { delete g; }

int llmi_hip_matmul_mfma_dev(const llmi_hip_weight* weight, const float* x, size_t rows, const float* bias, float* y,
                             void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(weight != nullptr, "gemm: null weight");
  return llmi_hip::launch_gemm_single(weight->m, x, rows, bias, y, pick(stream));
}

int llmi_hip_matmul_mfma_noalloc_dev(const llmi_hip_weight* weight, const float* x, size_t rows, const float* bias,
                                     float* y, void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(weight != nullptr, "matmul_mfma_noalloc: null weight");
  return llmi_hip::launch_gemm_noalloc(g_device, weight->m, x, rows, bias, y, pick(stream));
}

}  // extern "C"
