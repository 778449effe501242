// Device-resident Llama / Qwen2 decoder for the quantized-weight path:
// Transformer::load / new_cache / forward_cached / generate_greedy_cached of
// the reference (src/model/transformer.cpp:26-67, :182-327) with every
// weight matrix, activation and the KV cache in HBM.  Token ids go in, logits
// (or greedy ids) come out.
//
// Every glue operation restates the reference's arithmetic so that logits
// are bit-identical to the reference's on the same weights:
//   rmsnorm   kernels.cpp:115-120  double sum of squares, float scale,
//                                  y = w * (x * scale)
//   rope      kernels.cpp:122-134  cos/sin of the float angle pos*inv_freq[i]
//                                  (host sincosf tables), fused as
//                                  v[i] = fma(a,c,-(b*s)), v[i+h] = fma(b,c,a*s)
//   attention transformer.cpp:263-282  scores = dot(q, k_s) * (1/sqrt(hd))
//                                  with kernels::dot's summation order,
//                                  softmax (float max, expf, double sum,
//                                  float reciprocal), out = sequential
//                                  fma(p_s, v_s[i], out[i]) over positions
//   silu*up   kernels.cpp:148      x / (1 + expf(-x)), times up
//   residual  transformer.cpp:284  x += proj (GEMV epilogue)
//   argmax    transformer.cpp:22   first maximum
// expf is the exact restatement of the host libm's (exact_math.hpp).  The two
// double-precision sums are reduced in parallel; their float result is taken
// only when an error bound proves the reference's sequential sum rounds to
// the same float, and recomputed sequentially otherwise.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"
#include "exact_math.hpp"
#include "glue_math.hpp"

namespace llmi_hip {
namespace {

constexpr int kThreads = 256;

// ------------------------------------------------------------ reductions
__device__ __forceinline__ double block_sum_double(double v, double* red) {
  // Fixed-shape tree over the 256 threads: deterministic.
  const int tid = threadIdx.x;
  red[tid] = v;
  __syncthreads();
  for (int stride = kThreads / 2; stride > 0; stride >>= 1) {
    if (tid < stride) red[tid] = red[tid] + red[tid + stride];
    __syncthreads();
  }
  const double r = red[0];
  __syncthreads();
  return r;
}

__device__ __forceinline__ float block_max_float(float v, float* red) {
  const int tid = threadIdx.x;
  red[tid] = v;
  __syncthreads();
  for (int stride = kThreads / 2; stride > 0; stride >>= 1) {
    if (tid < stride) red[tid] = fmaxf(red[tid], red[tid + stride]);
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

// ------------------------------------------------------------ rmsnorm
// One workgroup per row: y = w * (x * scale), scale from the double sum of
// squares (kernels.cpp:115-120).
__global__ void __launch_bounds__(kThreads) rmsnorm_rows(const float* __restrict__ x, const float* __restrict__ w,
                                                         float* __restrict__ y, int n, float eps) {
  __shared__ double red[kThreads];
  __shared__ float scale_s;
  const float* xr = x + static_cast<std::size_t>(blockIdx.x) * n;
  float* yr = y + static_cast<std::size_t>(blockIdx.x) * n;
  double part = 0.0;
  for (int i = threadIdx.x; i < n; i += kThreads) {
    const double v = static_cast<double>(xr[i]);
    part = __builtin_fma(v, v, part);
  }
  const double ss = block_sum_double(part, red);
  if (threadIdx.x == 0) {
    // The function ss -> scale is monotone; the reference's sequential sum
    // lies in [lo, hi].  If both ends give one float, that is the answer.
    const double slack = sum_slack(n) * ss;
    const float a = rms_scale(ss - slack, n, eps);
    const float b = rms_scale(ss + slack, n, eps);
    float sc = rms_scale(ss, n, eps);
    if (a != b) {
      double seq = 0.0;
      for (int i = 0; i < n; ++i) {
        const double v = static_cast<double>(xr[i]);
        seq = __builtin_fma(v, v, seq);
      }
      sc = rms_scale(seq, n, eps);
    }
    scale_s = sc;
  }
  __syncthreads();
  const float sc = scale_s;
  for (int i = threadIdx.x; i < n; i += kThreads) yr[i] = w[i] * (xr[i] * sc);
}

// --------------------------------------------------------- rope + cache
// grid.x = token t.  q [T][nh][hd] is rotated in place; k [T][nkv][hd] is
// rotated into the cache, v copied: cache[(kvh*cap + pos)*hd + i].
__global__ void __launch_bounds__(kThreads) rope_and_cache(float* __restrict__ q, const float* __restrict__ knew,
                                                           const float* __restrict__ vnew, float* __restrict__ kc,
                                                           float* __restrict__ vc, const float* __restrict__ cos_t,
                                                           const float* __restrict__ sin_t, int nh, int nkv, int hd,
                                                           int cap, int base) {
  const int t = blockIdx.x;
  const int pos = base + t;
  const int half = hd / 2;
  const float* cr = cos_t + static_cast<std::size_t>(pos) * half;
  const float* sr = sin_t + static_cast<std::size_t>(pos) * half;
  for (int e = threadIdx.x; e < nh * half; e += kThreads) {
    const int h = e / half, i = e % half;
    float* v = q + (static_cast<std::size_t>(t) * nh + h) * hd;
    const float a = v[i], b = v[i + half], c = cr[i], s = sr[i];
    v[i] = __builtin_fmaf(a, c, -(b * s));
    v[i + half] = __builtin_fmaf(b, c, a * s);
  }
  for (int e = threadIdx.x; e < nkv * half; e += kThreads) {
    const int h = e / half, i = e % half;
    const float* v = knew + (static_cast<std::size_t>(t) * nkv + h) * hd;
    float* dst = kc + (static_cast<std::size_t>(h) * cap + pos) * hd;
    const float a = v[i], b = v[i + half], c = cr[i], s = sr[i];
    dst[i] = __builtin_fmaf(a, c, -(b * s));
    dst[i + half] = __builtin_fmaf(b, c, a * s);
  }
  for (int e = threadIdx.x; e < nkv * hd; e += kThreads) {
    const int h = e / hd, i = e % hd;
    vc[(static_cast<std::size_t>(h) * cap + pos) * hd + i] = vnew[(static_cast<std::size_t>(t) * nkv + h) * hd + i];
  }
}

// ------------------------------------------------------------- attention
// kernels::dot (kernels.cpp:41-95, the AVX2 build): 16 fused lanes over
// 16-element chunks reduced (j + j+8), (+4), (+2), (+1); then the scalar
// tail: 8 fused lanes over 8-element chunks, then up to 7 leftovers (when 4
// or more remain, the first 4 products are rounded on their own and added in
// order), the 8 lanes reduced pairwise, plus the leftovers.
__device__ __forceinline__ float ref_dot(const float* __restrict__ a, const float* __restrict__ b, int n) {
  float lane[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) lane[j] = 0.0f;
  int i = 0;
  for (; i + 16 <= n; i += 16) {
#pragma unroll
    for (int j = 0; j < 16; ++j) lane[j] = __builtin_fmaf(a[i + j], b[i + j], lane[j]);
  }
  float s8[8], s4[4];
#pragma unroll
  for (int j = 0; j < 8; ++j) s8[j] = lane[j] + lane[j + 8];
#pragma unroll
  for (int j = 0; j < 4; ++j) s4[j] = s8[j] + s8[j + 4];
  const float head = (s4[0] + s4[2]) + (s4[1] + s4[3]);
  return head + ref_dot_rest(a + i, b + i, n - i);
}

__device__ __forceinline__ float recip_float(double s) { return static_cast<float>(1.0 / s); }

// Softmax over sc[0..npos) in LDS (kernels.cpp:136-146): float max, exact
// expf, double sum (order-checked), p = e * float(1/sum).  Ends with a
// barrier; every thread of the 256 takes part.
__device__ __forceinline__ void softmax_lds(float* sc, int npos, float mx_local, double* red_d, float* red_f,
                                            float* inv_s) {
  const float mx = block_max_float(mx_local, red_f);
  double part = 0.0;
  for (int s = threadIdx.x; s < npos; s += kThreads) {
    const float e = exact::expf(sc[s] - mx);
    sc[s] = e;
    part += static_cast<double>(e);
  }
  const double sum = block_sum_double(part, red_d);  // ends with a barrier: sc[] is complete
  if (threadIdx.x == 0) {
    const double slack = sum_slack(npos) * sum;
    float inv = recip_float(sum);
    if (recip_float(sum - slack) != recip_float(sum + slack)) {
      double seq = 0.0;
      for (int s = 0; s < npos; ++s) seq += static_cast<double>(sc[s]);
      inv = recip_float(seq);
    }
    *inv_s = inv;
  }
  __syncthreads();
  const float inv = *inv_s;
  for (int s = threadIdx.x; s < npos; s += kThreads) sc[s] = sc[s] * inv;
  __syncthreads();
}

// Generic head size: one thread per position with ref_dot, the P.V chain
// read straight from the cache.  grid = (head, token); dynamic LDS: scores.
__global__ void __launch_bounds__(kThreads) attention_generic(const float* __restrict__ q, const float* __restrict__ kc,
                                                              const float* __restrict__ vc, float* __restrict__ out,
                                                              int nh, int nkv, int hd, int cap, int base, float scale) {
  extern __shared__ float sc[];
  __shared__ double red_d[kThreads];
  __shared__ float red_f[kThreads];
  __shared__ float inv_s;
  const int h = blockIdx.x;
  const int t = blockIdx.y;
  const int npos = base + t + 1;
  const int kvh = h / (nh / nkv);
  const float* qv = q + (static_cast<std::size_t>(t) * nh + h) * hd;
  const float* kh = kc + static_cast<std::size_t>(kvh) * cap * hd;
  const float* vh = vc + static_cast<std::size_t>(kvh) * cap * hd;
  float mx_local = -__builtin_inff();
  for (int s = threadIdx.x; s < npos; s += kThreads) {
    const float v = ref_dot(qv, kh + static_cast<std::size_t>(s) * hd, hd) * scale;
    sc[s] = v;
    mx_local = fmaxf(mx_local, v);
  }
  softmax_lds(sc, npos, mx_local, red_d, red_f, &inv_s);
  for (int i = threadIdx.x; i < hd; i += kThreads) {
    float acc = 0.0f;
    for (int s = 0; s < npos; ++s) acc = __builtin_fmaf(sc[s], vh[static_cast<std::size_t>(s) * hd + i], acc);
    out[(static_cast<std::size_t>(t) * nh + h) * hd + i] = acc;
  }
}

// head_dim a multiple of 16 (64 for SmolLM2 and Qwen2.5).
//  scores: 16 lanes per position; lane j accumulates elements j, j+16, ...
//          with fused multiply-adds exactly like the AVX2 build's 16
//          accumulators, and the xor-8/4/2/1 shuffle tree is its horizontal
//          sum (j+8, then +4, +2, +1); + 0.0f is the empty scalar tail.
//  P.V:    wavefront 0 runs out[i] = fma(p_s, v_s[i], out[i]) over s in
//          order from LDS tiles of V that wavefronts 1-3 prefetch (double
//          buffered), so the chain never waits on global memory.
// grid = (head, token); dynamic LDS: scores (npos floats) then 2 V tiles.
constexpr int kVTile = 64;  // positions per V tile

__global__ void __launch_bounds__(kThreads) attention_hd16(const float* __restrict__ q, const float* __restrict__ kc,
                                                           const float* __restrict__ vc, float* __restrict__ out,
                                                           int nh, int nkv, int hd, int cap, int base, float scale,
                                                           int sc_len) {
  extern __shared__ float lds_dyn[];
  float* sc = lds_dyn;
  float* vtile = lds_dyn + sc_len;  // [2][kVTile][hd]
  __shared__ double red_d[kThreads];
  __shared__ float red_f[kThreads];
  __shared__ float inv_s;
  const int h = blockIdx.x;
  const int t = blockIdx.y;
  const int npos = base + t + 1;
  const int kvh = h / (nh / nkv);
  const float* qv = q + (static_cast<std::size_t>(t) * nh + h) * hd;
  const float* kh = kc + static_cast<std::size_t>(kvh) * cap * hd;
  const float* vh = vc + static_cast<std::size_t>(kvh) * cap * hd;
  const int tid = threadIdx.x;
  const int j = tid & 15;   // accumulator lane
  const int grp = tid >> 4;  // 16 positions per pass of the 256 threads
  const int nchunk = hd / 16;

  float mx_local = -__builtin_inff();
  for (int s0 = 0; s0 < npos; s0 += kThreads / 16) {
    const int s = s0 + grp;
    float lane = 0.0f;
    if (s < npos) {
      const float* kr = kh + static_cast<std::size_t>(s) * hd;
      for (int c = 0; c < nchunk; ++c) lane = __builtin_fmaf(qv[16 * c + j], kr[16 * c + j], lane);
    }
    lane = lane + __shfl_xor(lane, 8, 16);
    lane = lane + __shfl_xor(lane, 4, 16);
    lane = lane + __shfl_xor(lane, 2, 16);
    lane = lane + __shfl_xor(lane, 1, 16);
    if (s < npos && j == 0) {
      const float v = (lane + 0.0f) * scale;
      sc[s] = v;
      mx_local = fmaxf(mx_local, v);
    }
  }
  softmax_lds(sc, npos, mx_local, red_d, red_f, &inv_s);

  const int wave = tid >> 6;
  const int tile_floats = kVTile * hd;
  const int ntile = (npos + kVTile - 1) / kVTile;
  auto load_tile = [&](int k, float* dst, int first_thread, int nthreads) {
    const int s0 = k * kVTile;
    const int count = min(kVTile, npos - s0) * hd;
    const float* src = vh + static_cast<std::size_t>(s0) * hd;
    for (int e = tid - first_thread; e < count; e += nthreads) dst[e] = src[e];
  };
  load_tile(0, vtile, 0, kThreads);
  __syncthreads();
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // hd <= 256: lanes own i = lane + 64r
  for (int k = 0; k < ntile; ++k) {
    float* cur = vtile + (k & 1) * tile_floats;
    if (wave != 0) {
      if (k + 1 < ntile) load_tile(k + 1, vtile + ((k + 1) & 1) * tile_floats, 64, kThreads - 64);
    } else {
      const int s0 = k * kVTile;
      const int cnt = min(kVTile, npos - s0);
      for (int r = 0; r < 4; ++r) {
        const int i = tid + 64 * r;
        if (i < hd) {
          float a = acc[r];
          for (int s = 0; s < cnt; ++s) a = __builtin_fmaf(sc[s0 + s], cur[s * hd + i], a);
          acc[r] = a;
        }
      }
    }
    __syncthreads();
  }
  if (wave == 0) {
    for (int r = 0; r < 4; ++r) {
      const int i = tid + 64 * r;
      if (i < hd) out[(static_cast<std::size_t>(t) * nh + h) * hd + i] = acc[r];
    }
  }
}

// ------------------------------------------------ prefill attention, hd 64
// The same arithmetic as attention_hd16 with one workgroup per (KV head,
// tile of tq tokens).  Its rows are the G = nh / nkv query heads of that KV
// head for each token of the tile (row = tt * G + g, at most ROWS = 16 or
// 32), and they share every K and V row the workgroup stages.  Phases:
//  scores  64-position K tiles in LDS (double buffered through registers);
//          thread (rg, pg) computes rows rg + RG*r (r < 4, RG = ROWS / 4) x
//          positions pg + (64 / P)*p (p < P = RG / 4): each score is 16 fused
//          lanes (lane j over elements j, j+16, j+32, j+48), lanes j and j+8
//          added, then j and j+4, then (0 + 2) + (1 + 3) -- kernels::dot's
//          order -- plus 0.0f, times scale.  Scores go to LDS
//          sc[position][row].
//  softmax thread (row, phase): float max, exact expf and double partial
//          sums over positions phase, phase + 256/ROWS, ...; the partials are
//          added in a fixed order and the float reciprocal is taken from that
//          sum when the order bound proves the sequential sum gives the same
//          float, otherwise one thread re-adds the row in order.
//  P.V     64-position V tiles in LDS; thread (rp, dq) runs the chains of
//          rows RP*rp.. (RP = ROWS / 16) x dims 4dq..4dq+3 in position order:
//          out = fma(p_s, v_s[i], out).  Positions every row of the
//          workgroup attends to run unchecked; the diagonal ones are checked
//          per row.
constexpr int kAttnTile = 64;
constexpr int kAttnStride = 68;  // LDS floats per staged row: 16-byte aligned, consecutive rows 4 banks apart
template <int ROWS>
constexpr std::size_t attn_static_lds() {
  return (ROWS * kAttnStride + 2 * kAttnTile * kAttnStride + (kThreads / ROWS) * ROWS + ROWS) * sizeof(float) +
         (kThreads / ROWS) * ROWS * sizeof(double) + 256;
}

// One thread's share (4 float4) of a 64 x 64 tile of the cache starting at
// position s0; positions at or past npos are not read.
__device__ __forceinline__ void attn_load_tile(const float* __restrict__ src, int s0, int npos, float4 (&r)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = threadIdx.x + kThreads * i;
    const int p = s0 + (f >> 4);
    if (p < npos) r[i] = *reinterpret_cast<const float4*>(src + static_cast<std::size_t>(p) * 64 + 4 * (f & 15));
  }
}
__device__ __forceinline__ void attn_store_tile(float* dst, const float4 (&r)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int f = threadIdx.x + kThreads * i;
    *reinterpret_cast<float4*>(dst + (f >> 4) * kAttnStride + 4 * (f & 15)) = r[i];
  }
}

// Lanes j0..j0+3 of the 16-lane dot for 4 rows (RG apart) x P positions
// (PS apart).
template <int RG, int P, int PS>
__device__ __forceinline__ void attn_quad(const float* q0, const float* k0, int j0, float (&L)[4][P][4]) {
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int u = 0; u < 4; ++u) L[r][p][u] = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    float4 qv[4], kv[P];
#pragma unroll
    for (int r = 0; r < 4; ++r) qv[r] = *reinterpret_cast<const float4*>(q0 + RG * r * kAttnStride + 16 * c + j0);
#pragma unroll
    for (int p = 0; p < P; ++p) kv[p] = *reinterpret_cast<const float4*>(k0 + PS * p * kAttnStride + 16 * c + j0);
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int p = 0; p < P; ++p) {
        L[r][p][0] = __builtin_fmaf(qv[r].x, kv[p].x, L[r][p][0]);
        L[r][p][1] = __builtin_fmaf(qv[r].y, kv[p].y, L[r][p][1]);
        L[r][p][2] = __builtin_fmaf(qv[r].z, kv[p].z, L[r][p][2]);
        L[r][p][3] = __builtin_fmaf(qv[r].w, kv[p].w, L[r][p][3]);
      }
  }
}

template <int ROWS>
__global__ void __launch_bounds__(kThreads) attention_rows64(const float* __restrict__ q, const float* __restrict__ kc,
                                                             const float* __restrict__ vc, float* __restrict__ out,
                                                             int nh, int nkv, int cap, int base, int T, int tq,
                                                             float scale) {
  constexpr int RG = ROWS / 4;            // row groups of the scores phase
  constexpr int PG = kThreads / RG;       // position groups
  constexpr int P = kAttnTile / PG;       // positions per thread
  constexpr int PH = kThreads / ROWS;     // softmax phases per row
  constexpr int RP = ROWS / 16;           // P.V rows per thread
  static_assert(P >= 1 && RP >= 1 && P * PG == kAttnTile, "attention_rows64: ROWS must be 16 or 32");
  extern __shared__ float sc[];  // [position][ROWS]
  __shared__ __attribute__((aligned(16))) float qs[ROWS * kAttnStride];
  __shared__ __attribute__((aligned(16))) float tile[2][kAttnTile * kAttnStride];
  __shared__ double red_d[PH][ROWS];
  __shared__ float red_f[PH][ROWS];
  __shared__ float inv_s[ROWS];
  const int G = nh / nkv;
  const int kvh = blockIdx.y;
  const int t0 = (static_cast<int>(gridDim.x) - 1 - static_cast<int>(blockIdx.x)) * tq;  // longest rows first
  const int ntok = min(tq, T - t0);
  const int nrows = ntok * G;
  const int npos_max = base + t0 + ntok;  // positions of the tile's last token
  const int npos_min = base + t0 + 1;     // positions every row attends to
  const float* kh = kc + static_cast<std::size_t>(kvh) * cap * 64;
  const float* vh = vc + static_cast<std::size_t>(kvh) * cap * 64;
  const int tid = threadIdx.x;

  for (int f = tid; f < ROWS * 16; f += kThreads) {
    const int row = f >> 4, e4 = f & 15;
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (row < nrows) {
      const int tt = row / G, g = row - tt * G;
      v = *reinterpret_cast<const float4*>(q + (static_cast<std::size_t>(t0 + tt) * nh + kvh * G + g) * 64 + 4 * e4);
    }
    *reinterpret_cast<float4*>(qs + row * kAttnStride + 4 * e4) = v;
  }

  // ---- scores
  const int ntile = (npos_max + kAttnTile - 1) / kAttnTile;
  float4 st[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) st[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  attn_load_tile(kh, 0, npos_max, st);
  attn_store_tile(tile[0], st);
  if (ntile > 1) attn_load_tile(kh, kAttnTile, npos_max, st);
  __syncthreads();
  {
    const int rg = tid % RG, pg = tid / RG;
    const float* q0 = qs + rg * kAttnStride;
    for (int k = 0; k < ntile; ++k) {
      const float* k0 = tile[k & 1] + pg * kAttnStride;
      float A[4][P][4], B[4][P][4], C[4][P][4];
      attn_quad<RG, P, PG>(q0, k0, 0, A);
      attn_quad<RG, P, PG>(q0, k0, 8, B);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
          for (int u = 0; u < 4; ++u) A[r][p][u] = A[r][p][u] + B[r][p][u];  // lanes j + (j + 8), j < 4
      attn_quad<RG, P, PG>(q0, k0, 4, B);
      attn_quad<RG, P, PG>(q0, k0, 12, C);
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int p = 0; p < P; ++p) {
          float s4[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) s4[u] = A[r][p][u] + (B[r][p][u] + C[r][p][u]);  // + lanes (j+4) + (j+12)
          const float head = (s4[0] + s4[2]) + (s4[1] + s4[3]);
          sc[(k * kAttnTile + pg + PG * p) * ROWS + rg + RG * r] = (head + 0.0f) * scale;
        }
      if (k + 1 < ntile) {
        attn_store_tile(tile[(k + 1) & 1], st);
        if (k + 2 < ntile) attn_load_tile(kh, (k + 2) * kAttnTile, npos_max, st);
      }
      __syncthreads();
    }
  }
  attn_load_tile(vh, 0, npos_max, st);  // in flight during the softmax

  // ---- softmax
  {
    const int row = tid % ROWS, ph = tid / ROWS;
    const int np = row < nrows ? base + t0 + row / G + 1 : 0;
    float m = -__builtin_inff();
    for (int s = ph; s < np; s += PH) m = fmaxf(m, sc[s * ROWS + row]);
    red_f[ph][row] = m;
    __syncthreads();
    float mx = red_f[0][row];
#pragma unroll
    for (int i = 1; i < PH; ++i) mx = fmaxf(mx, red_f[i][row]);
    double part = 0.0;
    for (int s = ph; s < np; s += PH) {
      const float e = exact::expf(sc[s * ROWS + row] - mx);
      sc[s * ROWS + row] = e;
      part += static_cast<double>(e);
    }
    red_d[ph][row] = part;
    __syncthreads();
    if (ph == 0 && row < nrows) {
      double sum = red_d[0][row];
#pragma unroll
      for (int i = 1; i < PH; ++i) sum = sum + red_d[i][row];
      const double slack = sum_slack(np) * sum;
      float inv = recip_float(sum);
      if (recip_float(sum - slack) != recip_float(sum + slack)) {
        double seq = 0.0;
        for (int s = 0; s < np; ++s) seq += static_cast<double>(sc[s * ROWS + row]);
        inv = recip_float(seq);
      }
      inv_s[row] = inv;
    }
    __syncthreads();
    if (np > 0) {
      const float inv = inv_s[row];
      for (int s = ph; s < np; s += PH) sc[s * ROWS + row] = sc[s * ROWS + row] * inv;
    }
  }

  // ---- P.V
  attn_store_tile(tile[0], st);
  if (ntile > 1) attn_load_tile(vh, kAttnTile, npos_max, st);
  __syncthreads();
  const int rp = tid >> 4, dq = tid & 15;
  const int ra = RP * rp;
  int np_r[RP];
#pragma unroll
  for (int i = 0; i < RP; ++i) np_r[i] = ra + i < nrows ? base + t0 + (ra + i) / G + 1 : npos_max;
  float acc[RP][4];
#pragma unroll
  for (int i = 0; i < RP; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  const auto step = [&](const float* vt, int s, int u, bool checked) {
    float p[RP];
    if constexpr (RP == 2) {
      const float2 p2 = *reinterpret_cast<const float2*>(sc + s * ROWS + ra);
      p[0] = p2.x;
      p[1] = p2.y;
    } else {
      p[0] = sc[s * ROWS + ra];
    }
    const float4 v = *reinterpret_cast<const float4*>(vt + u * kAttnStride + 4 * dq);
#pragma unroll
    for (int i = 0; i < RP; ++i) {
      if (!checked || s < np_r[i]) {
        acc[i][0] = __builtin_fmaf(p[i], v.x, acc[i][0]);
        acc[i][1] = __builtin_fmaf(p[i], v.y, acc[i][1]);
        acc[i][2] = __builtin_fmaf(p[i], v.z, acc[i][2]);
        acc[i][3] = __builtin_fmaf(p[i], v.w, acc[i][3]);
      }
    }
  };
  for (int k = 0; k < ntile; ++k) {
    const float* vt = tile[k & 1];
    const int s0 = k * kAttnTile;
    const int cnt = min(kAttnTile, npos_max - s0);
    const int full = max(0, min(cnt, npos_min - s0));
    int u = 0;
    for (; u + 8 <= full; u += 8) {
#pragma unroll
      for (int w = 0; w < 8; ++w) step(vt, s0 + u + w, u + w, false);
    }
    for (; u < full; ++u) step(vt, s0 + u, u, false);
    for (; u < cnt; ++u) step(vt, s0 + u, u, true);
    if (k + 1 < ntile) {
      attn_store_tile(tile[(k + 1) & 1], st);
      if (k + 2 < ntile) attn_load_tile(vh, (k + 2) * kAttnTile, npos_max, st);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < RP; ++i) {
    const int row = ra + i;
    if (row < nrows) {
      const int tt = row / G, g = row - tt * G;
      *reinterpret_cast<float4*>(out + (static_cast<std::size_t>(t0 + tt) * nh + kvh * G + g) * 64 + 4 * dq) =
          make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
    }
  }
}

// ------------------------------------------------- decode attention (T = 1)
// The same arithmetic as attention_hd16 for one new token, restructured for
// latency: the one-workgroup-per-head kernel spends ~140 ns per cached
// position waiting on K and V loads, because each output element is one
// sequential chain over the positions.  Here
//  1. attn_scores_1: grid (position tiles of 64, KV heads) computes every
//     score of the GQA group with all K loads of a thread issued at once, and
//     writes them to the cache's score buffer [head][cap];
//  2. attn_pv_1: grid (query heads, head_dim / 16) -- each workgroup runs
//     the softmax of its head and the P.V chains of 16 output columns, with
//     the V slice (positions x 16 columns) staged transposed in LDS first,
//     so the chains read 4 positions per 16-byte LDS load and never wait on
//     HBM.
// Positions are padded to a multiple of 4 with p = 0 and v = 0: the chains
// never hold -0.0 (they start at +0.0 and p >= 0), so fma(0, 0, acc) == acc.
constexpr int kScoreTile = 64;  // positions per attn_scores_1 workgroup

// v + (v of the lane n above, within each row of 16 lanes): one DPP add.
template <int N>
__device__ __forceinline__ float add_row_shl(float v) {
  const int src = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + N, 0xF, 0xF, true);
  return v + __int_as_float(src);
}

// RoPE of the new token is fused (rope_and_cache's arithmetic): q is rotated
// while it is staged, and the workgroup holding position npos - 1 rotates
// the new k (knew), uses it and writes it to the cache.  cr/sr: the cos/sin
// table rows of that position.
template <int NCH>  // head_dim / 16
__global__ void __launch_bounds__(kThreads) attn_scores_1(const float* __restrict__ q, const float* __restrict__ knew,
                                                          float* __restrict__ kc, const float* __restrict__ cos_t,
                                                          const float* __restrict__ sin_t, float* __restrict__ scores,
                                                          int nh, int nkv, int cap, int npos, float scale) {
  constexpr int hd = 16 * NCH, half = hd / 2;
  __shared__ float qs[16 * hd];  // the group's query heads (G <= 16)
  const int s0 = blockIdx.x * kScoreTile;
  const int kvh = blockIdx.y;
  const int G = nh / nkv;
  const int j = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const int pos = npos - 1;
  const float* cr = cos_t + static_cast<std::size_t>(pos) * half;
  const float* sr = sin_t + static_cast<std::size_t>(pos) * half;
  float* kh = kc + static_cast<std::size_t>(kvh) * cap * hd;
  float kv[kScoreTile / 16][NCH];
#pragma unroll
  for (int p = 0; p < kScoreTile / 16; ++p) {
    const int s = s0 + 16 * p + grp;
    if (s == pos) {
      const float* kn = knew + static_cast<std::size_t>(kvh) * hd;
#pragma unroll
      for (int c = 0; c < NCH / 2; ++c) {
        const int i = 16 * c + j;
        const float a = kn[i], b = kn[i + half], cs = cr[i], sn = sr[i];
        kv[p][c] = __builtin_fmaf(a, cs, -(b * sn));
        kv[p][c + NCH / 2] = __builtin_fmaf(b, cs, a * sn);
      }
#pragma unroll
      for (int c = 0; c < NCH; ++c) kh[static_cast<std::size_t>(s) * hd + 16 * c + j] = kv[p][c];
    } else {
#pragma unroll
      for (int c = 0; c < NCH; ++c) kv[p][c] = s < npos ? kh[static_cast<std::size_t>(s) * hd + 16 * c + j] : 0.0f;
    }
  }
  for (int e = threadIdx.x; e < G * half; e += kThreads) {
    const int g = e / half, i = e % half;
    const float* qh = q + static_cast<std::size_t>(kvh * G + g) * hd;
    const float a = qh[i], b = qh[i + half], cs = cr[i], sn = sr[i];
    qs[g * hd + i] = __builtin_fmaf(a, cs, -(b * sn));
    qs[g * hd + i + half] = __builtin_fmaf(b, cs, a * sn);
  }
  __syncthreads();
  for (int g = 0; g < G; ++g) {
    const int h = kvh * G + g;
    float qv[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) qv[c] = qs[g * hd + 16 * c + j];
#pragma unroll
    for (int p = 0; p < kScoreTile / 16; ++p) {
      float lane = 0.0f;
#pragma unroll
      for (int c = 0; c < NCH; ++c) lane = __builtin_fmaf(qv[c], kv[p][c], lane);
      // Lane 0 of each row of 16 ends with ((l0+l8)+(l4+l12)) + ... -- the
      // j+8, +4, +2, +1 tree of the 16 accumulators.
      lane = add_row_shl<8>(lane);
      lane = add_row_shl<4>(lane);
      lane = add_row_shl<2>(lane);
      lane = add_row_shl<1>(lane);
      const int s = s0 + 16 * p + grp;
      if (j == 0 && s < npos) scores[static_cast<std::size_t>(h) * cap + s] = (lane + 0.0f) * scale;
    }
  }
}

// grid (query heads, head_dim / 16), 256 threads.  Each workgroup first
// issues its loads: the head's scores (registers, positions tid, tid + 256,
// ...) and the first kPvBatch * 256 float4s of its V slice (positions x 16
// columns).  While the V loads are in flight it runs the head's softmax on
// the scores (softmax_lds's arithmetic: float max, exact expf with an LDS
// copy of its table, double sum taken when the error bound proves it rounds
// like the sequential sum, else summed sequentially); then it parks p and
// the transposed V slice in LDS and lanes 0-15 run the P.V chains of the 16
// columns.  Dynamic LDS: p[npad] then vt[16][npad + 4] (npad = npos rounded
// up to 64, zero-padded; rows start 4 banks apart).  The padding adds
// fma(0, 0, acc) = acc: acc starts at +0 and never becomes -0.
constexpr int kPvCols = 16;
constexpr int kPvBatch = 16;   // V float4 loads per thread per round (1024 positions)
constexpr int kPvScores = 10;  // score registers per thread: npos <= 2560
constexpr int kPvChain = 8;    // float4 reads per operand per chain round (16 LDS reads in flight)

__host__ __device__ __forceinline__ int pv_pad(int npos) { return (npos + 63) & ~63; }

__device__ __forceinline__ float row_max16(float v) {
  // Lanes whose source is outside the row keep their own value.
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x111, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x112, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x114, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x118, 0xF, 0xF, false)));
  return v;
}

// The new token's v (vnew) is read in place of cache row npos - 1, and the
// first head of each group writes its slice of it to the cache.
template <int NCH>
__global__ void __launch_bounds__(kThreads) attn_pv_1(const float* __restrict__ scores, const float* __restrict__ vnew,
                                                      float* __restrict__ vc, float* __restrict__ out, int nh, int nkv,
                                                      int cap, int npos) {
  constexpr int hd = 16 * NCH;
  constexpr int kRows = kThreads / 16;
  extern __shared__ float4 pv_lds[];  // 16-byte aligned: the chains read float4
  __shared__ std::uint64_t exp_tab[32];
  __shared__ float red_f[kRows];
  __shared__ double red_d[kRows];
  float* lds = reinterpret_cast<float*>(pv_lds);
  const int h = blockIdx.x;
  const int kvh = h / (nh / nkv);
  const int i0 = blockIdx.y * kPvCols;
  const int npad = pv_pad(npos);
  const int stride = npad + 4;
  float* p = lds;
  float* vt = lds + npad;
  const int tid = threadIdx.x;
  if (tid < 32) exp_tab[tid] = exact::kExp2Tab[tid];

  const float* vh = vc + static_cast<std::size_t>(kvh) * cap * hd + i0;
  const float* vn = vnew + static_cast<std::size_t>(kvh) * hd + i0;
  const float* src = scores + static_cast<std::size_t>(h) * cap;
  if (h % (nh / nkv) == 0 && tid < kPvCols)
    vc[(static_cast<std::size_t>(kvh) * cap + npos - 1) * hd + i0 + tid] = vn[tid];

  float sv[kPvScores];
#pragma unroll
  for (int u = 0; u < kPvScores; ++u) {
    const int sp = u * kThreads + tid;
    sv[u] = sp < npos ? src[sp] : -__builtin_inff();
  }
  // V element e: position e / 4, columns 4 * (e % 4) .. + 3 of the slice.
  const int n4 = npad * 4;
  float4 v[kPvBatch];
  const auto load_v = [&](int e0) {
#pragma unroll
    for (int u = 0; u < kPvBatch; ++u) {
      const int e = e0 + u * kThreads + tid;
      const int sp = e >> 2;
      v[u] = sp < npos - 1 ? *reinterpret_cast<const float4*>(vh + static_cast<std::size_t>(sp) * hd + 4 * (e & 3))
             : sp == npos - 1 ? *reinterpret_cast<const float4*>(vn + 4 * (e & 3))
                              : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  };
  const auto store_v = [&](int e0) {
#pragma unroll
    for (int u = 0; u < kPvBatch; ++u) {
      const int e = e0 + u * kThreads + tid;
      if (e < n4) {
        const int sp = e >> 2, qd = e & 3;
        vt[(4 * qd + 0) * stride + sp] = v[u].x;
        vt[(4 * qd + 1) * stride + sp] = v[u].y;
        vt[(4 * qd + 2) * stride + sp] = v[u].z;
        vt[(4 * qd + 3) * stride + sp] = v[u].w;
      }
    }
  };
  load_v(0);

  // Softmax while the V loads are in flight.
  float mx = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < kPvScores; ++u) mx = fmaxf(mx, sv[u]);
  mx = row_max16(mx);
  if ((tid & 15) == 15) red_f[tid >> 4] = mx;
  __syncthreads();  // red_f and exp_tab
  mx = red_f[0];
#pragma unroll
  for (int r = 1; r < kRows; ++r) mx = fmaxf(mx, red_f[r]);
  double part = 0.0;
#pragma unroll
  for (int u = 0; u < kPvScores; ++u) {
    const int sp = u * kThreads + tid;
    if (sp < npos) {
      const float e = exact::expf_with(sv[u] - mx, exp_tab);
      sv[u] = e;
      p[sp] = e;
      part += static_cast<double>(e);
    }
  }
  part = row_sum16_f64(part);
  if ((tid & 15) == 15) red_d[tid >> 4] = part;
  __syncthreads();  // red_d and every e in p
  // The row partials summed by each wave's lanes as a tree, and the three
  // reciprocals of the bound check (sum - slack, sum, sum + slack) on lanes
  // 0, 1, 2 at once.
  const int lane = tid & 63;
  double rs = lane < kRows ? red_d[lane] : 0.0;
  rs = row_sum16_f64(rs);
  const double sum = readlane_f64(rs, 15);
  const double slack = sum_slack(npos) * sum;
  const float mine = recip_float(lane == 0 ? sum - slack : lane == 2 ? sum + slack : sum);
  float inv = readlane_f32(mine, 1);
  if (readlane_f32(mine, 0) != readlane_f32(mine, 2)) {
    double seq = 0.0;
    for (int sp = 0; sp < npos; ++sp) seq += static_cast<double>(p[sp]);
    inv = recip_float(seq);
    __syncthreads();  // (uniform branch) p is read before it is scaled
  }
#pragma unroll
  for (int u = 0; u < kPvScores; ++u) {
    const int sp = u * kThreads + tid;
    if (sp < npos) p[sp] = sv[u] * inv;
  }
  for (int sp = npos + tid; sp < npad; sp += kThreads) p[sp] = 0.0f;
  store_v(0);
  for (int e0 = kPvBatch * kThreads; e0 < n4; e0 += kPvBatch * kThreads) {
    load_v(e0);
    store_v(e0);
  }
  __syncthreads();

  if (tid < kPvCols) {
    const float4* pr = reinterpret_cast<const float4*>(p);
    const float4* vr = reinterpret_cast<const float4*>(vt + static_cast<std::size_t>(tid) * stride);
    const int nq = npad / 4;  // a multiple of 2 * kPvChain
    // Two register sets, A and B: the reads of one round are issued before
    // the chain steps of the other, so LDS latency overlaps the chain.  The
    // reads walk two pointers with constant offsets (a clamped index would
    // put the next address in a register an outstanding read still
    // targets, and every round would wait for all reads in flight); the last
    // round's look-ahead reads the padding attn_pv_lds adds (unused).
    float4 pa[kPvChain], va[kPvChain], pb[kPvChain], vb[kPvChain];
    const auto read = [&](float4* pp, float4* vv, const float4* ps, const float4* vs) {
#pragma unroll
      for (int u = 0; u < kPvChain; ++u) {
        pp[u] = ps[u];
        vv[u] = vs[u];
      }
    };
    float acc = 0.0f;
    const auto steps = [&](const float4* pp, const float4* vv) {
#pragma unroll
      for (int u = 0; u < kPvChain; ++u) {
        acc = __builtin_fmaf(pp[u].x, vv[u].x, acc);
        acc = __builtin_fmaf(pp[u].y, vv[u].y, acc);
        acc = __builtin_fmaf(pp[u].z, vv[u].z, acc);
        acc = __builtin_fmaf(pp[u].w, vv[u].w, acc);
      }
    };
    read(pa, va, pr, vr);
    for (int q4 = 0; q4 < nq; q4 += 2 * kPvChain) {
      read(pb, vb, pr + kPvChain, vr + kPvChain);
      __builtin_amdgcn_sched_barrier(0);
      steps(pa, va);
      read(pa, va, pr + 2 * kPvChain, vr + 2 * kPvChain);
      __builtin_amdgcn_sched_barrier(0);
      steps(pb, vb);
      pr += 2 * kPvChain;
      vr += 2 * kPvChain;
    }
    out[static_cast<std::size_t>(h) * hd + i0 + tid] = acc;
  }
}

std::size_t attn_pv_lds(std::size_t npos) {
  const std::size_t npad = static_cast<std::size_t>(pv_pad(static_cast<int>(npos)));
  // + one look-ahead round of reads past the last row (4 * kPvChain floats)
  return (npad + kPvCols * (npad + 4) + 4 * kPvChain) * sizeof(float);
}

// Static LDS of attn_pv_1: the expf table and the two reduction arrays.
constexpr std::size_t kPvStaticLds = 32 * sizeof(std::uint64_t) + (kThreads / 16) * (sizeof(float) + sizeof(double));

// The two-kernel decode path applies to one token with head_dim 64 or 128,
// at most 16 query heads per KV head and p plus a V slice that fit in LDS
// beside attn_pv_1's static arrays.

bool decode_attention_fits(int nh, int nkv, int hd, std::size_t npos) {
  const int G = nh / nkv;
  return (hd == 64 || hd == 128) && G >= 1 && G <= 16 && nh % nkv == 0 &&
         npos <= static_cast<std::size_t>(kPvScores) * kThreads &&
         attn_pv_lds(npos) + kPvStaticLds <= max_lds_per_block();
}

// npos positions, the new token at npos - 1.
void launch_decode_attention(const float* q, const float* knew, const float* vnew, float* kc, float* vc,
                             const float* cos_t, const float* sin_t, float* scores, float* out, int nh, int nkv,
                             int hd, int cap, int npos, float scale, hipStream_t s) {
  const dim3 sgrid(static_cast<unsigned>((npos + kScoreTile - 1) / kScoreTile), static_cast<unsigned>(nkv));
  const dim3 pgrid(static_cast<unsigned>(nh), static_cast<unsigned>(hd / kPvCols));
  const std::size_t lds = attn_pv_lds(static_cast<std::size_t>(npos));
  if (hd == 64) {
    attn_scores_1<4><<<sgrid, kThreads, 0, s>>>(q, knew, kc, cos_t, sin_t, scores, nh, nkv, cap, npos, scale);
    attn_pv_1<4><<<pgrid, kThreads, lds, s>>>(scores, vnew, vc, out, nh, nkv, cap, npos);
  } else {
    attn_scores_1<8><<<sgrid, kThreads, 0, s>>>(q, knew, kc, cos_t, sin_t, scores, nh, nkv, cap, npos, scale);
    attn_pv_1<8><<<pgrid, kThreads, lds, s>>>(scores, vnew, vc, out, nh, nkv, cap, npos);
  }
}

// ------------------------------- tolerance-mode decode attention (T = 1)
// The one-token attention with the positions split into chunks (flash
// decoding): not the reference's summation order -- the softmax is taken
// per chunk against the chunk's own maximum and the chunks are merged by the
// consumer (the o_proj launch's kAttnCombine staging) -- so it is used only
// by the tolerance-mode decode step (llmi_hip_model_set_decode_mode).
// grid (chunks, KV heads, head groups of kAttnHeads), one wavefront per
// query head: a workgroup takes `chunk` positions of one KV head,
// kAttnSub = 64 at a time staged in LDS by all its threads (K rows padded
// by one float against bank conflicts); then each wavefront works on its own
// head without further barriers -- lane r scores position r, a wavefront
// max and sum update the head's running softmax, and lane d accumulates
// output column d (and d + 64) over the sub-block's positions.  Each thread
// loads its share of the next sub-block's K and V into registers before the
// current one is used, and the first sub-block's loads are in flight while
// q is read and rotated.  It writes o, m and l of each of its heads (the
// layout at kAttnMaxChunks, common.hpp).  q and the new k are rotated (RoPE,
// the same arithmetic as rope_and_cache); the workgroups holding position
// npos - 1 take the new k and v in place of that cache row, and the first
// head group writes them there (no workgroup reads that row).
constexpr int kAttnSub = 64;    // positions per staged sub-block = lanes of a wavefront
constexpr int kAttnHeads = 4;   // query heads (wavefronts) per workgroup

// GRAPH (a step replayed from a graph): the positions come from device
// memory (npos_dev), the chunk length is the run's (fixed when the graph
// was captured), RoPE's cos / sin row from rope_dev (the state kernels keep
// it at the step's position), and kAttnMaxChunks chunks' workgroups run,
// those past the last exiting.  Every load that starts the workgroup is
// then independent of the positions: the chunk's first K / V rows (clamped
// into the cache; rows past the last position are zeroed when staged), the
// new v, q and the cos / sin row.
template <int NCH, bool GRAPH>
// The arguments the first loads need come first (q, the cos / sin row, the
// cache, the new v, its shape, the chunk, G = query heads per KV head, the
// positions): the first 14 dwords arrive preloaded in SGPRs.
__global__ void __launch_bounds__(kAttnHeads * 64) attn_part_1(const float* __restrict__ q,
                                                               const float* __restrict__ rope_dev,
                                                               float* __restrict__ kc, float* __restrict__ vc,
                                                               const float* __restrict__ vnew, int cap, int chunk,
                                                               int G, int npos, const float* __restrict__ knew,
                                                               const int* __restrict__ npos_dev,
                                                               const float* __restrict__ cos_t,
                                                               const float* __restrict__ sin_t,
                                                               float* __restrict__ part, int nh, float scale) {
  constexpr int hd = 16 * NCH, half = hd / 2;
  constexpr int kT = kAttnHeads * 64;
  constexpr int kLd = kAttnSub * hd / 4 / kT;  // float4 of K (and of V) per thread per sub-block
  constexpr int kCols = hd / 64;               // output columns per lane
  __shared__ float qs[kAttnHeads * hd];
  __shared__ float kt[kAttnSub * (hd + 1)];
  __shared__ float vt[kAttnSub * hd];
  __shared__ __attribute__((aligned(16))) float ps[kAttnHeads * kAttnSub];
  __shared__ float kn[hd];
  if constexpr (!GRAPH) {
    if (static_cast<int>(blockIdx.x) * chunk >= npos) return;
  }
  const int c = blockIdx.x, kvh = blockIdx.y;
  const int g0 = blockIdx.z * kAttnHeads;
  const int ng = min(kAttnHeads, G - g0);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int s_begin = c * chunk;
  const float* kh = kc + static_cast<std::size_t>(kvh) * cap * hd;
  const float* vh = vc + static_cast<std::size_t>(kvh) * cap * hd;
  const float* vn = vnew + static_cast<std::size_t>(kvh) * hd;

  // Element e of a sub-block: row e / (hd / 4), columns 4 * (e % (hd / 4)) ..
  // (GRAPH: every row loaded, clamped into the cache, and the rows at or
  // past the newest position replaced when staged.)
  float4 kr[kLd], vr[kLd], vnr[kLd];
  int s_end = GRAPH ? 0 : min(npos, s_begin + chunk), pos = npos - 1;
  const auto load_sub = [&](int sb) {
#pragma unroll
    for (int u = 0; u < kLd; ++u) {
      const int e = u * kT + tid;
      const int r = e / (hd / 4), c4 = 4 * (e - r * (hd / 4));
      const int sp = sb + r;
      if constexpr (GRAPH) {
        const std::size_t row = static_cast<std::size_t>(min(sp, cap - 1)) * hd + c4;
        kr[u] = *reinterpret_cast<const float4*>(kh + row);
        vr[u] = *reinterpret_cast<const float4*>(vh + row);
      } else {
        const bool cached = sp < s_end && sp != pos;
        kr[u] = cached ? *reinterpret_cast<const float4*>(kh + static_cast<std::size_t>(sp) * hd + c4)
                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        vr[u] = cached ? *reinterpret_cast<const float4*>(vh + static_cast<std::size_t>(sp) * hd + c4)
                       : sp == pos ? *reinterpret_cast<const float4*>(vn + c4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
    }
  };
  const auto store_sub = [&](int sb) {
#pragma unroll
    for (int u = 0; u < kLd; ++u) {
      const int e = u * kT + tid;
      const int r = e / (hd / 4), c4 = 4 * (e - r * (hd / 4));
      // The newest position's k row is not used from here: its score
      // reads the rotated new k (kn) itself, so staging needs no barrier
      // after kn is written.
      float4 kv = kr[u], vv = vr[u];
      if constexpr (GRAPH) {
        const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (sb + r == pos) vv = vnr[u];
        else if (sb + r >= s_end) kv = vv = z;
      }
      float* kd = kt + r * (hd + 1) + c4;
      kd[0] = kv.x;
      kd[1] = kv.y;
      kd[2] = kv.z;
      kd[3] = kv.w;
      *reinterpret_cast<float4*>(vt + r * hd + c4) = vv;
    }
  };
  // q's pair, the new k's pair and their cos / sin first (at most one pair
  // per thread: ng * half <= kT), unconditional from clamped indices, so
  // that the rotations below wait for them only and overlap the K / V trip.
  static_assert(kAttnHeads * 64 <= kT, "one q pair per thread");
  const float* cr = GRAPH ? rope_dev : cos_t + static_cast<std::size_t>(pos) * half;
  const float* sr = GRAPH ? rope_dev + half : sin_t + static_cast<std::size_t>(pos) * half;
  const bool has_q = tid < ng * half;
  const int gq = has_q ? tid / half : 0, iq = tid % half;
  const float* qh = q + static_cast<std::size_t>(kvh * G + g0 + gq) * hd;
  const float* kq = knew + static_cast<std::size_t>(kvh) * hd;
  const float qa = qh[iq], qb = qh[iq + half], ka = kq[iq], kb = kq[iq + half], cs = cr[iq], sn = sr[iq];
  __builtin_amdgcn_sched_barrier(0);  // these loads stay in front of the sub-block's
  load_sub(s_begin);
  if constexpr (GRAPH) {
#pragma unroll
    for (int u = 0; u < kLd; ++u) {
      const int e = u * kT + tid;
      vnr[u] = *reinterpret_cast<const float4*>(vn + 4 * (e % (hd / 4)));
    }
  }
  // q rotated before the positions are read (its cos / sin row does not
  // depend on them): these LDS stores, ahead of the exit below, keep the
  // loads they use from being sunk past it.
  if (has_q) {
    qs[gq * hd + iq] = __builtin_fmaf(qa, cs, -(qb * sn));
    qs[gq * hd + iq + half] = __builtin_fmaf(qb, cs, qa * sn);
  }
  if constexpr (GRAPH) {
    npos = __builtin_amdgcn_readfirstlane(*npos_dev);
    pos = npos - 1;
    s_end = min(npos, s_begin + chunk);
    if (s_begin >= npos) return;  // a chunk past the last (after its loads were issued)
  }

  const bool has_new = pos >= s_begin && pos < s_end;
  if (has_new && tid < half) {  // iq = tid here, so cs / sn are this column's
    kn[tid] = __builtin_fmaf(ka, cs, -(kb * sn));
    kn[tid + half] = __builtin_fmaf(kb, cs, ka * sn);
  }
  // The first sub-block staged (and the next one's loads issued) before the
  // one barrier that publishes it together with qs and kn.
  store_sub(s_begin);
  if (s_begin + kAttnSub < s_end) load_sub(s_begin + kAttnSub);
  __syncthreads();  // qs, kn, the first sub-block
  if (has_new && blockIdx.z == 0 && tid < hd) {
    kc[(static_cast<std::size_t>(kvh) * cap + pos) * hd + tid] = kn[tid];
    vc[(static_cast<std::size_t>(kvh) * cap + pos) * hd + tid] = vn[tid];
  }
  const bool active = w < ng;
  const float* qg = qs + w * hd;
  float* pw = ps + w * kAttnSub;
  float mrun = -__builtin_inff(), lrun = 0.0f;
  float acc[kCols];
#pragma unroll
  for (int k = 0; k < kCols; ++k) acc[k] = 0.0f;
  for (int sb = s_begin; sb < s_end; sb += kAttnSub) {
    const int n = min(kAttnSub, s_end - sb);
    if (sb != s_begin) {
      __syncthreads();  // every wavefront is done with the previous sub-block
      store_sub(sb);
      if (sb + kAttnSub < s_end) load_sub(sb + kAttnSub);
      __syncthreads();  // the sub-block in LDS
    }
    if (active) {
      // Score of position `lane` (the newest position's from kn).
      const float* kq = sb + lane == pos ? kn : kt + lane * (hd + 1);
      float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
      for (int i = 0; i < hd; i += 4) {
        a0 = __builtin_fmaf(qg[i], kq[i], a0);
        a1 = __builtin_fmaf(qg[i + 1], kq[i + 1], a1);
        a2 = __builtin_fmaf(qg[i + 2], kq[i + 2], a2);
        a3 = __builtin_fmaf(qg[i + 3], kq[i + 3], a3);
      }
      const float sc = lane < n ? ((a0 + a1) + (a2 + a3)) * scale : -__builtin_inff();
      const float mnew = fmaxf(mrun, wave_max_dpp(sc));
      const float e = lane < n ? __expf(sc - mnew) : 0.0f;
      const float f = __expf(mrun - mnew);  // 0 on the first sub-block (mrun = -inf)
      lrun = __builtin_fmaf(lrun, f, wave_sum_dpp(e));
      mrun = mnew;
      pw[lane] = e;
      __builtin_amdgcn_wave_barrier();
      // Column lane (+ 64): the sub-block's P.V -- a whole sub-block fully
      // unrolled (four chains, p read four at a time by broadcast), so its
      // LDS reads are in flight together rather than one round trip per
      // position.
#pragma unroll
      for (int k = 0; k < kCols; ++k) {
        const int d = lane + 64 * k;
        float b0 = acc[k] * f, b1 = 0.0f, b2 = 0.0f, b3 = 0.0f;
        if (n == kAttnSub) {
#pragma unroll
          for (int r = 0; r < kAttnSub; r += 4) {
            const float4 p4 = *reinterpret_cast<const float4*>(pw + r);
            b0 = __builtin_fmaf(p4.x, vt[r * hd + d], b0);
            b1 = __builtin_fmaf(p4.y, vt[(r + 1) * hd + d], b1);
            b2 = __builtin_fmaf(p4.z, vt[(r + 2) * hd + d], b2);
            b3 = __builtin_fmaf(p4.w, vt[(r + 3) * hd + d], b3);
          }
        } else {
          int r = 0;
          for (; r + 1 < n; r += 2) {
            b0 = __builtin_fmaf(pw[r], vt[r * hd + d], b0);
            b1 = __builtin_fmaf(pw[r + 1], vt[(r + 1) * hd + d], b1);
          }
          if (r < n) b0 = __builtin_fmaf(pw[r], vt[r * hd + d], b0);
        }
        acc[k] = (b0 + b1) + (b2 + b3);
      }
    }
  }
  // Partials: o[h][c][d], m[h][c], l[h][c].
  if (active) {
    const int h = kvh * G + g0 + w;
    float* po = part + (static_cast<std::size_t>(h) * kAttnMaxChunks + c) * hd;
#pragma unroll
    for (int k = 0; k < kCols; ++k) po[lane + 64 * k] = acc[k];
    if (lane == 0) {
      float* pm = part + static_cast<std::size_t>(kAttnMaxChunks) * nh * hd;
      pm[h * kAttnMaxChunks + c] = mrun;
      pm[kAttnMaxChunks * nh + h * kAttnMaxChunks + c] = lrun;
    }
  }
}

static_assert(kAttnSub == kAttnChunkUnit, "chunks are whole sub-blocks");

// The tolerance-mode decode path applies to head_dim 64 or 128 and at most
// 16 query heads per KV head (any number of positions).
bool tol_attention_fits(int nh, int nkv, int hd) {
  const int G = nh / nkv;
  return (hd == 64 || hd == 128) && G >= 1 && G <= 16 && nh % nkv == 0;
}

// Returns the number of chunks written.  g (may be null): a step replayed
// from a graph (GraphStep: positions in device memory, the run's chunk
// length, the cos / sin row; the grid is kAttnMaxChunks chunks wide and
// the return value unused).
struct GraphStep {
  const int* npos_dev;
  const float* rope_dev;
  int chunk;
};
int launch_tol_attention(const float* q, const float* knew, const float* vnew, float* kc, float* vc,
                         const float* cos_t, const float* sin_t, float* part, int nh, int nkv, int hd, int cap,
                         int npos, float scale, hipStream_t s, const GraphStep* g = nullptr) {
  const int chunk = g != nullptr ? g->chunk : attn_chunk_len(npos);
  const int nch = (npos + chunk - 1) / chunk;
  const int G = nh / nkv;
  const dim3 grid(static_cast<unsigned>(g != nullptr ? kAttnMaxChunks : nch), static_cast<unsigned>(nkv),
                  static_cast<unsigned>((G + kAttnHeads - 1) / kAttnHeads));
  const int* nd = g != nullptr ? g->npos_dev : nullptr;
  const float* rd = g != nullptr ? g->rope_dev : nullptr;
#define LLMI_ATTN_ARGS q, rd, kc, vc, vnew, cap, chunk, G, npos, knew, nd, cos_t, sin_t, part, nh, scale
  if (g != nullptr) {
    if (hd == 64) attn_part_1<4, true><<<grid, kAttnHeads * 64, 0, s>>>(LLMI_ATTN_ARGS);
    else attn_part_1<8, true><<<grid, kAttnHeads * 64, 0, s>>>(LLMI_ATTN_ARGS);
  } else {
    if (hd == 64) attn_part_1<4, false><<<grid, kAttnHeads * 64, 0, s>>>(LLMI_ATTN_ARGS);
    else attn_part_1<8, false><<<grid, kAttnHeads * 64, 0, s>>>(LLMI_ATTN_ARGS);
  }
#undef LLMI_ATTN_ARGS
  return nch;
}

std::size_t attention_static_lds() { return kThreads * (sizeof(double) + sizeof(float)) + 16; }

// Dynamic LDS of the attention launch for npos positions.
std::size_t attention_dyn_lds(std::size_t npos, std::size_t hd) {
  return hd % 16 == 0 && hd <= 256 ? (npos + 2 * kVTile * hd) * sizeof(float) : npos * sizeof(float);
}

// Rows per workgroup of the prefill attention: 16 when the GQA group fits
// (measured faster on MI355X than 32: twice the workgroups, half the LDS),
// else 32.
int attention_rows(int nh, int nkv) { return nh / nkv <= 16 ? 16 : 32; }

// Scores LDS of attention_rows64 with `rows` rows when its longest row
// attends to npos positions (whole 64-position tiles).
std::size_t attention_rows_lds(std::size_t npos, int rows) {
  return ceil_div(npos, static_cast<std::size_t>(kAttnTile)) * kAttnTile * rows * sizeof(float);
}

bool attention_rows_fits(int nh, int nkv, int hd, std::size_t npos) {
  if (hd != 64 || nkv < 1 || nh % nkv != 0 || nh / nkv > 32) return false;
  const int rows = attention_rows(nh, nkv);
  const std::size_t stat = rows == 16 ? attn_static_lds<16>() : attn_static_lds<32>();
  return attention_rows_lds(npos, rows) + stat <= max_lds_per_block();
}

void launch_attention(const float* q, const float* kc, const float* vc, float* out, int nh, int nkv, int hd, int cap,
                      int base, int T, float scale, hipStream_t s) {
  const std::size_t npos = static_cast<std::size_t>(base) + T;
  if (attention_rows_fits(nh, nkv, hd, npos)) {
    const int rows = attention_rows(nh, nkv);
    // Tokens per workgroup: the tile's full G x tq rows, fewer when that
    // would leave fewer than ~256 workgroups (short prompts, few KV heads).
    const int tq = std::clamp(static_cast<int>(ceil_div(static_cast<std::size_t>(T) * nkv, 256)), 1, rows / (nh / nkv));
    const dim3 grid(static_cast<unsigned>(ceil_div(T, tq)), static_cast<unsigned>(nkv));
    const std::size_t lds = attention_rows_lds(npos, rows);
    if (rows == 16) {
      attention_rows64<16><<<grid, kThreads, lds, s>>>(q, kc, vc, out, nh, nkv, cap, base, T, tq, scale);
    } else {
      attention_rows64<32><<<grid, kThreads, lds, s>>>(q, kc, vc, out, nh, nkv, cap, base, T, tq, scale);
    }
    return;
  }
  const dim3 grid(static_cast<unsigned>(nh), static_cast<unsigned>(T));
  if (hd % 16 == 0 && hd <= 256) {
    attention_hd16<<<grid, kThreads, attention_dyn_lds(npos, hd), s>>>(q, kc, vc, out, nh, nkv, hd, cap, base, scale,
                                                                       static_cast<int>(npos));
  } else {
    attention_generic<<<grid, kThreads, attention_dyn_lds(npos, hd), s>>>(q, kc, vc, out, nh, nkv, hd, cap, base,
                                                                          scale);
  }
}

// ------------------------------------------------------------- silu * up
__global__ void __launch_bounds__(kThreads) silu_mul(float* __restrict__ g, const float* __restrict__ u,
                                                     std::size_t n) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= n) return;
  const float v = g[i];
  const float silu = v / (1.0f + exact::expf(-v));
  g[i] = silu * u[i];
}

// --------------------------------------------------------------- argmax
// First maximum (lowest index on ties), transformer.cpp:22-24.
struct Best {
  float v;
  int i;  // -1: empty
};

__device__ __forceinline__ Best better(Best a, Best b) {
  if (b.i < 0) return a;
  if (a.i < 0) return b;
  if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
  return a;
}

// The workgroup's best, returned to every thread: within each wavefront by
// lane exchanges (no barrier), then over the NT / 64 wavefronts' bests in LDS
// (one barrier).  With finite values the result -- the maximum, and the
// lowest index among its ties -- does not depend on the order of the pairings.
template <int NT>
__device__ __forceinline__ Best block_best(Best b, float* bv, int* bi) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) b = better(b, Best{__shfl_xor(b.v, off, 64), __shfl_xor(b.i, off, 64)});
  const int tid = threadIdx.x;
  if ((tid & 63) == 0) {
    bv[tid >> 6] = b.v;
    bi[tid >> 6] = b.i;
  }
  __syncthreads();
  Best r{bv[0], bi[0]};
#pragma unroll
  for (int w = 1; w < NT / 64; ++w) r = better(r, Best{bv[w], bi[w]});
  return r;
}

// One block over all of x (small n, and the standalone entry point).
__global__ void __launch_bounds__(1024) argmax_first(const float* __restrict__ x, int n, std::int32_t* __restrict__ out,
                                                     std::int32_t* __restrict__ also) {
  __shared__ float bv[1024];
  __shared__ int bi[1024];
  Best b{-__builtin_inff(), -1};
  for (int i = threadIdx.x; i < n; i += 1024) b = better(b, Best{x[i], i});
  b = block_best<1024>(b, bv, bi);
  if (threadIdx.x == 0) {
    const int r = b.i < 0 ? 0 : b.i;
    *out = r;
    if (also != nullptr) *also = r;
  }
}

// Many blocks, each over a contiguous slice; each block publishes its best
// and the last block to finish (counted with a device-scope atomic) combines
// them and resets the counter for the next launch.  No block waits.
// adv (may be null; a step replayed from a graph): the state of the step
// about to run, moved on by the last block once the id is recorded -- st[0]
// (the positions) and st[1] (the output slot, also_idx) each up by one, and
// rope set to the cos / sin row of the new step's newest position -- so no
// launch of its own does it (the layout at step_state_set).
constexpr int kArgmaxBlocks = 128;

__global__ void __launch_bounds__(kThreads) argmax_many(const float* __restrict__ x, int n, float* __restrict__ part_v,
                                                        int* __restrict__ part_i, unsigned* __restrict__ counter,
                                                        std::int32_t* __restrict__ out,
                                                        std::int32_t* __restrict__ also,
                                                        const int* __restrict__ also_idx, int* __restrict__ adv,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t, float* __restrict__ rope,
                                                        int half) {
  __shared__ float bv[kThreads];
  __shared__ int bi[kThreads];
  __shared__ bool last;
  const int per = (n + gridDim.x - 1) / gridDim.x;
  const int lo = blockIdx.x * per;
  const int hi = min(n, lo + per);
  // Each thread's elements in increasing order, kBatch loads issued before
  // the first comparison (one memory round trip per batch).
  constexpr int kBatch = 8;
  Best b{-__builtin_inff(), -1};
  for (int i0 = lo + threadIdx.x; i0 < hi; i0 += kBatch * kThreads) {
    float v[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int i = i0 + u * kThreads;
      v[u] = i < hi ? x[i] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
      if (i0 + u * kThreads < hi) b = better(b, Best{v[u], i0 + u * kThreads});
  }
  b = block_best<kThreads>(b, bv, bi);
  if (threadIdx.x == 0) {
    part_v[blockIdx.x] = b.v;
    part_i[blockIdx.x] = b.i;
    // The release half of the update publishes this block's partials; the
    // last block reads them with agent-scope atomic loads after its barrier.
    // (An extra agent-scope fence would write back or invalidate the XCD's
    // whole L2 per wavefront.)
    const unsigned done = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    last = done == gridDim.x - 1;
  }
  __syncthreads();
  if (!last) return;
  Best r{-__builtin_inff(), -1};
  for (int k = threadIdx.x; k < static_cast<int>(gridDim.x); k += kThreads) {
    const float v = __hip_atomic_load(part_v + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int i = __hip_atomic_load(part_i + k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    r = better(r, Best{v, i});
  }
  r = block_best<kThreads>(r, bv, bi);
  if (threadIdx.x == 0) {
    const int idx = r.i < 0 ? 0 : r.i;
    *out = idx;
    // also_idx (may be null): the slot of `also` in device memory (a step
    // replayed from a graph).
    if (also != nullptr) also[also_idx != nullptr ? *also_idx : 0] = idx;
    __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (adv != nullptr) {
    const int np = adv[0];  // the step before; the next one's newest position is np
    __syncthreads();        // every thread has read st[0], thread 0 the slot, before they move
    const int t = threadIdx.x;
    if (t < 2) adv[t] += 1;
    if (t < half) {
      rope[t] = cos_t[static_cast<std::size_t>(np) * half + t];
      rope[half + t] = sin_t[static_cast<std::size_t>(np) * half + t];
    }
  }
}

// The state of a graph-replayed tolerance step: st[0] = the step's positions
// (the cache length after it), st[1] = the generated token's slot.  Set
// before the first replay to the step before the first (its argmax moves it
// on); advanced by the argmax that starts each replayed step (argmax_many's
// adv).  rope[0, half) / rope[half, hd): the cos / sin row of the step's
// newest position (npos - 1), which the replayed attention reads.  One
// workgroup of at least max(2, half) threads.
__global__ void step_state_set(int* st, int npos, int slot, const float* __restrict__ cos_t,
                               const float* __restrict__ sin_t, float* __restrict__ rope, int half) {
  const int t = threadIdx.x;
  if (t < 2) st[t] = t == 0 ? npos : slot;
  if (t < half) {
    rope[t] = cos_t[static_cast<std::size_t>(npos - 1) * half + t];
    rope[half + t] = sin_t[static_cast<std::size_t>(npos - 1) * half + t];
  }
}

// Standalone glue kernels (the device counterparts of kernels.hpp:13-32).
// The scoring of llmi-perplexity (apps/llmi-perplexity/main.cpp:158-166) on
// one logits row per workgroup: mx = the float maximum; sum_exp = sum over v
// of exp(double(row[v] - mx)) (the float difference, widened); lse =
// log(sum_exp) + mx; nll = -(double(row[next]) - lse).  The reference sums
// sequentially; here the double sum is a fixed tree, so nll can differ from
// the reference's in the last bits.
__global__ void __launch_bounds__(kThreads) row_nll(const float* __restrict__ logits, int V,
                                                    const std::int32_t* __restrict__ next,
                                                    double* __restrict__ nll) {
  __shared__ double red_d[kThreads];
  __shared__ float red_f[kThreads];
  const float* row = logits + static_cast<std::size_t>(blockIdx.x) * V;
  float mx = -__builtin_inff();
  for (int v = threadIdx.x; v < V; v += kThreads) mx = fmaxf(mx, row[v]);
  mx = block_max_float(mx, red_f);
  double part = 0.0;
  for (int v = threadIdx.x; v < V; v += kThreads) part += exp(static_cast<double>(row[v] - mx));
  const double sum = block_sum_double(part, red_d);
  if (threadIdx.x == 0) {
    const double lse = log(sum) + static_cast<double>(mx);
    nll[blockIdx.x] = -(static_cast<double>(row[next[blockIdx.x]]) - lse);
  }
}

__global__ void __launch_bounds__(kThreads) dot_many(const float* __restrict__ a, const float* __restrict__ b,
                                                     const int* __restrict__ lens, int count, float* __restrict__ out) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i < count) out[i] = ref_dot(a, b, lens[i]);
}

// kernels.cpp:136-146 on each row of x (rows x n), in place; n <= LDS.
__global__ void __launch_bounds__(kThreads) softmax_rows(float* __restrict__ x, int n) {
  extern __shared__ float sc[];
  __shared__ double red_d[kThreads];
  __shared__ float red_f[kThreads];
  __shared__ float inv_s;
  float* row = x + static_cast<std::size_t>(blockIdx.x) * n;
  float mx_local = -__builtin_inff();
  for (int s = threadIdx.x; s < n; s += kThreads) {
    sc[s] = row[s];
    mx_local = fmaxf(mx_local, sc[s]);
  }
  softmax_lds(sc, n, mx_local, red_d, red_f, &inv_s);
  for (int s = threadIdx.x; s < n; s += kThreads) row[s] = sc[s];
}

__global__ void __launch_bounds__(kThreads) zero_floats(float* __restrict__ x, int n) {
  const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  if (i < n) x[i] = 0.0f;
}

__global__ void __launch_bounds__(kThreads) silu_inplace(float* __restrict__ x, std::size_t n) {
  const std::size_t i = static_cast<std::size_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n) x[i] = x[i] / (1.0f + exact::expf(-x[i]));
}

unsigned blocks_for(std::size_t n) { return static_cast<unsigned>(ceil_div(n, kThreads)); }

}  // namespace

// ---------------------------------------------------------------- model
struct DeviceLayer {
  float *attn_norm = nullptr, *mlp_norm = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr;
  DeviceMatrix wq, wk, wv, wo, gate, up, down;
  // q|k|v and gate|up as one matrix each (consecutive tiles of one
  // allocation that wq, wk, wv / gate, up view), when every part has a
  // multiple of 64 rows; out == 0 otherwise.  bqkv: the biases likewise.
  DeviceMatrix wqkv, gate_up_w;
  float* bqkv = nullptr;
  // The fused one-token step's launches (see decode_step).
  DeviceGroup qkv, gate_up, down_silu;
  // The tolerance-mode step's products split over K (with fused q|k|v and
  // gate|up weights): q|k|v (clearing g|u), o_proj (clearing q|k|v for the
  // next layer), gate|up, down_proj.
  SplitProduct s_qkv, s_o, s_gu, s_dn;
};

// Fixed one-token buffers of the fused decode step.
struct DecodeBuffers {
  float *x = nullptr, *h = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *g = nullptr,
        *u = nullptr;
  float* part = nullptr;  // the tolerance-mode attention's chunk partials
};

// Sampled steps queued per host read-back in generate_sampled.
constexpr std::size_t kSampleWindow = 32;

struct Workspace {
  std::size_t tokens = 0;  // capacity in tokens
  float *x = nullptr, *h = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr, *g = nullptr,
        *u = nullptr, *logits = nullptr;
  std::int32_t* ids = nullptr;
  std::int32_t* next = nullptr;  // argmax result
  std::int32_t* gen = nullptr;   // generated ids of the current greedy run
  std::size_t gen_cap = 0;
  SampleLog* slog = nullptr;     // the sampled loop's per-step draws (kSampleWindow)
  double* nll = nullptr;         // per-position NLL of chunk_nll
  std::size_t nll_cap = 0;
  float* am_v = nullptr;         // argmax partials and completion counter
  int* am_i = nullptr;
  unsigned* am_count = nullptr;
  int* step_state = nullptr;     // a graph-replayed step's positions and output slot (step_state_*)
  float* step_rope = nullptr;    // and its newest position's cos / sin row
};

}  // namespace llmi_hip

struct llmi_hip_model {
  llmi_model_config c{};
  int type = 0;
  std::size_t H = 0, hd = 0, Q = 0, KV = 0, F = 0, V = 0;
  llmi_hip::DeviceMatrix embed, lm_head;
  bool tied = true;
  float* final_norm = nullptr;
  std::vector<llmi_hip::DeviceLayer> layers;
  std::vector<float> inv_freq;
  float* cos_t = nullptr;
  float* sin_t = nullptr;
  std::size_t table_len = 0;
  llmi_hip::Workspace ws;
  llmi_hip::DecodeBuffers dec;
  // The cache of the calls that need one only for their own duration
  // (forward without a cache, generate_*, chunk_nll): kept and reused while
  // its allocation is large enough, reset on every use.
  llmi_hip_cache* scratch = nullptr;
  std::vector<void*> allocations;
  double last_prefill_ms = 0.0, last_decode_ms = 0.0;  // of the last greedy run
  int decode_mode = LLMI_DECODE_EXACT;  // llmi_hip_model_set_decode_mode
  bool tol_ready = false;               // build_decode made the tolerance-mode step
  bool qkv_clear = false;               // the last queued step left dec.q|k|v at zero (split step)
  bool decode_graph = true;             // llmi_hip_model_set_decode_graph
  std::size_t last_redraws = 0;  // generate_sampled: queued draws redrawn step by step
};

struct llmi_hip_cache {
  const llmi_hip_model* model = nullptr;
  std::size_t cap = 0, len = 0;
  float* k = nullptr;  // [layer][kv_head][cap][hd]
  float* v = nullptr;
  float* scores = nullptr;  // [head][cap], decode attention scratch
  std::size_t kv_elems = 0, score_elems = 0;  // allocated floats of k (= v) and scores
};

namespace llmi_hip {
namespace {

int dev_alloc(llmi_hip_model* m, void** p, std::size_t bytes) {
  *p = nullptr;
  if (bytes == 0) return LLMI_OK;
  LLMI_TRY_HIP(hipMalloc(p, bytes));
  m->allocations.push_back(*p);
  return LLMI_OK;
}

// Copies n floats from host or device memory into a new device array.
int dev_vector(llmi_hip_model* m, const float* src, std::size_t n, bool src_on_device, float** dst) {
  if (int rc = dev_alloc(m, reinterpret_cast<void**>(dst), n * sizeof(float))) return rc;
  if (n > 0)
    LLMI_TRY_HIP(hipMemcpyAsync(*dst, src, n * sizeof(float), src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                                library_stream()));
  return LLMI_OK;
}

// Quantizes an out x in fp32 matrix (host or device) into the tiled layout.
int dev_matrix(llmi_hip_model* m, const float* src, std::size_t out, std::size_t in, bool src_on_device,
               float* staging, DeviceMatrix* dm) {
  dm->type = m->type;
  dm->out = out;
  dm->in = in;
  dm->nblk = ceil_div(in, kBlock);
  dm->ntiles = ceil_div(out, kTileRows);
  if (m->type == LLMI_TYPE_F32) {  // row-major floats (weight.cpp:17: kept as they are)
    dm->code_bytes = out * in * sizeof(float);
    dm->scale_bytes = 0;
    if (int rc = dev_alloc(m, reinterpret_cast<void**>(&dm->codes), dm->code_bytes)) return rc;
    LLMI_TRY_HIP(hipMemcpyAsync(dm->codes, src, dm->code_bytes,
                                src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, library_stream()));
    LLMI_TRY_HIP(hipStreamSynchronize(library_stream()));
    return LLMI_OK;
  }
  dm->code_bytes = dm->ntiles * dm->nblk * kTileRows * block_code_bytes(m->type);
  dm->scale_bytes = dm->ntiles * dm->nblk * kTileRows * sizeof(float);
  if (int rc = dev_alloc(m, reinterpret_cast<void**>(&dm->codes), dm->code_bytes)) return rc;
  if (int rc = dev_alloc(m, reinterpret_cast<void**>(&dm->scales), dm->scale_bytes)) return rc;
  LLMI_TRY_HIP(hipMemsetAsync(dm->codes, 0, dm->code_bytes, library_stream()));
  LLMI_TRY_HIP(hipMemsetAsync(dm->scales, 0, dm->scale_bytes, library_stream()));
  const float* w = src;
  if (!src_on_device) {
    LLMI_TRY_HIP(hipMemcpyAsync(staging, src, out * in * sizeof(float), hipMemcpyHostToDevice, library_stream()));
    w = staging;
  }
  if (int rc = launch_quantize(w, out, in, m->type, nullptr, nullptr, dm, library_stream())) return rc;
  // The staging buffer is reused by the next matrix: finish this one first.
  LLMI_TRY_HIP(hipStreamSynchronize(library_stream()));
  return LLMI_OK;
}

// Quantizes n fp32 matrices of the same `in` (host or device) into
// consecutive tiles of one allocation when every one has a multiple of 64
// rows -- each *dms[i] views its tiles and *fused views them all as one
// matrix of sum(outs) rows -- else one by one (fused->out = 0).
int dev_matrices(llmi_hip_model* m, const float* const* src, const std::size_t* outs, int n, std::size_t in,
                 bool src_on_device, float* staging, DeviceMatrix* const* dms, DeviceMatrix* fused) {
  *fused = DeviceMatrix{};
  bool whole = m->type != LLMI_TYPE_F32;
  std::size_t total = 0;
  for (int i = 0; i < n; ++i) {
    whole = whole && outs[i] % kTileRows == 0;
    total += outs[i];
  }
  if (!whole) {
    for (int i = 0; i < n; ++i)
      if (int rc = dev_matrix(m, src[i], outs[i], in, src_on_device, staging, dms[i])) return rc;
    return LLMI_OK;
  }
  fused->type = m->type;
  fused->out = total;
  fused->in = in;
  fused->nblk = ceil_div(in, kBlock);
  fused->ntiles = total / kTileRows;
  fused->code_bytes = fused->ntiles * fused->nblk * kTileRows * block_code_bytes(m->type);
  fused->scale_bytes = fused->ntiles * fused->nblk * kTileRows * sizeof(float);
  if (int rc = dev_alloc(m, reinterpret_cast<void**>(&fused->codes), fused->code_bytes)) return rc;
  if (int rc = dev_alloc(m, reinterpret_cast<void**>(&fused->scales), fused->scale_bytes)) return rc;
  LLMI_TRY_HIP(hipMemsetAsync(fused->codes, 0, fused->code_bytes, library_stream()));
  LLMI_TRY_HIP(hipMemsetAsync(fused->scales, 0, fused->scale_bytes, library_stream()));
  std::size_t tile0 = 0;
  for (int i = 0; i < n; ++i) {
    DeviceMatrix* dm = dms[i];
    dm->type = m->type;
    dm->out = outs[i];
    dm->in = in;
    dm->nblk = fused->nblk;
    dm->ntiles = outs[i] / kTileRows;
    dm->code_bytes = dm->ntiles * dm->nblk * kTileRows * block_code_bytes(m->type);
    dm->scale_bytes = dm->ntiles * dm->nblk * kTileRows * sizeof(float);
    dm->codes = fused->codes + tile0 * fused->nblk * kTileRows * block_code_bytes(m->type);
    dm->scales = fused->scales + tile0 * fused->nblk * kTileRows;
    tile0 += dm->ntiles;
    const float* w = src[i];
    if (!src_on_device) {
      LLMI_TRY_HIP(hipMemcpyAsync(staging, src[i], outs[i] * in * sizeof(float), hipMemcpyHostToDevice,
                                  library_stream()));
      w = staging;
    }
    if (int rc = launch_quantize(w, outs[i], in, m->type, nullptr, nullptr, dm, library_stream())) return rc;
    LLMI_TRY_HIP(hipStreamSynchronize(library_stream()));
  }
  return LLMI_OK;
}

int check_config(const llmi_model_config& c) {
  LLMI_REQUIRE(c.arch == 0 || c.arch == 1, "model: arch must be 0 (Llama) or 1 (Qwen2)");
  LLMI_REQUIRE(c.vocab_size > 0 && c.hidden_size > 0 && c.intermediate_size > 0 && c.num_layers > 0,
               "model: sizes must be positive");
  LLMI_REQUIRE(c.num_heads > 0 && c.num_kv_heads > 0, "model: head counts must be positive");
  LLMI_REQUIRE(c.hidden_size % c.num_heads == 0, "model: hidden_size is not a multiple of num_attention_heads");
  LLMI_REQUIRE((c.hidden_size / c.num_heads) % 2 == 0, "model: head_dim must be even for rotary embeddings");
  LLMI_REQUIRE(c.num_heads % c.num_kv_heads == 0, "model: num_attention_heads is not a multiple of num_key_value_heads");
  LLMI_REQUIRE(c.max_position_embeddings > 0, "model: max_position_embeddings must be positive");
  return LLMI_OK;
}

// The fused one-token step (decode_step): per layer
//   qkv:       RMSNorm(x) staged in each workgroup, then q, k, v (+ biases)
//   attention: attn_scores_1 (RoPE of q and of the new k fused, the k written
//              to the cache) and attn_pv_1 (the new v written to the cache)
//   o_proj:    x += W_o att
//   gate_up:   RMSNorm(x) staged again, then gate and up
//   down_silu: SiLU(gate) * up staged, then x += W_down (...)
// -- 6 launches instead of 13, with the same arithmetic.
int build_decode(llmi_hip_model* m) {
  DecodeBuffers& d = m->dec;
  const auto get = [&](float** p, std::size_t n) { return dev_alloc(m, reinterpret_cast<void**>(p), n * sizeof(float)); };
  if (int rc = get(&d.x, m->H)) return rc;
  if (int rc = get(&d.h, m->H)) return rc;
  // q|k|v and g|u contiguous: the fused products write them in one go.
  if (int rc = get(&d.q, m->Q + 2 * m->KV)) return rc;
  d.k = d.q + m->Q;
  d.v = d.k + m->KV;
  if (int rc = get(&d.att, m->Q)) return rc;
  if (int rc = get(&d.g, 2 * m->F)) return rc;
  d.u = d.g + m->F;
  if (int rc = get(&d.part, static_cast<std::size_t>(kAttnMaxChunks) * m->c.num_heads * (m->hd + 2))) return rc;
  // The o_proj combine reads every chunk slot (unused ones with weight 0):
  // they start as zeros, never as uninitialised bits.
  LLMI_TRY_HIP(hipMemsetAsync(d.part, 0, static_cast<std::size_t>(kAttnMaxChunks) * m->c.num_heads * (m->hd + 2) *
                                             sizeof(float), library_stream()));
  const float eps = static_cast<float>(m->c.rms_norm_eps);
  for (DeviceLayer& l : m->layers) {
    const GroupEntry qkv[3] = {{&l.wq, d.x, l.bq, d.q, 1, false, kRmsNorm, l.attn_norm, eps},
                               {&l.wk, d.x, l.bk, d.k, 1, false, kRmsNorm, l.attn_norm, eps},
                               {&l.wv, d.x, l.bv, d.v, 1, false, kRmsNorm, l.attn_norm, eps}};
    const GroupEntry gu[2] = {{&l.gate, d.x, nullptr, d.g, 1, false, kRmsNorm, l.mlp_norm, eps},
                              {&l.up, d.x, nullptr, d.u, 1, false, kRmsNorm, l.mlp_norm, eps}};
    const GroupEntry dn[1] = {{&l.down, d.g, nullptr, d.x, 1, true, kSiluUp, d.u, 0.0f}};
    // One fused product each where the weights are fused (its rows are
    // q|k|v and gate|up, its output the contiguous buffers).
    const GroupEntry qkv1[1] = {{&l.wqkv, d.x, l.bqkv, d.q, 1, false, kRmsNorm, l.attn_norm, eps}};
    const GroupEntry gu1[1] = {{&l.gate_up_w, d.x, nullptr, d.g, 1, false, kRmsNorm, l.mlp_norm, eps}};
    if (int rc = l.wqkv.out != 0 ? l.qkv.build(qkv1, 1) : l.qkv.build(qkv, 3)) return rc;
    if (int rc = l.gate_up_w.out != 0 ? l.gate_up.build(gu1, 1) : l.gate_up.build(gu, 2)) return rc;
    if (int rc = l.down_silu.build(dn, 1)) return rc;
  }
  // The tolerance-mode step: head sizes attn_part_1 takes, whole blocks per
  // head (the o_proj splits take whole heads), and the fused q|k|v and
  // gate|up weights its split products run on.
  bool tol = tol_attention_fits(static_cast<int>(m->c.num_heads), static_cast<int>(m->c.num_kv_heads),
                                static_cast<int>(m->hd)) &&
             m->hd % kBlock == 0;
  for (const DeviceLayer& l : m->layers) tol = tol && l.wqkv.out != 0 && l.gate_up_w.out != 0;
  for (DeviceLayer& l : m->layers) {
    if (!tol) break;
    l.s_qkv = SplitProduct{&l.wqkv, d.x, l.attn_norm, l.bqkv, d.q, kRmsNorm, eps};
    l.s_qkv.zero = d.g;
    l.s_qkv.nzero = static_cast<int>(2 * m->F);
    l.s_o = SplitProduct{&l.wo, d.part, d.part, nullptr, d.x, kAttnCombine};
    l.s_o.comb_hd = static_cast<int>(m->hd);
    l.s_o.zero = d.q;
    l.s_o.nzero = static_cast<int>(m->Q + 2 * m->KV);
    l.s_gu = SplitProduct{&l.gate_up_w, d.x, l.mlp_norm, nullptr, d.g, kRmsNorm, eps};
    l.s_dn = SplitProduct{&l.down, d.g, d.u, nullptr, d.x, kSiluUp};
    for (SplitProduct* sp : {&l.s_qkv, &l.s_o, &l.s_gu, &l.s_dn})
      if (int rc = plan_split(sp)) return rc;
  }
  m->tol_ready = tol;
  return LLMI_OK;
}

void release_decode(llmi_hip_model* m) {
  for (DeviceLayer& l : m->layers) {
    l.qkv.release();
    l.gate_up.release();
    l.down_silu.release();
  }
}

int create_model(const llmi_model_config* cfg, const float* const* t, int type, bool on_device,
                 llmi_hip_model** out) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(cfg != nullptr && t != nullptr && out != nullptr, "model_create: null pointer");
  LLMI_REQUIRE(type == LLMI_TYPE_Q8_0 || type == LLMI_TYPE_Q4_0 || type == LLMI_TYPE_F32,
               "model_create: type must be Q8_0, Q4_0 or F32");
  if (int rc = check_config(*cfg)) return rc;
  *out = nullptr;
  auto m = std::make_unique<llmi_hip_model>();
  m->c = *cfg;
  m->type = type;
  const auto& c = m->c;
  m->H = c.hidden_size;
  m->hd = c.hidden_size / c.num_heads;
  m->Q = static_cast<std::size_t>(c.num_heads) * m->hd;
  m->KV = static_cast<std::size_t>(c.num_kv_heads) * m->hd;
  m->F = c.intermediate_size;
  m->V = c.vocab_size;
  m->tied = c.tie_word_embeddings != 0;
  auto cleanup = [&](int rc) {
    release_decode(m.get());
    for (void* p : m->allocations) (void)hipFree(p);
    m->allocations.clear();
    return rc;
  };
  const std::size_t biggest = std::max({m->V * m->H, m->F * m->H, m->Q * m->H});
  float* staging = nullptr;
  if (!on_device) {
    if (int rc = dev_alloc(m.get(), reinterpret_cast<void**>(&staging), biggest * sizeof(float))) return cleanup(rc);
  }
  std::size_t k = 0;
  int rc = dev_matrix(m.get(), t[k++], m->V, m->H, on_device, staging, &m->embed);
  m->layers.resize(c.num_layers);
  for (auto& l : m->layers) {
    if (rc == LLMI_OK) rc = dev_vector(m.get(), t[k++], m->H, on_device, &l.attn_norm);
    {
      const float* src[3] = {t[k], t[k + 1], t[k + 2]};
      const std::size_t outs[3] = {m->Q, m->KV, m->KV};
      DeviceMatrix* const dms[3] = {&l.wq, &l.wk, &l.wv};
      if (rc == LLMI_OK) rc = dev_matrices(m.get(), src, outs, 3, m->H, on_device, staging, dms, &l.wqkv);
      k += 3;
    }
    if (c.qkv_bias) {
      if (rc == LLMI_OK && l.wqkv.out != 0) {
        // One bias vector for the fused q|k|v product; bq, bk, bv view it.
        rc = dev_alloc(m.get(), reinterpret_cast<void**>(&l.bqkv), (m->Q + 2 * m->KV) * sizeof(float));
        if (rc == LLMI_OK) {
          l.bq = l.bqkv;
          l.bk = l.bqkv + m->Q;
          l.bv = l.bk + m->KV;
          const auto kind = on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
          if (hipMemcpyAsync(l.bq, t[k], m->Q * sizeof(float), kind, library_stream()) != hipSuccess ||
              hipMemcpyAsync(l.bk, t[k + 1], m->KV * sizeof(float), kind, library_stream()) != hipSuccess ||
              hipMemcpyAsync(l.bv, t[k + 2], m->KV * sizeof(float), kind, library_stream()) != hipSuccess)
            rc = fail(LLMI_ERR_HIP, "model_create: bias copy");
        }
        k += 3;
      } else {
        if (rc == LLMI_OK) rc = dev_vector(m.get(), t[k++], m->Q, on_device, &l.bq);
        if (rc == LLMI_OK) rc = dev_vector(m.get(), t[k++], m->KV, on_device, &l.bk);
        if (rc == LLMI_OK) rc = dev_vector(m.get(), t[k++], m->KV, on_device, &l.bv);
      }
    }
    if (rc == LLMI_OK) rc = dev_matrix(m.get(), t[k++], m->H, m->Q, on_device, staging, &l.wo);
    if (rc == LLMI_OK) rc = dev_vector(m.get(), t[k++], m->H, on_device, &l.mlp_norm);
    {
      const float* src[2] = {t[k], t[k + 1]};
      const std::size_t outs[2] = {m->F, m->F};
      DeviceMatrix* const dms[2] = {&l.gate, &l.up};
      if (rc == LLMI_OK) rc = dev_matrices(m.get(), src, outs, 2, m->H, on_device, staging, dms, &l.gate_up_w);
      k += 2;
    }
    if (rc == LLMI_OK) rc = dev_matrix(m.get(), t[k++], m->H, m->F, on_device, staging, &l.down);
  }
  if (rc == LLMI_OK) rc = dev_vector(m.get(), t[k++], m->H, on_device, &m->final_norm);
  if (rc == LLMI_OK && !m->tied) rc = dev_matrix(m.get(), t[k++], m->V, m->H, on_device, staging, &m->lm_head);
  if (rc == LLMI_OK && hipStreamSynchronize(library_stream()) != hipSuccess) rc = fail(LLMI_ERR_HIP, "model_create: sync");
  if (rc != LLMI_OK) return cleanup(rc);
  if (staging != nullptr) {
    (void)hipFree(staging);
    m->allocations.erase(std::find(m->allocations.begin(), m->allocations.end(), static_cast<void*>(staging)));
  }
  // The fused one-token step (grouped quantized GEMVs) exists for Q8_0 / Q4_0;
  // an fp32 model decodes through the per-operation path.
  if (m->type != LLMI_TYPE_F32)
    if (int rc2 = build_decode(m.get())) return cleanup(rc2);
  // inv_freq[i] = 1 / theta^(2i/d) in float, as transformer.cpp:59-66.
  m->inv_freq.resize(m->hd / 2);
  for (std::size_t i = 0; i < m->hd / 2; ++i) {
    const float e = static_cast<float>(2 * i) / static_cast<float>(m->hd);
    m->inv_freq[i] = 1.0F / std::pow(static_cast<float>(c.rope_theta), e);
  }
  *out = m.release();
  return LLMI_OK;
}

// cos/sin of the float angle pos*inv_freq[i] for pos < n, computed on the
// host with the same libm call the reference makes (kernels.cpp:126-128).
int ensure_tables(llmi_hip_model* m, std::size_t n) {
  if (m->table_len >= n) return LLMI_OK;
  const std::size_t half = m->hd / 2;
  std::vector<float> c(n * half), s(n * half);
  for (std::size_t pos = 0; pos < n; ++pos)
    for (std::size_t i = 0; i < half; ++i) {
      const float angle = static_cast<float>(pos) * m->inv_freq[i];
      sincosf(angle, &s[pos * half + i], &c[pos * half + i]);
    }
  float *dc = nullptr, *dsn = nullptr;
  LLMI_TRY_HIP(hipMalloc(&dc, c.size() * sizeof(float)));
  const hipError_t e = hipMalloc(&dsn, s.size() * sizeof(float));
  if (e != hipSuccess) {
    (void)hipFree(dc);
    return fail(LLMI_ERR_HIP, "rope tables: hipMalloc");
  }
  LLMI_TRY_HIP(hipMemcpy(dc, c.data(), c.size() * sizeof(float), hipMemcpyHostToDevice));
  LLMI_TRY_HIP(hipMemcpy(dsn, s.data(), s.size() * sizeof(float), hipMemcpyHostToDevice));
  LLMI_TRY_HIP(hipStreamSynchronize(library_stream()));
  if (m->cos_t != nullptr) (void)hipFree(m->cos_t);
  if (m->sin_t != nullptr) (void)hipFree(m->sin_t);
  m->cos_t = dc;
  m->sin_t = dsn;
  m->table_len = n;
  return LLMI_OK;
}

void free_workspace(Workspace& w) {
  for (void* p : {static_cast<void*>(w.x), static_cast<void*>(w.h), static_cast<void*>(w.q), static_cast<void*>(w.k),
                  static_cast<void*>(w.v), static_cast<void*>(w.att), static_cast<void*>(w.g), static_cast<void*>(w.u),
                  static_cast<void*>(w.logits), static_cast<void*>(w.ids), static_cast<void*>(w.next),
                  static_cast<void*>(w.gen), static_cast<void*>(w.slog), static_cast<void*>(w.nll),
                  static_cast<void*>(w.am_v),
                  static_cast<void*>(w.am_i),
                  static_cast<void*>(w.am_count), static_cast<void*>(w.step_state),
                  static_cast<void*>(w.step_rope)})
    if (p != nullptr) (void)hipFree(p);
  w = Workspace{};
}

int ensure_workspace(llmi_hip_model* m, std::size_t T) {
  Workspace& w = m->ws;
  if (w.tokens >= T) return LLMI_OK;
  LLMI_TRY_HIP(hipStreamSynchronize(library_stream()));
  free_workspace(w);
  const std::size_t n = std::max<std::size_t>(T, 1);
  auto get = [&](auto** p, std::size_t elems, std::size_t size) -> int {
    LLMI_TRY_HIP(hipMalloc(reinterpret_cast<void**>(p), std::max<std::size_t>(elems, 1) * size));
    return LLMI_OK;
  };
  int rc = get(&w.x, n * m->H, 4);
  if (rc == LLMI_OK) rc = get(&w.h, n * m->H, 4);
  if (rc == LLMI_OK) rc = get(&w.q, n * m->Q, 4);
  if (rc == LLMI_OK) rc = get(&w.k, n * m->KV, 4);
  if (rc == LLMI_OK) rc = get(&w.v, n * m->KV, 4);
  if (rc == LLMI_OK) rc = get(&w.att, n * m->Q, 4);
  if (rc == LLMI_OK) rc = get(&w.g, n * m->F, 4);
  if (rc == LLMI_OK) rc = get(&w.u, n * m->F, 4);
  if (rc == LLMI_OK) rc = get(&w.logits, n * m->V, 4);
  if (rc == LLMI_OK) rc = get(&w.ids, n, 4);
  if (rc == LLMI_OK) rc = get(&w.next, 1, 4);
  if (rc == LLMI_OK) rc = get(&w.am_v, kArgmaxBlocks, 4);
  if (rc == LLMI_OK) rc = get(&w.am_i, kArgmaxBlocks, 4);
  if (rc == LLMI_OK) rc = get(&w.am_count, 1, 4);
  if (rc == LLMI_OK) rc = get(&w.step_state, 2, 4);
  if (rc == LLMI_OK) rc = get(&w.step_rope, m->hd, 4);
  if (rc == LLMI_OK && hipMemsetAsync(w.am_count, 0, sizeof(unsigned), library_stream()) != hipSuccess)
    rc = fail(LLMI_ERR_HIP, "workspace: memset");
  if (rc != LLMI_OK) {
    free_workspace(w);
    return rc;
  }
  w.tokens = n;
  return LLMI_OK;
}

// One token (T = 1) through the fused per-layer launches built by
// build_decode; the same arithmetic as forward_device.  Logits land in
// ws.logits.
// tolerance: llmi_hip_model_set_decode_mode's tolerance-mode step (needs
// tol_ready): the attention over position chunks, merged in the o_proj
// product's staging, and every matmul split over K (SplitProduct).
// g (tolerance mode only; may be null): a step captured once and replayed
// from a graph (its positions in device memory, GraphStep); the caller then
// advances cache->len itself.
int decode_step(llmi_hip_model* m, llmi_hip_cache* cache, hipStream_t s, bool tolerance = false,
                const GraphStep* g = nullptr) {
  const auto& c = m->c;
  Workspace& w = m->ws;
  DecodeBuffers& d = m->dec;
  const std::size_t pos = cache->len;
  if (pos + 1 > cache->cap || pos + 1 > m->table_len) return fail(LLMI_ERR_STATE, "forward_cached: cache is full");
  const int nh = static_cast<int>(c.num_heads), nkv = static_cast<int>(c.num_kv_heads);
  const int hd = static_cast<int>(m->hd);
  const float eps = static_cast<float>(c.rms_norm_eps);
  const float scale = 1.0F / std::sqrt(static_cast<float>(m->hd));
  const std::size_t per_layer = static_cast<std::size_t>(c.num_kv_heads) * cache->cap * m->hd;
  if (int rc = launch_dequantize_rows(m->embed, w.ids, 1, d.x, s)) return rc;
  const bool split = tolerance && m->tol_ready;
  // q|k|v start at zero in a split step: cleared by the previous layer's
  // o_proj launch (the previous split step's last layer for the first), or
  // here when the step before was not a split step.
  if (split && !m->qkv_clear)
    zero_floats<<<blocks_for(m->Q + 2 * m->KV), kThreads, 0, s>>>(d.q, static_cast<int>(m->Q + 2 * m->KV));
  m->qkv_clear = false;
  for (std::size_t li = 0; li < m->layers.size(); ++li) {
    const DeviceLayer& l = m->layers[li];
    if (split) {
      if (int rc = launch_split(l.s_qkv, s)) return rc;
      const int nch = launch_tol_attention(d.q, d.k, d.v, cache->k + li * per_layer, cache->v + li * per_layer,
                                           m->cos_t, m->sin_t, d.part, nh, nkv, hd, static_cast<int>(cache->cap),
                                           static_cast<int>(pos + 1), scale, s, g);
      // From a graph the combine takes the chunk count from the positions
      // in device memory and the run's chunk length (passed in its place).
      if (int rc = g != nullptr ? launch_split(l.s_o, s, g->chunk, g->npos_dev) : launch_split(l.s_o, s, nch))
        return rc;
      if (int rc = launch_split(l.s_gu, s)) return rc;
      if (int rc = launch_split(l.s_dn, s)) return rc;
      continue;
    }
    if (int rc = l.qkv.launch(s)) return rc;
    launch_decode_attention(d.q, d.k, d.v, cache->k + li * per_layer, cache->v + li * per_layer, m->cos_t,
                            m->sin_t, cache->scores, d.att, nh, nkv, hd, static_cast<int>(cache->cap),
                            static_cast<int>(pos + 1), scale, s);
    if (int rc = launch_matmul(l.wo, d.att, 1, nullptr, d.x, s, true)) return rc;
    if (int rc = l.gate_up.launch(s)) return rc;
    if (int rc = l.down_silu.launch(s)) return rc;
  }
  rmsnorm_rows<<<1, kThreads, 0, s>>>(d.x, m->final_norm, d.h, static_cast<int>(m->H), eps);
  const DeviceMatrix& head = m->tied ? m->embed : m->lm_head;
  if (int rc = launch_matmul(head, d.h, 1, nullptr, w.logits, s)) return rc;
  LLMI_TRY_HIP(hipGetLastError());
  m->qkv_clear = split;
  if (g == nullptr) cache->len = pos + 1;
  return LLMI_OK;
}

// The body of forward_device: the lm_head runs on rows [head_first,
// head_first + head_rows) of the final normalised states (exact GEMV, or the
// bf16-MFMA GEMM with mfma_head), logits from ws.logits row 0.
int forward_rows(llmi_hip_model* m, llmi_hip_cache* cache, std::size_t T, std::size_t head_first,
                 std::size_t head_rows, bool mfma_head, hipStream_t s, float* trace, bool mfma_all = false) {
  // Every linear of the layers on the bf16-MFMA GEMM (mfma_all) or exact.
  const auto linear = [&](const DeviceMatrix& w, const float* x, const float* bias, float* y, bool acc) {
    return mfma_all ? launch_gemm_single(w, x, T, bias, y, s, acc) : launch_matmul(w, x, T, bias, y, s, acc);
  };
  const auto& c = m->c;
  Workspace& w = m->ws;
  const std::size_t base = cache->len;
  if (base + T > cache->cap || base + T > m->table_len) return fail(LLMI_ERR_STATE, "forward_cached: cache is full");
  const int nh = static_cast<int>(c.num_heads), nkv = static_cast<int>(c.num_kv_heads);
  const int hd = static_cast<int>(m->hd);
  const float eps = static_cast<float>(c.rms_norm_eps);
  const float scale = 1.0F / std::sqrt(static_cast<float>(m->hd));
  const std::size_t per_layer = static_cast<std::size_t>(c.num_kv_heads) * cache->cap * m->hd;
  const unsigned tt = static_cast<unsigned>(T);

  if (int rc = launch_dequantize_rows(m->embed, w.ids, T, w.x, s)) return rc;
  const std::size_t state = T * m->H;
  if (trace != nullptr) LLMI_TRY_HIP(hipMemcpyAsync(trace, w.x, state * sizeof(float), hipMemcpyDeviceToHost, s));
  for (std::size_t li = 0; li < m->layers.size(); ++li) {
    const DeviceLayer& l = m->layers[li];
    float* kc = cache->k + li * per_layer;
    float* vc = cache->v + li * per_layer;
    rmsnorm_rows<<<tt, kThreads, 0, s>>>(w.x, l.attn_norm, w.h, static_cast<int>(m->H), eps);
    bool roped = false;
    if (mfma_all) {
      // q, k and v share h: one conversion and one GEMM launch.
      const GroupEntry qkv[3] = {{&l.wq, w.h, l.bq, w.q, T, false},
                                 {&l.wk, w.h, l.bk, w.k, T, false},
                                 {&l.wv, w.h, l.bv, w.v, T, false}};
      if (int rc = launch_gemm_entries(qkv, 3, s)) return rc;
    } else {
      const DeviceMatrix* qkv[3] = {&l.wq, &l.wk, &l.wv};
      const float* qkv_bias[3] = {l.bq, l.bk, l.bv};
      float* qkv_out[3] = {w.q, w.k, w.v};
      RopeCache rc_args;
      rc_args.cos_t = m->cos_t;
      rc_args.sin_t = m->sin_t;
      rc_args.kc = kc;
      rc_args.vc = vc;
      rc_args.base = static_cast<int>(base);
      rc_args.cap = static_cast<int>(cache->cap);
      if (int rc = launch_matmul_shared(qkv, qkv_bias, qkv_out, 3, w.h, T, s, hd == 64 ? &rc_args : nullptr, &roped))
        return rc;
    }
    if (!roped)
      rope_and_cache<<<tt, kThreads, 0, s>>>(w.q, w.k, w.v, kc, vc, m->cos_t, m->sin_t, nh, nkv, hd,
                                             static_cast<int>(cache->cap), static_cast<int>(base));
    launch_attention(w.q, kc, vc, w.att, nh, nkv, hd, static_cast<int>(cache->cap), static_cast<int>(base),
                     static_cast<int>(T), scale, s);
    if (int rc = linear(l.wo, w.att, nullptr, w.x, true)) return rc;
    rmsnorm_rows<<<tt, kThreads, 0, s>>>(w.x, l.mlp_norm, w.h, static_cast<int>(m->H), eps);
    bool fused = false;
    if (!mfma_all) {
      if (int rc = launch_gate_up_silu(l.gate, l.up, w.h, T, w.g, s, &fused)) return rc;
    }
    if (!fused) {
      if (mfma_all) {
        const GroupEntry gu[2] = {{&l.gate, w.h, nullptr, w.g, T, false}, {&l.up, w.h, nullptr, w.u, T, false}};
        if (int rc = launch_gemm_entries(gu, 2, s)) return rc;
      } else {
        const DeviceMatrix* gu[2] = {&l.gate, &l.up};
        const float* gu_bias[2] = {nullptr, nullptr};
        float* gu_out[2] = {w.g, w.u};
        if (int rc = launch_matmul_shared(gu, gu_bias, gu_out, 2, w.h, T, s)) return rc;
      }
      silu_mul<<<blocks_for(T * m->F), kThreads, 0, s>>>(w.g, w.u, T * m->F);
    }
    if (int rc = linear(l.down, w.g, nullptr, w.x, true)) return rc;
    if (trace != nullptr)
      LLMI_TRY_HIP(hipMemcpyAsync(trace + (li + 1) * state, w.x, state * sizeof(float), hipMemcpyDeviceToHost, s));
  }
  // The reference normalises every row (transformer.cpp:298), then applies the
  // head to the last one or to all of them.
  const std::size_t first = head_first;
  const std::size_t rows = head_rows;
  const std::size_t norm_first = trace != nullptr ? 0 : first;
  rmsnorm_rows<<<static_cast<unsigned>(T - norm_first), kThreads, 0, s>>>(
      w.x + norm_first * m->H, m->final_norm, w.h + norm_first * m->H, static_cast<int>(m->H), eps);
  if (trace != nullptr)
    LLMI_TRY_HIP(hipMemcpyAsync(trace + (m->layers.size() + 1) * state, w.h, state * sizeof(float),
                                hipMemcpyDeviceToHost, s));
  const DeviceMatrix& head = m->tied ? m->embed : m->lm_head;
  if (mfma_head) {
    if (int rc = launch_gemm_single(head, w.h + first * m->H, rows, nullptr, w.logits, s)) return rc;
  } else if (int rc = launch_matmul(head, w.h + first * m->H, rows, nullptr, w.logits, s)) {
    return rc;
  }
  LLMI_TRY_HIP(hipGetLastError());
  cache->len = base + T;
  return LLMI_OK;
}

// transformer.cpp:192-306 with the ids already on the device (ws.ids).  The
// logits of rows first..T-1 land in ws.logits.  trace (host, optional):
// (layers + 2) x T x H floats -- the embeddings, every layer's output and
// the final RMSNorm, as the reference's ForwardTrace (transformer.hpp:14-19).
int forward_device(llmi_hip_model* m, llmi_hip_cache* cache, std::size_t T, bool all_positions, hipStream_t s,
                   float* trace = nullptr) {
  // The capacity and context checks of transformer.cpp:209-210, repeated
  // here because the generate loops call this once per step without going
  // through validate(): a step past the cache would write K/V and read RoPE
  // tables out of bounds.
  if (cache->len + T > cache->cap) return fail(LLMI_ERR_STATE, "forward_cached: cache is full");
  if (cache->len + T > m->c.max_position_embeddings)
    return fail(LLMI_ERR_STATE, "forward_cached: sequence longer than the model's context");
  const int nh = static_cast<int>(m->c.num_heads), nkv = static_cast<int>(m->c.num_kv_heads);
  if (T == 1 && trace == nullptr && m->type != LLMI_TYPE_F32) {
    if (m->decode_mode == LLMI_DECODE_TOLERANCE && m->tol_ready) return decode_step(m, cache, s, true);
    if (decode_attention_fits(nh, nkv, static_cast<int>(m->hd), cache->len + 1)) return decode_step(m, cache, s);
  }
  const std::size_t first = all_positions ? 0 : T - 1;
  return forward_rows(m, cache, T, first, T - first, false, s, trace);
}

// A cache of `cap` positions (the caller has clamped cap to the context):
// new_cache's allocation (transformer.cpp:182-190), or -- reuse != nullptr --
// that cache re-shaped to cap positions when its allocation holds them.
// The layout [layer][kv_head][cap][hd] changes with cap, so a reused cache
// starts empty.
int alloc_cache(llmi_hip_model* m, std::size_t cap, llmi_hip_cache* reuse, llmi_hip_cache** out) {
  *out = nullptr;
  if (cap == 0) return fail(LLMI_ERR_ARG, "new_cache: max_len must be positive");
  LLMI_REQUIRE(attention_dyn_lds(cap, m->hd) + attention_static_lds() <= max_lds_per_block(),
               "new_cache: capacity exceeds the attention kernel's LDS");
  if (int rc = ensure_tables(m, cap)) return rc;
  const std::size_t kv = m->layers.size() * m->c.num_kv_heads * cap * m->hd;
  const std::size_t sc = static_cast<std::size_t>(m->c.num_heads) * cap;
  if (reuse != nullptr && reuse->kv_elems >= kv && reuse->score_elems >= sc) {
    reuse->cap = cap;
    reuse->len = 0;
    *out = reuse;
    return LLMI_OK;
  }
  auto c = std::make_unique<llmi_hip_cache>();
  c->model = m;
  c->cap = cap;
  LLMI_TRY_HIP(hipMalloc(&c->k, kv * sizeof(float)));
  if (hipMalloc(&c->v, kv * sizeof(float)) != hipSuccess) {
    (void)hipFree(c->k);
    return fail(LLMI_ERR_HIP, "new_cache: hipMalloc");
  }
  if (hipMalloc(&c->scores, sc * sizeof(float)) != hipSuccess) {
    (void)hipFree(c->k);
    (void)hipFree(c->v);
    return fail(LLMI_ERR_HIP, "new_cache: hipMalloc");
  }
  c->kv_elems = kv;
  c->score_elems = sc;
  *out = c.release();
  return LLMI_OK;
}

// The model's own cache for calls that need one only while they run,
// sized for min(max_len, context) positions and empty.
int scratch_cache(llmi_hip_model* m, std::size_t max_len, llmi_hip_cache** out) {
  const std::size_t cap = std::min<std::size_t>(max_len, m->c.max_position_embeddings);
  llmi_hip_cache* c = nullptr;
  if (int rc = alloc_cache(m, cap, m->scratch, &c)) return rc;
  if (c != m->scratch) {
    (void)llmi_hip_cache_free(m->scratch);  // synchronises the stream first
    m->scratch = c;
  }
  *out = c;
  return LLMI_OK;
}

// Validation of transformer.cpp:204-212, with the reference's messages.
int validate(llmi_hip_model* m, llmi_hip_cache* cache, const std::int32_t* tokens, std::size_t T) {
  if (T == 0) return fail(LLMI_ERR_ARG, "forward_cached: no tokens");
  if (cache == nullptr || cache->model != m) return fail(LLMI_ERR_STATE, "forward_cached: cache was not created by this model");
  if (cache->len + T > cache->cap) return fail(LLMI_ERR_STATE, "forward_cached: cache is full");
  if (cache->len + T > m->c.max_position_embeddings)
    return fail(LLMI_ERR_STATE, "forward_cached: sequence longer than the model's context");
  for (std::size_t t = 0; t < T; ++t)
    if (tokens[t] < 0 || static_cast<std::size_t>(tokens[t]) >= m->V)
      return fail(LLMI_ERR_ARG, "forward_cached: token id " + std::to_string(tokens[t]) + " out of range");
  return LLMI_OK;
}

}  // namespace
}  // namespace llmi_hip

using namespace llmi_hip;

extern "C" {

int llmi_hip_dot_dev(const float* a, const float* b, const int32_t* lens, size_t count, float* out, void* stream) {
  LLMI_REQUIRE_INIT();
  if (count == 0) return LLMI_OK;
  dot_many<<<blocks_for(count), kThreads, 0, pick(stream)>>>(a, b, lens, static_cast<int>(count), out);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int llmi_hip_rmsnorm_dev(const float* x, const float* w, size_t rows, size_t n, float eps, float* y, void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(n > 0 && n <= 0x7FFFFFFFu && rows <= 0x7FFFFFFFu, "rmsnorm: bad shape");
  if (rows == 0) return LLMI_OK;
  rmsnorm_rows<<<static_cast<unsigned>(rows), kThreads, 0, pick(stream)>>>(x, w, y, static_cast<int>(n), eps);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int llmi_hip_softmax_dev(float* x, size_t rows, size_t n, void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(n * sizeof(float) + 4096 <= max_lds_per_block(), "softmax: row longer than the kernel's LDS");
  if (rows == 0 || n == 0) return LLMI_OK;
  softmax_rows<<<static_cast<unsigned>(rows), kThreads, n * sizeof(float), pick(stream)>>>(x, static_cast<int>(n));
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int llmi_hip_silu_dev(float* x, size_t n, void* stream) {
  LLMI_REQUIRE_INIT();
  if (n == 0) return LLMI_OK;
  silu_inplace<<<blocks_for(n), kThreads, 0, pick(stream)>>>(x, n);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int llmi_hip_argmax_dev(const float* x, size_t n, int32_t* out, void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(n > 0 && n <= 0x7FFFFFFFu, "argmax: bad length");
  argmax_first<<<1, 1024, 0, pick(stream)>>>(x, static_cast<int>(n), out, nullptr);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int llmi_hip_model_create(const llmi_model_config* cfg, const float* const* tensors, int type, llmi_hip_model** model) {
  return create_model(cfg, tensors, type, false, model);
}

int llmi_hip_model_create_dev(const llmi_model_config* cfg, const float* const* tensors_dev, int type,
                              llmi_hip_model** model) {
  return create_model(cfg, tensors_dev, type, true, model);
}

int llmi_hip_model_free(llmi_hip_model* m) {
  if (m == nullptr) return LLMI_OK;
  if (library_stream() != nullptr) (void)hipStreamSynchronize(library_stream());
  release_decode(m);
  (void)llmi_hip_cache_free(m->scratch);
  for (void* p : m->allocations) (void)hipFree(p);
  if (m->cos_t != nullptr) (void)hipFree(m->cos_t);
  if (m->sin_t != nullptr) (void)hipFree(m->sin_t);
  free_workspace(m->ws);
  delete m;
  return LLMI_OK;
}

size_t llmi_hip_model_weight_bytes(const llmi_hip_model* m) {
  if (m == nullptr) return 0;
  // Weight::byte_size (weight.cpp:26-28): fp32 values, or packed codes + scales.
  auto qbytes = [&](std::size_t out, std::size_t in) {
    if (m->type == LLMI_TYPE_F32) return out * in * sizeof(float);
    return out * row_bytes(in, m->type) + out * ceil_div(in, kBlock) * sizeof(float);
  };
  std::size_t total = qbytes(m->V, m->H) + (m->tied ? 0 : qbytes(m->V, m->H));
  total += m->layers.size() * (qbytes(m->Q, m->H) + 2 * qbytes(m->KV, m->H) + qbytes(m->H, m->Q) +
                               2 * qbytes(m->F, m->H) + qbytes(m->H, m->F));
  return total;
}

int llmi_hip_model_new_cache(llmi_hip_model* m, size_t max_len, llmi_hip_cache** cache) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(m != nullptr && cache != nullptr, "new_cache: null pointer");
  *cache = nullptr;
  return alloc_cache(m, std::min<std::size_t>(max_len, m->c.max_position_embeddings), nullptr, cache);
}

int llmi_hip_cache_free(llmi_hip_cache* c) {
  if (c == nullptr) return LLMI_OK;
  if (library_stream() != nullptr) (void)hipStreamSynchronize(library_stream());
  (void)hipFree(c->k);
  (void)hipFree(c->v);
  (void)hipFree(c->scores);
  delete c;
  return LLMI_OK;
}

size_t llmi_hip_cache_length(const llmi_hip_cache* c) { return c == nullptr ? 0 : c->len; }
size_t llmi_hip_cache_capacity(const llmi_hip_cache* c) { return c == nullptr ? 0 : c->cap; }
int llmi_hip_cache_reset(llmi_hip_cache* c) {
  LLMI_REQUIRE(c != nullptr, "cache_reset: null cache");
  c->len = 0;
  return LLMI_OK;
}

int llmi_hip_model_forward_cached_trace(llmi_hip_model* m, llmi_hip_cache* cache, const int32_t* tokens, size_t n,
                                        int all_positions, float* logits, float* states) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(m != nullptr, "forward_cached: null model");
  if (int rc = validate(m, cache, tokens, n)) return rc;
  if (int rc = ensure_workspace(m, n)) return rc;
  hipStream_t s = library_stream();
  LLMI_TRY_HIP(hipMemcpyAsync(m->ws.ids, tokens, n * sizeof(std::int32_t), hipMemcpyHostToDevice, s));
  if (int rc = forward_device(m, cache, n, all_positions != 0, s, states)) return rc;
  const std::size_t rows = all_positions ? n : 1;
  if (logits != nullptr)
    LLMI_TRY_HIP(hipMemcpyAsync(logits, m->ws.logits, rows * m->V * sizeof(float), hipMemcpyDeviceToHost, s));
  LLMI_TRY_HIP(hipStreamSynchronize(s));
  return LLMI_OK;
}

// Transformer::forward (transformer.cpp:78-166): the whole sequence through
// the model's own scratch cache, reset first -- bit-identical to
// forward_cached on a fresh cache (transformer_test.cpp:322-339).
int llmi_hip_model_forward(llmi_hip_model* m, const int32_t* tokens, size_t n, int all_positions, float* logits,
                           float* states) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(m != nullptr, "forward: null model");
  if (n == 0) return fail(LLMI_ERR_ARG, "forward: no tokens");
  if (n > m->c.max_position_embeddings)
    return fail(LLMI_ERR_STATE, "forward: sequence longer than the model's context");
  for (std::size_t t = 0; t < n; ++t)
    if (tokens[t] < 0 || static_cast<std::size_t>(tokens[t]) >= m->V)
      return fail(LLMI_ERR_ARG, "forward: token id " + std::to_string(tokens[t]) + " out of range");
  llmi_hip_cache* cache = nullptr;
  if (int rc = scratch_cache(m, n, &cache)) return rc;
  return llmi_hip_model_forward_cached_trace(m, cache, tokens, n, all_positions, logits, states);
}

int llmi_hip_model_forward_cached(llmi_hip_model* m, llmi_hip_cache* cache, const int32_t* tokens, size_t n,
                                  int all_positions, float* logits) {
  return llmi_hip_model_forward_cached_trace(m, cache, tokens, n, all_positions, logits, nullptr);
}

// transformer.cpp:308-327: prefill once, then one token per step; the argmax
// runs on the device and feeds the next step's embedding gather directly.
// Without stop ids nothing waits for the host between steps: the ids collect
// in device memory and are copied back once.
// The tolerance-mode greedy loop from graphs (generate_greedy).  Capture
// (before the prompt's prefill, so that its host time is not in the decode
// span) of one token -- argmax of the logits into ids and gen[state[1]],
// which then advances the state, and the decode step with its positions from
// state[0] -- once into a one-token graph and kGraphTokens times into another (a
// replay's fixed cost, once per kGraphTokens tokens).  A capture the runtime
// refuses leaves the graphs null (the eager loop runs).  Replay (after the
// prefill): the state set, the graphs for every token but the last, the
// last argmax; the caller synchronizes before the destructor frees them.
constexpr std::size_t kGraphMinSteps = 8;
constexpr int kGraphTokens = 4;
struct GreedyGraph {
  hipGraph_t graph[2] = {nullptr, nullptr};
  hipGraphExec_t exec[2] = {nullptr, nullptr};  // one token, kGraphTokens tokens
  GreedyGraph() = default;
  GreedyGraph(const GreedyGraph&) = delete;
  GreedyGraph& operator=(const GreedyGraph&) = delete;
  bool ready() const { return exec[0] != nullptr && exec[1] != nullptr; }
  ~GreedyGraph() {
    for (int i = 0; i < 2; ++i) {
      if (exec[i] != nullptr) (void)hipGraphExecDestroy(exec[i]);
      if (graph[i] != nullptr) (void)hipGraphDestroy(graph[i]);
    }
  }
};
void greedy_graph_capture(llmi_hip_model* m, llmi_hip_cache* cache, std::size_t last_npos, hipStream_t s,
                          GreedyGraph* g) {
  Workspace& w = m->ws;
  const int V = static_cast<int>(m->V);
  const int half = static_cast<int>(m->hd / 2);
  // The run's chunk length: that of its last step, so every step's positions
  // fit kAttnMaxChunks chunks.
  const GraphStep gs{w.step_state, w.step_rope, attn_chunk_len(static_cast<int>(last_npos))};
  const bool clear = m->qkv_clear;
  for (int i = 0; i < 2; ++i) {
    if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) break;
    m->qkv_clear = true;  // the replays' q|k|v are cleared by the step before (or before the first)
    bool ok = true;
    for (int t = 0; ok && t < (i == 0 ? 1 : kGraphTokens); ++t) {
      argmax_many<<<kArgmaxBlocks, kThreads, 0, s>>>(w.logits, V, w.am_v, w.am_i, w.am_count, w.ids, w.gen,
                                                     w.step_state + 1, w.step_state, m->cos_t, m->sin_t, w.step_rope,
                                                     half);
      ok = hipGetLastError() == hipSuccess;
      if (ok) ok = decode_step(m, cache, s, true, &gs) == LLMI_OK;
    }
    const hipError_t ended = hipStreamEndCapture(s, &g->graph[i]);
    if (!ok || ended != hipSuccess || g->graph[i] == nullptr ||
        hipGraphInstantiate(&g->exec[i], g->graph[i], nullptr, nullptr, 0) != hipSuccess)
      break;
  }
  m->qkv_clear = clear;
  (void)hipGetLastError();
  if (!g->ready()) {
    for (int i = 0; i < 2; ++i) {
      if (g->exec[i] != nullptr) (void)hipGraphExecDestroy(g->exec[i]);
      g->exec[i] = nullptr;
    }
  }
}
int greedy_graph_run(llmi_hip_model* m, llmi_hip_cache* cache, std::size_t max_new, hipStream_t s,
                     const GreedyGraph& g) {
  Workspace& w = m->ws;
  DecodeBuffers& d = m->dec;
  const int V = static_cast<int>(m->V);
  if (cache->len + max_new > cache->cap || cache->len + max_new > m->table_len)
    return fail(LLMI_ERR_STATE, "forward_cached: cache is full");
  if (!m->qkv_clear)
    zero_floats<<<blocks_for(m->Q + 2 * m->KV), kThreads, 0, s>>>(d.q, static_cast<int>(m->Q + 2 * m->KV));
  // The state of the step before the first replayed one (cache->len >= 1
  // after the prefill): the first replay's argmax moves it on.
  step_state_set<<<1, 64, 0, s>>>(w.step_state, static_cast<int>(cache->len), 0, m->cos_t, m->sin_t, w.step_rope,
                                  static_cast<int>(m->hd / 2));
  LLMI_TRY_HIP(hipGetLastError());
  std::size_t k = 0;
  for (; k + kGraphTokens + 1 <= max_new; k += kGraphTokens) LLMI_TRY_HIP(hipGraphLaunch(g.exec[1], s));
  for (; k + 1 < max_new; ++k) LLMI_TRY_HIP(hipGraphLaunch(g.exec[0], s));
  argmax_many<<<kArgmaxBlocks, kThreads, 0, s>>>(w.logits, V, w.am_v, w.am_i, w.am_count, w.ids, w.gen,
                                                 w.step_state + 1, nullptr, nullptr, nullptr, nullptr, 0);
  LLMI_TRY_HIP(hipGetLastError());
  cache->len += max_new - 1;
  m->qkv_clear = true;
  return LLMI_OK;
}

int llmi_hip_model_generate_greedy(llmi_hip_model* m, const int32_t* prompt, size_t n, size_t max_new,
                                   const int32_t* stop_ids, size_t n_stop, int32_t* ids, size_t* n_ids) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(m != nullptr && ids != nullptr && n_ids != nullptr, "generate_greedy: null pointer");
  *n_ids = 0;
  llmi_hip_cache* cache = nullptr;
  if (int rc = scratch_cache(m, n + max_new, &cache)) return rc;
  if (int rc = validate(m, cache, prompt, n)) return rc;
  if (max_new == 0) return LLMI_OK;
  if (int rc = ensure_workspace(m, n)) return rc;
  Workspace& w = m->ws;
  if (w.gen_cap < max_new) {
    if (w.gen != nullptr) (void)hipFree(w.gen);
    w.gen = nullptr;
    w.gen_cap = 0;
    LLMI_TRY_HIP(hipMalloc(&w.gen, max_new * sizeof(std::int32_t)));
    w.gen_cap = max_new;
  }
  hipStream_t s = library_stream();
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  for (auto& e : ev) LLMI_TRY_HIP(hipEventCreate(&e));
  struct EvGuard {
    hipEvent_t* e;
    ~EvGuard() {
      for (int i = 0; i < 3; ++i)
        if (e[i] != nullptr) (void)hipEventDestroy(e[i]);
    }
  } ev_guard{ev};
  // Tolerance-mode steps (no stop ids) replay one captured graph: the host
  // then enqueues one launch per token instead of ~5 per layer.  Anything
  // the capture does not take leaves the eager loop below.
  GreedyGraph graph;
  if (m->decode_graph && m->decode_mode == LLMI_DECODE_TOLERANCE && m->tol_ready && n_stop == 0 &&
      max_new >= kGraphMinSteps)
    greedy_graph_capture(m, cache, n + max_new - 1, s, &graph);
  LLMI_TRY_HIP(hipMemcpyAsync(w.ids, prompt, n * sizeof(std::int32_t), hipMemcpyHostToDevice, s));
  LLMI_TRY_HIP(hipEventRecord(ev[0], s));
  if (int rc = forward_device(m, cache, n, false, s)) return rc;
  LLMI_TRY_HIP(hipEventRecord(ev[1], s));
  const int V = static_cast<int>(m->V);
  std::size_t produced = 0;
  if (graph.ready()) {
    if (int rc = greedy_graph_run(m, cache, max_new, s, graph)) return rc;
    produced = max_new;
  }
  for (std::size_t step = produced; step < max_new; ++step) {
    argmax_many<<<kArgmaxBlocks, kThreads, 0, s>>>(w.logits, V, w.am_v, w.am_i, w.am_count, w.ids, w.gen + step,
                                                   nullptr, nullptr, nullptr, nullptr, nullptr, 0);
    LLMI_TRY_HIP(hipGetLastError());
    produced = step + 1;
    if (n_stop > 0) {
      std::int32_t next = 0;
      LLMI_TRY_HIP(hipMemcpyAsync(&next, w.ids, sizeof(next), hipMemcpyDeviceToHost, s));
      LLMI_TRY_HIP(hipStreamSynchronize(s));
      bool stop = false;
      for (std::size_t k = 0; k < n_stop; ++k) stop = stop || stop_ids[k] == next;
      if (stop) break;
    }
    if (step + 1 == max_new) break;
    if (int rc = forward_device(m, cache, 1, false, s)) return rc;
  }
  LLMI_TRY_HIP(hipEventRecord(ev[2], s));
  LLMI_TRY_HIP(hipMemcpyAsync(ids, w.gen, produced * sizeof(std::int32_t), hipMemcpyDeviceToHost, s));
  LLMI_TRY_HIP(hipStreamSynchronize(s));
  float pre = 0.0f, dec = 0.0f;
  LLMI_TRY_HIP(hipEventElapsedTime(&pre, ev[0], ev[1]));
  LLMI_TRY_HIP(hipEventElapsedTime(&dec, ev[1], ev[2]));
  m->last_prefill_ms = pre;
  m->last_decode_ms = dec;
  *n_ids = produced;
  return LLMI_OK;
}

// One serving step: forward_cached, then sample() on the last position's
// logits in HBM (sampling.hip).
int llmi_hip_model_forward_sample(llmi_hip_model* m, llmi_hip_cache* cache, const int32_t* tokens, size_t n,
                                  const llmi_hip_sampling* cfg, double target, int32_t* id) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(m != nullptr && cfg != nullptr && id != nullptr, "forward_sample: null pointer");
  if (int rc = validate(m, cache, tokens, n)) return rc;
  if (int rc = ensure_workspace(m, n)) return rc;
  hipStream_t s = library_stream();
  LLMI_TRY_HIP(hipMemcpyAsync(m->ws.ids, tokens, n * sizeof(std::int32_t), hipMemcpyHostToDevice, s));
  if (int rc = forward_device(m, cache, n, false, s)) return rc;
  return sample_device(m->ws.logits, m->V, *cfg, target, id, nullptr, s);
}

// generate_greedy with sample() per step: the drawn index also lands in the
// next step's token slot on the device, so the host only reads it (to stop).
int llmi_hip_model_generate_sampled(llmi_hip_model* m, const int32_t* prompt, size_t n, size_t max_new,
                                    const llmi_hip_sampling* cfg, const double* targets, const int32_t* stop_ids,
                                    size_t n_stop, int32_t* ids, size_t* n_ids) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(m != nullptr && cfg != nullptr && ids != nullptr && n_ids != nullptr, "generate_sampled: null pointer");
  LLMI_REQUIRE(targets != nullptr || max_new == 0 || cfg->temperature <= 0.0f, "generate_sampled: null targets");
  *n_ids = 0;
  m->last_redraws = 0;
  llmi_hip_cache* cache = nullptr;
  if (int rc = scratch_cache(m, n + max_new, &cache)) return rc;
  if (int rc = validate(m, cache, prompt, n)) return rc;
  if (max_new == 0) return LLMI_OK;
  if (int rc = ensure_workspace(m, n)) return rc;
  Workspace& w = m->ws;
  hipStream_t s = library_stream();
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  for (auto& e : ev) LLMI_TRY_HIP(hipEventCreate(&e));
  struct EvGuard {
    hipEvent_t* e;
    ~EvGuard() {
      for (int i = 0; i < 3; ++i)
        if (e[i] != nullptr) (void)hipEventDestroy(e[i]);
    }
  } ev_guard{ev};
  LLMI_TRY_HIP(hipMemcpyAsync(w.ids, prompt, n * sizeof(std::int32_t), hipMemcpyHostToDevice, s));
  LLMI_TRY_HIP(hipEventRecord(ev[0], s));
  if (int rc = forward_device(m, cache, n, false, s)) return rc;
  LLMI_TRY_HIP(hipEventRecord(ev[1], s));
  std::size_t produced = 0;
  std::size_t step = 0;
  bool done = false;
  if (cfg->temperature > 0.0f) {
    // Windows of steps queued without a host round trip: each draw writes its
    // index where the next step's forward reads it, and its outcome to the
    // window's log; the host reads the log once per window.  Stop ids end the
    // run at the first one (the window's later steps are discarded).  At the
    // first undecided draw of a window (a bound left the index open, or bad
    // logits) the cache is rolled back to that step and its logits
    // recomputed; sample_device settles the draw exactly (or reports the bad
    // logits), and queueing resumes after it.  Only steps whose following
    // forward fits the cache are queued: a run that reaches the end of the
    // cache does so step by step below, so a stop id drawn first still ends
    // it without the "cache is full" failure.
    if (w.slog == nullptr) LLMI_TRY_HIP(hipMalloc(&w.slog, kSampleWindow * sizeof(SampleLog)));
    SampleLog hlog[kSampleWindow];
    const std::size_t queued_end = std::min(max_new, cache->cap - n);
    auto is_stop = [&](std::int32_t id) {
      for (std::size_t k = 0; k < n_stop; ++k)
        if (stop_ids[k] == id) return true;
      return false;
    };
    while (step < queued_end && !done) {
      const std::size_t end = std::min(queued_end, step + kSampleWindow);
      for (std::size_t t = step; t < end; ++t) {
        if (int rc = sample_device_async(w.logits, m->V, *cfg, targets[t], w.ids, w.slog + (t - step), s)) return rc;
        if (t + 1 < max_new)
          if (int rc = forward_device(m, cache, 1, false, s)) return rc;
      }
      LLMI_TRY_HIP(hipMemcpyAsync(hlog, w.slog, (end - step) * sizeof(SampleLog), hipMemcpyDeviceToHost, s));
      LLMI_TRY_HIP(hipStreamSynchronize(s));
      std::size_t t = step;
      for (; t < end && !done; ++t) {
        if ((hlog[t - step].state & 1) == 0) break;
        ids[t] = hlog[t - step].id;
        produced = t + 1;
        done = is_stop(ids[t]);
      }
      step = t;
      if (done || t == end) continue;
      // Undecided draw at step t: its logits come from the prompt (t = 0) or
      // from token t - 1 at position n + t - 1.
      ++m->last_redraws;
      if (t == 0) {
        cache->len = 0;
        LLMI_TRY_HIP(hipMemcpyAsync(w.ids, prompt, n * sizeof(std::int32_t), hipMemcpyHostToDevice, s));
        if (int rc = forward_device(m, cache, n, false, s)) return rc;
      } else {
        cache->len = n + t - 1;
        LLMI_TRY_HIP(hipMemcpyAsync(w.ids, &ids[t - 1], sizeof(std::int32_t), hipMemcpyHostToDevice, s));
        if (int rc = forward_device(m, cache, 1, false, s)) return rc;
      }
      if (int rc = sample_device(w.logits, m->V, *cfg, targets[t], &ids[t], w.ids, s)) return rc;
      produced = t + 1;
      done = is_stop(ids[t]);
      step = t + 1;
      if (!done && step < max_new)
        if (int rc = forward_device(m, cache, 1, false, s)) return rc;
    }
  }
  // Step by step: temperature <= 0, and the steps whose forward would not
  // fit the cache.
  for (; step < max_new && !done; ++step) {
    std::int32_t next = 0;
    const double target = cfg->temperature > 0.0f ? targets[step] : 0.0;
    if (int rc = sample_device(w.logits, m->V, *cfg, target, &next, w.ids, s)) return rc;
    ids[step] = next;
    produced = step + 1;
    bool stop = false;
    for (std::size_t k = 0; k < n_stop; ++k) stop = stop || stop_ids[k] == next;
    if (stop || step + 1 == max_new) break;
    if (int rc = forward_device(m, cache, 1, false, s)) return rc;
  }
  LLMI_TRY_HIP(hipEventRecord(ev[2], s));
  LLMI_TRY_HIP(hipStreamSynchronize(s));
  float pre = 0.0f, dec = 0.0f;
  LLMI_TRY_HIP(hipEventElapsedTime(&pre, ev[0], ev[1]));
  LLMI_TRY_HIP(hipEventElapsedTime(&dec, ev[1], ev[2]));
  m->last_prefill_ms = pre;
  m->last_decode_ms = dec;
  *n_ids = produced;
  return LLMI_OK;
}

int llmi_hip_model_chunk_nll(llmi_hip_model* m, const int32_t* tokens, size_t n, size_t t_start, int mode,
                             double* nll) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(m != nullptr, "chunk_nll: null model");
  LLMI_REQUIRE(mode == LLMI_SCORE_EXACT || mode == LLMI_SCORE_MFMA_HEAD || mode == LLMI_SCORE_MFMA,
               "chunk_nll: mode must be LLMI_SCORE_EXACT, _MFMA_HEAD or _MFMA");
  llmi_hip_cache* cache = nullptr;
  if (int rc = scratch_cache(m, n, &cache)) return rc;
  if (int rc = validate(m, cache, tokens, n)) return rc;
  LLMI_REQUIRE(nll != nullptr || t_start + 1 >= n, "chunk_nll: null nll");
  if (int rc = ensure_workspace(m, n)) return rc;
  Workspace& w = m->ws;
  hipStream_t s = library_stream();
  const std::size_t first = std::min(t_start, n - 1);
  const std::size_t rows = n - 1 - first;  // the last position predicts nothing inside the chunk
  LLMI_TRY_HIP(hipMemcpyAsync(w.ids, tokens, n * sizeof(std::int32_t), hipMemcpyHostToDevice, s));
  if (int rc = forward_rows(m, cache, n, first, rows, mode != LLMI_SCORE_EXACT, s, nullptr, mode == LLMI_SCORE_MFMA))
    return rc;
  if (rows == 0) return LLMI_OK;
  if (w.nll_cap < rows) {
    LLMI_TRY_HIP(hipStreamSynchronize(s));
    if (w.nll != nullptr) (void)hipFree(w.nll);
    w.nll = nullptr;
    w.nll_cap = 0;
    LLMI_TRY_HIP(hipMalloc(&w.nll, w.tokens * sizeof(double)));  // rows < n <= w.tokens
    w.nll_cap = w.tokens;
  }
  row_nll<<<static_cast<unsigned>(rows), kThreads, 0, s>>>(w.logits, static_cast<int>(m->V), w.ids + first + 1, w.nll);
  LLMI_TRY_HIP(hipGetLastError());
  LLMI_TRY_HIP(hipMemcpyAsync(nll, w.nll, rows * sizeof(double), hipMemcpyDeviceToHost, s));
  LLMI_TRY_HIP(hipStreamSynchronize(s));
  return LLMI_OK;
}

int llmi_hip_model_last_timing(const llmi_hip_model* m, double* prefill_ms, double* decode_ms) {
  LLMI_REQUIRE(m != nullptr, "last_timing: null model");
  if (prefill_ms != nullptr) *prefill_ms = m->last_prefill_ms;
  if (decode_ms != nullptr) *decode_ms = m->last_decode_ms;
  return LLMI_OK;
}

int llmi_hip_model_last_redraws(const llmi_hip_model* m, size_t* steps) {
  LLMI_REQUIRE(m != nullptr && steps != nullptr, "last_redraws: null pointer");
  *steps = m->last_redraws;
  return LLMI_OK;
}

int llmi_hip_model_set_decode_mode(llmi_hip_model* m, int mode) {
  LLMI_REQUIRE(m != nullptr, "set_decode_mode: null model");
  LLMI_REQUIRE(mode == LLMI_DECODE_EXACT || mode == LLMI_DECODE_TOLERANCE, "set_decode_mode: unknown mode");
  m->decode_mode = mode;
  return LLMI_OK;
}

int llmi_hip_model_set_decode_graph(llmi_hip_model* m, int enable) {
  LLMI_REQUIRE(m != nullptr, "set_decode_graph: null model");
  m->decode_graph = enable != 0;
  return LLMI_OK;
}

}  // extern "C"
