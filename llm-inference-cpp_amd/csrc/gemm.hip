// Prefill GEMM on the matrix cores (bf16 MFMA, fp32 accumulate) for gfx950.
//
// Reference: the prefill calls of quant::matmul (src/model/quant.cpp:119-153)
// with rows = T tokens (transformer.cpp:245-291).  y[t][o] = sum_k x[t][k] *
// code[o][k] * scale[o][k/32] (+ bias[o]).  Here x and the dequantized weights
// are rounded to bf16 and the products summed in fp32 by v_mfma_f32_16x16x32_bf16,
// so y differs from the reference by bf16 rounding (relative error ~1e-3;
// the tested bound is max|dy| <= 2e-2 * max|y|).  The exact path for the
// same shapes is llmi_hip_matmul_dev.
//
// x is first converted to bf16 once (x_to_bf16: row stride padded to a
// multiple of 64 with zeros), so the GEMM reads half the activation bytes
// and never converts them again.  One workgroup computes a 128 (tokens) x
// 256 (outputs) tile of y with 8 wavefronts (qgemm_mfma below): wavefront w
// owns outputs 32w..32w+31 and all 128 tokens.  Per K-step of 64 (two
// quantization blocks) each wavefront loads its own weight codes and scales
// two steps ahead and dequantizes them (code * scale, rounded to bf16) in
// registers while the current step's MFMAs run; the 128 x 64 activation
// tile is staged by all wavefronts into one of two LDS buffers (also two
// steps ahead through registers), one barrier per step.  The loads are
// unconditional (clamped addresses, the scale of a block past the row's end
// taken as 0): a load behind a per-lane branch makes the compiler wait for
// every load in flight.  LDS rows are padded by 16 bytes so that the 16-byte
// operand reads of 8 consecutive lanes hit distinct banks.
//
// Products are launched as groups (one kernel for many products; a single
// product is passed by value): workgroup w first maps to a work index so that
// consecutive work items -- the token tiles sharing one weight tile -- run on
// the same XCD (workgroups are dealt to the 8 XCDs round-robin), then finds
// its product through a work -> product map.
#include <algorithm>
#include <string>
#include <type_traits>
#include <vector>

#include "common.hpp"

namespace llmi_hip {

namespace {

#define GMEM __attribute__((address_space(1)))

constexpr int kBM = 128, kBN = 256, kBK = 64;
// K of more than kSplitMinSteps steps of kBK may be split over workgroups;
// kCus is MI355X's CU count.
constexpr std::size_t kSplitMinSteps = 24, kCus = 256;
constexpr int kGemmThreads = 512;  // 8 wavefronts side by side over the outputs
constexpr int kWavesN = 8;
constexpr int kWaveN = kBN / kWavesN;                      // outputs per wavefront (32)
constexpr int kWaveM = kBM / (kGemmThreads / 64 / kWavesN);  // tokens per wavefront (128)
constexpr int kJ = kWaveN / 16;                            // 16-output MFMA blocks per wavefront
constexpr int kI = kWaveM / 16;                            // 16-token MFMA blocks per wavefront
constexpr int kXPer = kBM * kBK / 8 / kGemmThreads;        // 16-byte chunks of the activation tile per thread
constexpr int kLdsRow = kBK + 8;  // bf16 per LDS row (16 bytes of padding)
constexpr int kXcds = 8;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ std::uint32_t pack_bf16(float a, float b) {
  const bf16x2 v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(std::uint32_t, v);
}

__device__ __forceinline__ int sbyte(std::uint32_t w, int i) {
  return static_cast<int>(__builtin_amdgcn_sbfe(w, i * 8, 8));
}
__device__ __forceinline__ int snib(std::uint32_t w, int i) {
  return static_cast<int>(__builtin_amdgcn_sbfe(w ^ 0x88888888u, i * 4, 4));
}

// xb[r][k] = bf16(x[r][k]) for k < in, 0 for in <= k < ldx.
// Up to kConvBatch activation matrices converted by one x_to_bf16_batch
// launch, in octets (8 consecutive elements of a row, ldx being a multiple
// of 64): input i covers octets [oend[i-1], oend[i]) of the launch's range,
// cpr[i] = ldx[i] / 8 per row; vec[i]: x rows are 16-byte aligned (in % 4 ==
// 0 and an aligned base), so whole octets load as two 16-byte vectors.
constexpr int kConvBatch = 16;
struct ConvBatch {
  const float* x[kConvBatch];
  std::uint16_t* xb[kConvBatch];
  int in[kConvBatch], ldx[kConvBatch];
  unsigned oend[kConvBatch];
  unsigned char vec[kConvBatch];
  int n;
};
__global__ void __launch_bounds__(256) x_to_bf16_batch(ConvBatch c) {
  const unsigned total = c.oend[c.n - 1];
  for (unsigned o = blockIdx.x * blockDim.x + threadIdx.x; o < total; o += gridDim.x * blockDim.x) {
    // Select this octet's input without indexing the argument block.
    const float* x = c.x[0];
    std::uint16_t* xb = c.xb[0];
    int in = c.in[0], ldx = c.ldx[0];
    unsigned o0 = 0;
    bool vec = c.vec[0] != 0;
#pragma unroll
    for (int k = 1; k < kConvBatch; ++k)
      if (k < c.n && o >= c.oend[k - 1]) {
        x = c.x[k];
        xb = c.xb[k];
        in = c.in[k];
        ldx = c.ldx[k];
        o0 = c.oend[k - 1];
        vec = c.vec[k] != 0;
      }
    const unsigned lo = o - o0, cpr = static_cast<unsigned>(ldx) >> 3;
    const unsigned r = lo / cpr;
    const int k0 = static_cast<int>(lo - r * cpr) * 8;
    const float* src = x + static_cast<std::size_t>(r) * in + k0;
    float v[8];
    if (vec && k0 + 8 <= in) {
      const f32x4 lo4 = *reinterpret_cast<const f32x4*>(src), hi4 = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        v[u] = lo4[u];
        v[u + 4] = hi4[u];
      }
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = k0 + u < in ? src[u] : 0.0f;
    }
    *reinterpret_cast<u32x4*>(xb + static_cast<std::size_t>(r) * ldx + k0) =
        u32x4{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7])};
  }
}

// One K-step (64 = two quantization blocks) of a wavefront's weights as
// loaded.  The step's K order is permuted (the same permutation for the
// activations, so the sums are unchanged): lane quarter q holds 16
// consecutive codes of block q/2 -- elements 16(q%2) .. 16(q%2)+15, one
// 16-byte load for Q8_0, 8 bytes for Q4_0 -- and feeds the first 8 to the
// step's first MFMA and the other 8 to its second; so for each column group
// j a lane needs one code load and one scale (its block's).  live: the
// lane's block exists (else its scale counts as 0).
template <int TYPE>
struct WStage {
  using Code = std::conditional_t<TYPE == LLMI_TYPE_Q8_0, u32x4, u32x2>;
  Code c[kJ];
  float sc[kJ];
  bool live;
};
// One K-step of the activation tile held by one thread: chunks t + 512u
// (16 bytes each) of the 128 x 64 bf16 tile.
struct XStage {
  u32x4 v[kXPer];
};

// qgemm_mfma: a workgroup computes a 128-token x 256-output tile of y = x W^T
// (or one K chunk of it) with 8 wavefronts.  Wavefront w owns outputs
// 32w..32w+31 of the tile and all 128 tokens: it loads its own weight codes
// (two K-steps ahead), dequantizes them to bf16 in registers for the next
// step while the current step's MFMAs run, and reads the activations from a
// double-buffered LDS tile that all wavefronts fill together (also two steps
// ahead through registers).  One barrier per K-step publishes the next
// activation tile and frees the one just read.
// F32X: the activations come as fp32 (p.xf, K a multiple of 64, rows
// 16-byte aligned) and are rounded to bf16 (the same rounding as
// x_to_bf16_batch) when staged in LDS; they are loaded one K-step ahead
// instead of two, which keeps the registers of the bf16 ring.
template <int TYPE, bool F32X = false>
__global__ void __launch_bounds__(kGemmThreads) qgemm_mfma(const GemmProblem* __restrict__ probs,
                                                           const std::uint32_t* __restrict__ work_prob, int total,
                                                           GemmFew few) {
  __shared__ __attribute__((aligned(16))) std::uint16_t xs[2][kBM * kLdsRow];

  // Work index: workgroup w runs on XCD w % 8; give each XCD a contiguous
  // range of work items.
  const int wgi = blockIdx.x;
  const int per = total / kXcds, extra = total % kXcds;
  const int xcd = wgi % kXcds, slot = wgi / kXcds;
  const int work = xcd * per + min(xcd, extra) + slot;
  // Up to kGemmFew products come by value (no table; the product by
  // comparisons and selects, so the argument block is never indexed
  // dynamically); a group through the map.
  const int fi = (few.count > 2 && work >= few.p[2].first_wg) ? 2 : (few.count > 1 && work >= few.p[1].first_wg) ? 1 : 0;
  GemmProblem p = fi == 2 ? few.p[2] : fi == 1 ? few.p[1] : few.p[0];
  if (probs != nullptr) p = probs[__builtin_amdgcn_readfirstlane(static_cast<int>(work_prob[work]))];
  const int local = work - p.first_wg;
  // Consecutive work items: the token tiles of one (weight tile, K chunk).
  const int mt = local % p.mtiles, rest = local / p.mtiles;
  const int kc = rest % p.kchunks, nt = rest / p.kchunks;
  const int m0 = mt * kBM, n0 = nt * kBN;
  const int M = p.rows, N = p.out, nblk = p.nblk, ldx = p.ldx;
  // This workgroup's K-steps of 64: [kb, kb + nk) of the product's.
  const int nk_all = (p.in + kBK - 1) / kBK;
  const int kb = kc * p.kpc;
  const int nk = min(p.kpc, nk_all - kb);

  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wn0 = (wave % kWavesN) * kWaveN, wm0 = (wave / kWavesN) * kWaveM;
  const int arow = lane & 15, q = lane >> 4;

  // Every load is issued unconditionally from an address inside the
  // operands (rows past M or N are clamped to the last one; their results
  // are never stored; steps past the last re-read it), so no load sits
  // behind a branch.
  // Each load addresses a base common to the wavefront (the operand, the
  // tile and the K-step: SGPR arithmetic) plus a lane offset in bytes fixed
  // for the whole loop, so a step's loads take no per-lane address work.
  using GB = const GMEM unsigned char*;
  std::uint32_t xoff[kXPer], xfoff[kXPer];
  int xlds[kXPer];
#pragma unroll
  for (int u = 0; u < kXPer; ++u) {
    const int c = t + kGemmThreads * u, row = c >> 3, col = c & 7;
    const int r = min(m0 + row, M - 1) - m0;  // the tile's row, clamped
    xoff[u] = static_cast<std::uint32_t>((r * ldx + col * 8) * 2);
    xfoff[u] = static_cast<std::uint32_t>((r * p.in + col * 8) * 4);
    xlds[u] = row * kLdsRow + col * 8;
  }
  const GB xb_tile = (GB)p.xb + static_cast<std::size_t>(m0) * ldx * 2;
  const GB xf_tile = (GB)p.xf + static_cast<std::size_t>(m0) * p.in * 4;
  const auto xload = [&](XStage& st, int j) {
    const GB base = xb_tile + static_cast<std::size_t>(kb + min(j, nk - 1)) * (kBK * 2);
#pragma unroll
    for (int u = 0; u < kXPer; ++u) st.v[u] = *(const GMEM u32x4*)(base + xoff[u]);
  };
  const auto xstore = [&](const XStage& st, int buf) {
#pragma unroll
    for (int u = 0; u < kXPer; ++u) *reinterpret_cast<u32x4*>(&xs[buf][xlds[u]]) = st.v[u];
  };
  // F32X: the same chunks of 8 elements from the fp32 rows (two 16-byte
  // loads each), converted when stored.
  const auto xloadf = [&](f32x4 (&st)[kXPer][2], int j) {
    const GB base = xf_tile + static_cast<std::size_t>(kb + min(j, nk - 1)) * (kBK * 4);
#pragma unroll
    for (int u = 0; u < kXPer; ++u) {
      st[u][0] = *(const GMEM f32x4*)(base + xfoff[u]);
      st[u][1] = *(const GMEM f32x4*)(base + xfoff[u] + 16);
    }
  };
  const auto xstoref = [&](const f32x4 (&st)[kXPer][2], int buf) {
#pragma unroll
    for (int u = 0; u < kXPer; ++u)
      *reinterpret_cast<u32x4*>(&xs[buf][xlds[u]]) =
          u32x4{pack_bf16(st[u][0][0], st[u][0][1]), pack_bf16(st[u][0][2], st[u][0][3]),
                pack_bf16(st[u][1][0], st[u][1][1]), pack_bf16(st[u][1][2], st[u][1][3])};
  };

  // This lane's weight rows (columns of the tile): n0 + wn0 + 16j + lane%16,
  // clamped into the padded matrix.  A wavefront's rows are 32 aligned rows,
  // so they lie in one 64-row tile (the last one for rows past the matrix).
  const int wtile = min((n0 + wn0) / kTileRows, p.ntiles - 1);
  std::uint32_t wco[kJ], wso[kJ];  // lane offsets (bytes) of codes and scales in a block
#pragma unroll
  for (int jj = 0; jj < kJ; ++jj) {
    const int r = min(n0 + wn0 + 16 * jj + arow, p.ntiles * kTileRows - 1) - wtile * kTileRows;
    if constexpr (TYPE == LLMI_TYPE_Q8_0)
      wco[jj] = static_cast<std::uint32_t>((q & 1) * kTileRows * 16 + r * 16);  // 16-byte half q%2 of the row
    else
      wco[jj] = static_cast<std::uint32_t>(r * 16 + (q & 1) * 8);  // bytes 8(q%2) .. of the row
    wso[jj] = static_cast<std::uint32_t>(r * 4);
  }
  constexpr std::size_t kBlockBytes = (TYPE == LLMI_TYPE_Q8_0 ? 32 : 16) * kTileRows;  // codes of one 64-row block
  const GB wcodes = (GB)p.codes + static_cast<std::size_t>(wtile) * nblk * kBlockBytes;
  const GB wscales = (GB)p.scales + static_cast<std::size_t>(wtile) * nblk * kTileRows * 4;
  const auto wload = [&](WStage<TYPE>& st, int j) {
    const int k = kb + min(j, nk - 1);
    const int blk = 2 * k + (q >> 1);
    st.live = blk < nblk;
    const int bc = min(blk, nblk - 1);
    const GB cb = wcodes + static_cast<std::size_t>(bc) * kBlockBytes;
    const GB sb = wscales + static_cast<std::size_t>(bc) * kTileRows * 4;
#pragma unroll
    for (int jj = 0; jj < kJ; ++jj) {
      if constexpr (TYPE == LLMI_TYPE_Q8_0) st.c[jj] = *(const GMEM u32x4*)(cb + wco[jj]);
      else st.c[jj] = *(const GMEM u32x2*)(cb + wco[jj]);
      st.sc[jj] = *(const GMEM float*)(sb + wso[jj]);
    }
  };
  // bf16(code * scale), the operand of the fp32 restatement rounded once.
  // bf[t][j]: the codes the lane feeds the step's MFMA t for column group j.
  const auto dequant = [&](const WStage<TYPE>& st, bf16x8 (&bf)[2][kJ]) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int jj = 0; jj < kJ; ++jj) {
        const float sc = st.live ? st.sc[jj] : 0.0f;
        float c[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          int code;
          if constexpr (TYPE == LLMI_TYPE_Q8_0) code = sbyte(st.c[jj][2 * s + (e >> 2)], e & 3);
          else code = snib(st.c[jj][s], e);
          c[e] = static_cast<float>(code) * sc;
        }
        const u32x4 pk{pack_bf16(c[0], c[1]), pack_bf16(c[2], c[3]), pack_bf16(c[4], c[5]), pack_bf16(c[6], c[7])};
        bf[s][jj] = __builtin_bit_cast(bf16x8, pk);
      }
  };

  f32x4 acc[kI][kJ];
#pragma unroll
  for (int i = 0; i < kI; ++i)
#pragma unroll
    for (int j = 0; j < kJ; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  // One K-step: 2 kI activation fragments (lane quarter q reads the step's
  // elements 32(q/2) + 16(q%2) + 8s .. + 7 for MFMA s, the K order of its
  // weights), then 2 kI kJ MFMAs.  The product is W x^T: acc[i][j][e] holds
  // token m0 + wm0 + 16i + lane%16 and output n0 + wn0 + 16j + 4*(lane/16) +
  // e, so a lane's four values are consecutive outputs of one token.
  const auto step = [&](int buf, const bf16x8 (&bf)[2][kJ]) {
    // Token group i's two fragments, issued kAhead groups before its MFMAs.
    const auto frag = [&](bf16x8* a, int i) {
#pragma unroll
      for (int s = 0; s < 2; ++s)
        a[s] = *reinterpret_cast<const bf16x8*>(
            &xs[buf][(wm0 + 16 * i + arow) * kLdsRow + 32 * (q >> 1) + 16 * (q & 1) + 8 * s]);
    };
    constexpr int kAhead = 3;  // token groups read ahead of their MFMAs
    bf16x8 a[kAhead + 1][2];
#pragma unroll
    for (int i = 0; i < kAhead; ++i) frag(a[i], i);
#pragma unroll
    for (int i = 0; i < kI; ++i) {
      if (i + kAhead < kI) frag(a[(i + kAhead) % (kAhead + 1)], i + kAhead);
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int j = 0; j < kJ; ++j)
          acc[i][j] =
              __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf[s][j], a[i % (kAhead + 1)][s], acc[i][j], 0, 0, 0);
    }
  };

  // The K loop runs whole pairs of steps with no conditions inside: a store
  // or load meant for a step past the last writes an LDS buffer no later
  // step reads, or re-reads the last step (clamped).  With one exit, the
  // loads in flight at the loop head are the same on every entry, so each
  // use waits only for its own loads, not for the ones issued after them.
  WStage<TYPE> WA, WB;
  bf16x8 BA[2][kJ], BB[2][kJ];
  // Each half of the loop dequantizes the next step's weights, runs the
  // current step and stages the next step's activations (all three from
  // loads issued two halves earlier), and only then issues its own loads,
  // two steps ahead.  The scheduling fences keep the loads at the end of the
  // half: then every use waits only for loads at least one half old, never
  // for the ones just issued.
  const auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
  if constexpr (F32X) {
    // Rings: activations of step k in XA (even k) / XB (odd) as loaded
    // (fp32), raw weights in WA / WB likewise, dequantized weights of step k
    // in BA / BB.
    f32x4 XA[kXPer][2], XB[kXPer][2];
    xloadf(XA, 0);
    xloadf(XB, 1);
    wload(WA, 0);
    wload(WB, 1);
    xstoref(XA, 0);
    xloadf(XA, 2);
    dequant(WA, BA);
    wload(WA, 2);
    __syncthreads();  // step 0's activations staged
    int k = 0;
    for (; k + 2 <= nk; k += 2) {
      dequant(WB, BB);
      step(0, BA);
      xstoref(XB, 1);
      fence();
      wload(WB, k + 3);
      xloadf(XB, k + 3);
      fence();
      __syncthreads();
      dequant(WA, BA);
      step(1, BB);
      xstoref(XA, 0);
      fence();
      wload(WA, k + 4);
      xloadf(XA, k + 4);
      fence();
      __syncthreads();
    }
    if (k < nk) step(0, BA);  // an odd step count's last step (staged in buffer 0)
  } else {
    XStage XA, XB;
    xload(XA, 0);
    xload(XB, 1);
    wload(WA, 0);
    wload(WB, 1);
    xstore(XA, 0);
    xload(XA, 2);
    dequant(WA, BA);
    wload(WA, 2);
    __syncthreads();  // step 0's activations staged
    int k = 0;
    for (; k + 2 <= nk; k += 2) {
      dequant(WB, BB);
      step(0, BA);
      xstore(XB, 1);
      fence();
      wload(WB, k + 3);
      xload(XB, k + 3);
      fence();
      __syncthreads();
      dequant(WA, BA);
      step(1, BB);
      xstore(XA, 0);
      fence();
      wload(WA, k + 4);
      xload(XA, k + 4);
      fence();
      __syncthreads();
    }
    if (k < nk) step(0, BA);  // an odd step count's last step (staged in buffer 0)
  }

  // Rows of y / part are 16-byte aligned when N is a multiple of 4: a lane's
  // four outputs then go out as one 16-byte store (the only case in which
  // n < N implies n + 3 < N, since n is a multiple of 4).
  const bool vec = (N & 3) == 0;
  const int mrow = m0 + wm0 + arow, ncol = n0 + wn0 + 4 * q;
  const auto store4 = [&](GMEM float* dst, const f32x4& v, int n) {
    if (vec) {
      *(GMEM f32x4*)dst = v;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (n + e < N) dst[e] = v[e];
    }
  };
  if (p.kchunks > 1) {
    // A K chunk: the partial tile as it is (gemm_reduce adds the rest).
    GMEM float* part = (GMEM float*)(p.part + static_cast<std::size_t>(kc) * M * N);
#pragma unroll
    for (int i = 0; i < kI; ++i) {
      const int m = mrow + 16 * i;
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int n = ncol + 16 * j;
        if (n < N) store4(part + static_cast<std::size_t>(m) * N + n, acc[i][j], n);
      }
    }
    return;
  }
  GMEM float* y = (GMEM float*)p.y;
  const GMEM float* bias = (const GMEM float*)p.bias;
  f32x4 add[kJ];
#pragma unroll
  for (int j = 0; j < kJ; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int n = ncol + 16 * j + e;
      add[j][e] = bias != nullptr && n < N ? bias[n] : 0.0f;
    }
  // With accumulate, a token row's old vectors are loaded (clamped to a row
  // and column inside y) before any is used, so their latencies overlap.
#pragma unroll
  for (int i = 0; i < kI; ++i) {
    const int m = mrow + 16 * i;
    f32x4 old[kJ];
    if (p.accumulate) {
      const std::size_t row = static_cast<std::size_t>(min(m, M - 1)) * N;
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int n = ncol + 16 * j;
        if (vec) {
          old[j] = *(const GMEM f32x4*)(y + row + min(n, N - 4));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) old[j][e] = y[row + min(n + e, N - 1)];
        }
      }
    }
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < kJ; ++j) {
      const int n = ncol + 16 * j;
      if (n >= N) continue;
      const f32x4 v = acc[i][j] + add[j];
      store4(y + static_cast<std::size_t>(m) * N + n, p.accumulate ? old[j] + v : v, n);
    }
  }
}

// y = (part_0 + part_1 + ... in chunk order) + bias (+ the old y with
// accumulate): the epilogue of a split product, one thread per output.
__global__ void __launch_bounds__(256) gemm_reduce(const float* __restrict__ part, int kchunks, int rows, int out,
                                                   const float* __restrict__ bias, float* __restrict__ y,
                                                   int accumulate) {
  const std::size_t n_all = static_cast<std::size_t>(rows) * out;
  const std::size_t stride = n_all;
  for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n_all;
       i += static_cast<std::size_t>(gridDim.x) * blockDim.x) {
    float v[16];
    const int kc = min(kchunks, 16);
#pragma unroll
    for (int c = 0; c < 16; ++c)
      if (c < kc) v[c] = part[c * stride + i];
    float sum = v[0];
#pragma unroll
    for (int c = 1; c < 16; ++c)
      if (c < kc) sum = sum + v[c];
    for (int c = 16; c < kchunks; ++c) sum = sum + part[c * stride + i];
    const float add = bias != nullptr ? bias[i % out] : 0.0f;
    const float val = sum + add;
    y[i] = accumulate ? y[i] + val : val;
  }
}

// gemm_reduce for four consecutive outputs per thread (16-byte loads and
// stores): out a multiple of 4 and part, y and bias 16-byte aligned.  The
// same sums in the same order.
__global__ void __launch_bounds__(256) gemm_reduce4(const float4* __restrict__ part, int kchunks, int rows, int out,
                                                    const float4* __restrict__ bias, float4* __restrict__ y,
                                                    int accumulate) {
  const std::size_t n4 = static_cast<std::size_t>(rows) * out / 4;
  const int out4 = out / 4;
  for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n4;
       i += static_cast<std::size_t>(gridDim.x) * blockDim.x) {
    float4 v[8];
    const int kc = min(kchunks, 8);
#pragma unroll
    for (int c = 0; c < 8; ++c)
      if (c < kc) v[c] = part[c * n4 + i];
    float4 sum = v[0];
#pragma unroll
    for (int c = 1; c < 8; ++c)
      if (c < kc) sum = make_float4(sum.x + v[c].x, sum.y + v[c].y, sum.z + v[c].z, sum.w + v[c].w);
    for (int c = 8; c < kchunks; ++c) {
      const float4 u = part[c * n4 + i];
      sum = make_float4(sum.x + u.x, sum.y + u.y, sum.z + u.z, sum.w + u.w);
    }
    const float4 add = bias != nullptr ? bias[i % out4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 val = make_float4(sum.x + add.x, sum.y + add.y, sum.z + add.z, sum.w + add.w);
    if (accumulate) {
      const float4 o = y[i];
      val = make_float4(o.x + val.x, o.y + val.y, o.z + val.z, o.w + val.w);
    }
    y[i] = val;
  }
}

// The reduce of one split product: the 16-byte form where the shapes and
// pointers allow it.
void launch_reduce(const float* part, int kchunks, int rows, int out, const float* bias, float* y, int accumulate,
                   hipStream_t s) {
  const auto a16 = [](const void* q) { return reinterpret_cast<std::uintptr_t>(q) % 16 == 0; };
  const std::size_t n = static_cast<std::size_t>(rows) * out;
  if (out % 4 == 0 && a16(part) && a16(y) && (bias == nullptr || a16(bias))) {
    const unsigned blocks = static_cast<unsigned>(std::min<std::size_t>(ceil_div(n / 4, 256), 8192));
    gemm_reduce4<<<blocks, 256, 0, s>>>(reinterpret_cast<const float4*>(part), kchunks, rows, out,
                                        reinterpret_cast<const float4*>(bias), reinterpret_cast<float4*>(y),
                                        accumulate);
    return;
  }
  const unsigned blocks = static_cast<unsigned>(std::min<std::size_t>(ceil_div(n, 256), 8192));
  gemm_reduce<<<blocks, 256, 0, s>>>(part, kchunks, rows, out, bias, y, accumulate);
}

}  // namespace

int gemm_kchunks(std::size_t in, std::size_t launch_tiles, std::size_t split_tiles) {
  // One workgroup of qgemm_mfma fills a CU (8 wavefronts of ~250 VGPRs,
  // two per SIMD), so a launch of fewer tiles than CUs leaves CUs idle: a long
  // product takes as many K chunks (of at least 8 K-steps) as the CUs the
  // launch's other tiles leave over allow.
  const std::size_t nk = ceil_div(in, static_cast<std::size_t>(kBK));
  if (nk <= kSplitMinSteps || launch_tiles >= kCus || split_tiles == 0 || split_tiles > launch_tiles) return 1;
  const std::size_t k = std::min((kCus - (launch_tiles - split_tiles)) / split_tiles, nk / 8);
  if (k < 2) return 1;
  // No empty chunk: as many chunks as ceil(nk / k) K-steps need.
  return static_cast<int>(ceil_div(nk, ceil_div(nk, k)));
}

int gemm_kpc(std::size_t in, int kchunks) {
  return static_cast<int>(ceil_div(ceil_div(in, static_cast<std::size_t>(kBK)), static_cast<std::size_t>(kchunks)));
}

std::size_t gemm_tiles(std::size_t rows, std::size_t out) { return ceil_div(rows, kBM) * ceil_div(out, kBN); }

std::size_t gemm_split_tiles(std::size_t rows, std::size_t in, std::size_t out) {
  return ceil_div(in, static_cast<std::size_t>(kBK)) > kSplitMinSteps ? gemm_tiles(rows, out) : 0;
}

std::size_t gemm_ldx(std::size_t in) { return (in + kBK - 1) / kBK * kBK; }

int plan_gemm_group(const GroupEntry* entries, std::size_t count, GemmPlan* plan) {
  *plan = GemmPlan{};
  // fp32 activations read directly when every product allows it.
  plan->f32x = true;
  for (std::size_t i = 0; i < count; ++i)
    if (entries[i].m != nullptr && entries[i].rows > 0 && entries[i].m->out > 0)
      plan->f32x = plan->f32x && entries[i].m->in % kBK == 0 && reinterpret_cast<std::uintptr_t>(entries[i].x) % 16 == 0;
  // Distinct activation matrices, each converted to bf16 once per launch.
  for (std::size_t i = 0; i < count; ++i) {
    const GroupEntry& e = entries[i];
    LLMI_REQUIRE(e.m != nullptr, "gemm: null weight");
    LLMI_REQUIRE(e.x != nullptr && e.y != nullptr, "gemm: null x or y");
    LLMI_REQUIRE(e.m->type != LLMI_TYPE_F32, "gemm: fp32 weights are not part of the MFMA GEMM");
    const DeviceMatrix& m = *e.m;
    LLMI_REQUIRE(m.in > 0 && m.in <= 0x7FFFFFFFu && m.out <= 0x7FFFFFFFu, "gemm: bad shape");
    LLMI_REQUIRE(e.rows <= 0x7FFFFFFFu, "gemm: too many rows");
    if (e.rows == 0 || m.out == 0) continue;
    bool seen = false;
    for (const GemmInput& in : plan->inputs)
      if (in.x == e.x) {
        LLMI_REQUIRE(in.rows == e.rows && in.in == m.in, "gemm: one x used with two shapes");
        seen = true;
      }
    if (!seen) {
      GemmInput in;
      in.x = e.x;
      in.rows = e.rows;
      in.in = m.in;
      in.ldx = gemm_ldx(m.in);
      in.offset = plan->scratch_elems;
      if (!plan->f32x) plan->scratch_elems += in.rows * in.ldx;
      plan->inputs.push_back(in);
    }
  }
  // Output tiles of each launch (one per weight type), for the K split.
  std::size_t launch_tiles[3] = {0, 0, 0}, split_tiles[3] = {0, 0, 0};
  for (std::size_t i = 0; i < count; ++i)
    if (entries[i].rows > 0 && entries[i].m->out > 0) {
      launch_tiles[entries[i].m->type] += gemm_tiles(entries[i].rows, entries[i].m->out);
      split_tiles[entries[i].m->type] += gemm_split_tiles(entries[i].rows, entries[i].m->in, entries[i].m->out);
    }
  for (int type : {LLMI_TYPE_Q8_0, LLMI_TYPE_Q4_0}) {
    GemmLaunch l;
    l.type = type;
    l.prob_offset = plan->probs.size();
    l.map_offset = plan->work_prob.size();
    std::size_t wg = 0, nprob = 0;
    for (std::size_t i = 0; i < count; ++i) {
      const GroupEntry& e = entries[i];
      const DeviceMatrix& m = *e.m;
      if (m.type != type || e.rows == 0 || m.out == 0) continue;
      GemmProblem p{};
      p.codes = m.codes;
      p.scales = m.scales;
      p.xf = e.x;
      p.bias = e.bias;
      p.y = e.y;
      p.rows = static_cast<int>(e.rows);
      p.in = static_cast<int>(m.in);
      p.ldx = static_cast<int>(gemm_ldx(m.in));
      p.out = static_cast<int>(m.out);
      p.nblk = static_cast<int>(m.nblk);
      p.ntiles = static_cast<int>(m.ntiles);
      p.mtiles = static_cast<int>(ceil_div(e.rows, kBM));
      p.accumulate = e.accumulate ? 1 : 0;
      p.kchunks = gemm_kchunks(m.in, launch_tiles[type], split_tiles[type]);
      p.kpc = gemm_kpc(m.in, p.kchunks);
      p.part = nullptr;
      plan->part_off.push_back(plan->part_floats);
      plan->part_floats += p.kchunks > 1 ? static_cast<std::size_t>(p.kchunks) * e.rows * m.out : 0;
      for (std::size_t j = 0; j < plan->inputs.size(); ++j)
        if (plan->inputs[j].x == e.x) p.input = static_cast<int>(j);
      const std::size_t ntiles_n = ceil_div(m.out, kBN);
      p.first_wg = static_cast<int>(wg);
      const std::size_t wgs = static_cast<std::size_t>(p.mtiles) * ntiles_n * static_cast<std::size_t>(p.kchunks);
      wg += wgs;
      LLMI_REQUIRE(wg <= 0x7FFFFFFFu, "gemm: too many workgroups");
      plan->work_prob.insert(plan->work_prob.end(), wgs, static_cast<std::uint32_t>(nprob));
      plan->probs.push_back(p);
      ++nprob;
    }
    if (nprob == 0) continue;
    l.total_wgs = static_cast<int>(wg);
    l.f32x = plan->f32x;
    plan->launches.push_back(l);
  }
  return LLMI_OK;
}

std::size_t gemm_scratch_bytes(const GemmPlan& plan) {
  const std::size_t xbytes = (plan.scratch_elems * sizeof(std::uint16_t) + 255) / 256 * 256;
  return xbytes + plan.part_floats * sizeof(float);
}

void bind_gemm_scratch(GemmPlan* plan, std::uint16_t* scratch) {
  const std::size_t xbytes = (plan->scratch_elems * sizeof(std::uint16_t) + 255) / 256 * 256;
  float* parts = reinterpret_cast<float*>(reinterpret_cast<std::uint8_t*>(scratch) + xbytes);
  for (std::size_t i = 0; i < plan->probs.size(); ++i) {
    GemmProblem& p = plan->probs[i];
    p.xb = scratch + plan->inputs[p.input].offset;
    p.part = p.kchunks > 1 ? parts + plan->part_off[i] : nullptr;
  }
}

int launch_gemm_reduces(const GemmPlan& plan, hipStream_t s) {
  for (const GemmProblem& p : plan.probs) {
    if (p.kchunks <= 1) continue;
    launch_reduce(p.part, p.kchunks, p.rows, p.out, p.bias, p.y, p.accumulate, s);
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int launch_gemm_inputs(const GemmPlan& plan, std::uint16_t* scratch, hipStream_t s) {
  if (plan.f32x) return LLMI_OK;  // the GEMM reads the fp32 activations itself
  // The inputs in batches of kConvBatch per launch, each batch's octets
  // counted in 32 bits (a batch is cut short before it would overflow).
  std::size_t i0 = 0;
  while (i0 < plan.inputs.size()) {
    ConvBatch c{};
    std::size_t o = 0;
    int n = 0;
    while (n < kConvBatch && i0 + static_cast<std::size_t>(n) < plan.inputs.size()) {
      const GemmInput& in = plan.inputs[i0 + static_cast<std::size_t>(n)];
      const std::size_t octets = in.rows * (in.ldx / 8);
      LLMI_REQUIRE(octets < 0x80000000u, "gemm: activation matrix too large");
      if (o + octets > 0xFFFFFFFFu) break;
      o += octets;
      c.x[n] = in.x;
      c.xb[n] = scratch + in.offset;
      c.in[n] = static_cast<int>(in.in);
      c.ldx[n] = static_cast<int>(in.ldx);
      c.oend[n] = static_cast<unsigned>(o);
      c.vec[n] = in.in % 4 == 0 && reinterpret_cast<std::uintptr_t>(in.x) % 16 == 0 ? 1 : 0;
      ++n;
    }
    c.n = n;
    i0 += static_cast<std::size_t>(n);
    if (o == 0) continue;
    const unsigned blocks = static_cast<unsigned>(std::min<std::size_t>((o + 255) / 256, 16384));
    x_to_bf16_batch<<<blocks, 256, 0, s>>>(c);
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

// ------------------------------------------------- allocation-free launch
// llmi_hip_matmul_mfma_noalloc_dev keeps the bf16 copy of x in this
// file-scope device array instead of a buffer the library allocates: every
// GPU the library runs on holds its own copy until the process ends.  In
// host code `scratch` is only a symbol; its device address (per GPU) comes
// from hipGetSymbolAddress at llmi_hip_init and is what kernels are given.
// Nothing in it needs clearing: x_to_bf16 writes every element a launch
// reads (rows x ldx, the padding columns as zeros; the GEMM clamps token
// rows to rows - 1).  Calls that overlap on one GPU share it and race.
constexpr std::size_t kNoAllocBytes = LLMI_MFMA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) std::uint16_t scratch[kNoAllocBytes / sizeof(std::uint16_t)];

namespace {
constexpr int kMaxDevices = 64;
std::uint16_t* g_scratch_dev[kMaxDevices] = {};  // scratch's address on each GPU
}  // namespace

int noalloc_setup(int device) {
  LLMI_REQUIRE(device >= 0 && device < kMaxDevices, "llmi_hip_init: device ordinal above the library's limit");
  if (g_scratch_dev[device] != nullptr) return LLMI_OK;
  void* ptr = nullptr;
  LLMI_TRY_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
  g_scratch_dev[device] = static_cast<std::uint16_t*>(ptr);
  return LLMI_OK;
}

int launch_gemm_noalloc(int device, const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias,
                        float* y, hipStream_t s) {
  LLMI_REQUIRE(m.type == LLMI_TYPE_Q8_0 || m.type == LLMI_TYPE_Q4_0,
               "matmul_mfma_noalloc: weight must be Q8_0 or Q4_0");
  LLMI_REQUIRE(m.in > 0 && m.in <= 0x7FFFFFFFu && m.out <= 0x7FFFFFFFu, "matmul_mfma_noalloc: bad shape");
  if (rows == 0 || m.out == 0) return LLMI_OK;
  LLMI_REQUIRE(x != nullptr && y != nullptr, "matmul_mfma_noalloc: null x or y");
  const std::size_t ldx = gemm_ldx(m.in);
  // The bf16 copy of x (rounded up to 256 bytes), then a split product's
  // fp32 partials: the layout gemm_scratch_bytes / bind_gemm_scratch use.
  LLMI_REQUIRE(rows <= 0x7FFFFFFFu && rows <= kNoAllocBytes / (2 * ldx),
               "matmul_mfma_noalloc: the product exceeds the " + std::to_string(kNoAllocBytes) + "-byte scratch");
  const std::size_t xbytes = (rows * ldx * sizeof(std::uint16_t) + 255) / 256 * 256;
  const std::size_t tiles = gemm_tiles(rows, m.out);
  const int kchunks = gemm_kchunks(m.in, tiles, tiles);
  const std::size_t pbytes = kchunks > 1 ? static_cast<std::size_t>(kchunks) * rows * m.out * sizeof(float) : 0;
  LLMI_REQUIRE(xbytes + pbytes <= kNoAllocBytes,
               "matmul_mfma_noalloc: the product exceeds the " + std::to_string(kNoAllocBytes) + "-byte scratch");
  LLMI_REQUIRE(device >= 0 && device < kMaxDevices && g_scratch_dev[device] != nullptr,
               "matmul_mfma_noalloc: scratch not set up on this device");
  std::uint16_t* xb = g_scratch_dev[device];
  // The single-product launch of launch_gemm_single, planned on the stack.
  GemmProblem p{};
  p.codes = m.codes;
  p.scales = m.scales;
  p.xb = xb;
  p.bias = bias;
  p.y = y;
  p.rows = static_cast<int>(rows);
  p.in = static_cast<int>(m.in);
  p.ldx = static_cast<int>(ldx);
  p.out = static_cast<int>(m.out);
  p.nblk = static_cast<int>(m.nblk);
  p.ntiles = static_cast<int>(m.ntiles);
  p.mtiles = static_cast<int>(ceil_div(rows, kBM));
  p.first_wg = 0;
  p.input = 0;
  p.accumulate = 0;
  p.kchunks = kchunks;
  p.kpc = gemm_kpc(m.in, kchunks);
  p.part = p.kchunks > 1 ? reinterpret_cast<float*>(reinterpret_cast<std::uint8_t*>(xb) + xbytes) : nullptr;
  GemmLaunch l;
  l.type = m.type;
  l.total_wgs = static_cast<int>(static_cast<std::size_t>(p.mtiles) * ceil_div(m.out, kBN) *
                                 static_cast<std::size_t>(p.kchunks));
  // x's bf16 copy: one input of the batched conversion, planned on the stack.
  ConvBatch c{};
  const std::size_t octets = rows * (ldx / 8);
  LLMI_REQUIRE(octets < 0x80000000u, "matmul_mfma_noalloc: activation matrix too large");
  c.n = 1;
  c.x[0] = x;
  c.xb[0] = xb;
  c.in[0] = static_cast<int>(m.in);
  c.ldx[0] = static_cast<int>(ldx);
  c.oend[0] = static_cast<unsigned>(octets);
  c.vec[0] = m.in % 4 == 0 && reinterpret_cast<std::uintptr_t>(x) % 16 == 0 ? 1 : 0;
  x_to_bf16_batch<<<static_cast<unsigned>(std::min<std::size_t>(ceil_div(octets, 256), 16384)), 256, 0, s>>>(c);
  LLMI_TRY_HIP(hipGetLastError());
  if (int rc = launch_gemm(nullptr, nullptr, l, s, &p)) return rc;
  if (p.kchunks > 1) {
    launch_reduce(p.part, p.kchunks, p.rows, p.out, p.bias, p.y, p.accumulate, s);
    LLMI_TRY_HIP(hipGetLastError());
  }
  return LLMI_OK;
}

int launch_gemm(const GemmProblem* probs_dev, const std::uint32_t* map_dev, const GemmLaunch& l, hipStream_t s,
                const GemmProblem* one, int nfew) {
  if (l.total_wgs == 0) return LLMI_OK;
  LLMI_REQUIRE(one == nullptr || (nfew >= 1 && nfew <= kGemmFew), "gemm: 1..3 products by value");
  const GemmProblem* probs = one != nullptr ? nullptr : probs_dev + l.prob_offset;
  const std::uint32_t* map = one != nullptr ? nullptr : map_dev + l.map_offset;
  GemmFew few{};
  if (one != nullptr) {
    for (int i = 0; i < nfew; ++i) few.p[i] = one[i];
    few.count = nfew;
  }
  if (l.f32x) {
    if (l.type == LLMI_TYPE_Q8_0)
      qgemm_mfma<LLMI_TYPE_Q8_0, true><<<l.total_wgs, kGemmThreads, 0, s>>>(probs, map, l.total_wgs, few);
    else
      qgemm_mfma<LLMI_TYPE_Q4_0, true><<<l.total_wgs, kGemmThreads, 0, s>>>(probs, map, l.total_wgs, few);
  } else if (l.type == LLMI_TYPE_Q8_0) {
    qgemm_mfma<LLMI_TYPE_Q8_0><<<l.total_wgs, kGemmThreads, 0, s>>>(probs, map, l.total_wgs, few);
  } else {
    qgemm_mfma<LLMI_TYPE_Q4_0><<<l.total_wgs, kGemmThreads, 0, s>>>(probs, map, l.total_wgs, few);
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

}  // namespace llmi_hip
