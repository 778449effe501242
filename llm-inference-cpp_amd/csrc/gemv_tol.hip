// Tolerance-mode batch 1..8 Q4_0 product on the matrix cores (gfx950).
//
// Reference: src/model/quant.cpp:119-153, y[o] = sum_b scale_b * sum_i
// x[i] * code[i] (+ bias).  The exact kernels (gemv.hip) reproduce the
// reference's fp32 chains bit for bit, 32 dependent fused multiply-adds per
// row and block; this path computes the same sums in another order and meets
// the tolerance of the fp32-accumulate contract instead,
// |y - y_ref| <= 1e-4 * max|y_ref| (measured ~1e-6).
//
// Arithmetic, per 32-weight block and row, with c = n - 8 (n the stored
// nibble):
//   B (codes)        nibble n in bits 3..6 of a bf16 1.0 is exactly 1 + n/16
//                    (a shift and one v_and_or_b32 per two codes);
//   A (activations)  x split into two bf16 parts, x' = hi + lo (hi = bf16(x),
//                    lo = bf16(x - hi): 16 significant bits);
//   D                v_mfma_f32_16x16x32_bf16: sum_i x'_i (1 + n_i/16) in
//                    fp32, so T = sum_i x'_i c_i = 16 D - 24 sx with
//                    sx = sum_i x'_i of the block (computed once per input).
// Then acc = fma(T, scale, acc) over a wavefront's blocks, and the
// wavefronts' partial sums of a tile are added in wavefront order, so the
// result does not depend on timing.
//
// Operand layout.  Lane l holds tile row l's 16 code bytes (the tiled layout:
// one 16-byte load), row 16g + n with g = l/16, n = l%16.  For code word q
// (elements 8q..8q+7) the lane's four decoded registers are the MFMA's B
// operand B[k = 8g + e][n]: k-slice g carries row 16g + n.  A[m][k] is
// nonzero only for k in slice m/4, so D[m][n] is word q's dot product of row
// 16(m/4) + n, and D[m][n] sits at lane 16(m/4) + n, register m%4: every lane
// receives its own row's sums.  Of the four m = 4g + j of a row group, j&1 is
// the activation part (hi, lo) and j/2 picks one of two input rows, so one
// MFMA set covers two input rows; the four words accumulate in D (its C
// operand), four MFMAs per block and set.  Inside a word, register v of B
// holds nibbles v and v + 4, so A holds x in the order 0,4,1,5,2,6,3,7.
//
// Each wavefront splits the activations of its own blocks into its own LDS
// region (two elements per lane, the block sums by DPP rotations within rows
// of 16 lanes), so no workgroup barrier precedes the products; the loads of
// the activations are issued before the code loads, so waiting for them does
// not wait for HBM.  Lanes outside the active pattern read zero slots.
#include <algorithm>
#include <memory>
#include <vector>

#include "common.hpp"

namespace llmi_hip {
namespace {

#define TGMEM __attribute__((address_space(1)))
typedef unsigned int tu32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 tbf16x8 __attribute__((ext_vector_type(8)));
typedef float tf32x4 __attribute__((ext_vector_type(4)));

constexpr int kSlotsPerBlock = 8;  // 16-byte slots per row and block: 4 words x 2 parts
constexpr int kTolChunk = 4;       // blocks whose code loads are in flight per wavefront
constexpr int kZeroSlots = kTolChunk * kSlotsPerBlock;  // zero A operands for inactive lanes

struct TolProblem {
  const std::uint8_t* codes;
  const float* scales;
  const float* bias;
  float* y;
  const float* x;
  int in, nblk, out, rows, ntiles, bpw, accumulate, first_wg;
};

__device__ __forceinline__ std::uint32_t bf16_bits_rne(float f) {
  // Round to nearest even; the inputs are finite (inf/NaN pass through with
  // their payload's top bits, which the caller's check excludes anyway).
  const std::uint32_t u = __builtin_bit_cast(std::uint32_t, f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_value(std::uint32_t b) { return __builtin_bit_cast(float, b << 16); }

// v of lane (i + n) % 16 of this lane's row of 16 (DPP row_ror:n).
template <int N>
__device__ __forceinline__ float row_ror_n(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x120 + N, 0xF, 0xF, false));
}
__device__ __forceinline__ float row_ror(float v, int n) {
  return n == 8 ? row_ror_n<8>(v) : n == 4 ? row_ror_n<4>(v) : n == 2 ? row_ror_n<2>(v) : row_ror_n<1>(v);
}

// Four codes of word w as bf16 pairs 1 + n/16: register v holds nibbles v
// and v + 4 (the nibble moved to bits 3..6 of each half by a shift, then one
// v_and_or_b32, whose VOP3 form takes no literal: the constants sit in VGPRs).
struct TolMagic {
  std::uint32_t mask, one;
};
__device__ __forceinline__ TolMagic tol_magic() {
  TolMagic k{0x00780078u, 0x3F803F80u};
  asm("" : "+v"(k.mask), "+v"(k.one));
  return k;
}
__device__ __forceinline__ std::uint32_t and_or(std::uint32_t a, std::uint32_t mask, std::uint32_t bits) {
  std::uint32_t d;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(mask), "v"(bits));
  return d;
}
__device__ __forceinline__ tbf16x8 decode_word(std::uint32_t w, const TolMagic& k) {
  const tu32x4 r{and_or(w << 3, k.mask, k.one), and_or(w >> 1, k.mask, k.one), and_or(w >> 5, k.mask, k.one),
                 and_or(w >> 9, k.mask, k.one)};
  return __builtin_bit_cast(tbf16x8, r);
}

// One 64-row tile of one product for input rows [r0, r0 + nr), nr <= R.
// The workgroup's wavefronts split the tile's blocks, bpw each; each
// wavefront splits the activations of its own blocks into its own LDS region
// (no workgroup barrier before the products; LDS operations of one wavefront
// complete in order).  Region of wavefront w: kZeroSlots zero slots (the A
// operand of inactive lanes; every wavefront writes the same zeros), then
// [row][block][word][part] 16-byte slots, then 24 * sx per row and block.
template <int R>
__global__ void __launch_bounds__(1024) qgemv_tol(const TolProblem* __restrict__ probs,
                                                  const std::uint32_t* __restrict__ wg_prob, TolProblem single) {
  constexpr int kSets = (R + 1) / 2;
  extern __shared__ tu32x4 lds[];
  const int wg = blockIdx.x;
  TolProblem p = single;
  if (probs != nullptr) p = probs[__builtin_amdgcn_readfirstlane(static_cast<int>(wg_prob[wg]))];
  const int local = wg - p.first_wg;
  const int tile = local % p.ntiles;
  const int r0 = (local / p.ntiles) * R;
  const int nr = min(R, p.rows - r0);
  const int nblk = p.nblk, bpw = p.bpw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int nwaves = blockDim.x >> 6;
  const int b_begin = wave * bpw, b_end = min(nblk, b_begin + bpw);
  const int nwb = max(0, b_end - b_begin);

  const std::size_t tbase = static_cast<std::size_t>(tile) * nblk * kTileRows + lane;
  const TGMEM tu32x4* codes = (const TGMEM tu32x4*)p.codes + tbase;
  const TGMEM float* scales = (const TGMEM float*)p.scales + tbase;

  // This wavefront's LDS region.
  const int region_slots = kZeroSlots + R * bpw * kSlotsPerBlock;
  tu32x4* wl = lds + static_cast<std::size_t>(wave) * region_slots;
  float* wsx = reinterpret_cast<float*>(lds + static_cast<std::size_t>(nwaves) * region_slots) + wave * R * bpw;

  // Staging items: one pair of elements (v, v + 4) of word q of one of the
  // wavefront's blocks of one row, 16 per row-block; lane l takes items l,
  // l + 64, ...  The first round's activations are loaded before the first
  // code loads, so that waiting for them (loads complete in order) does not
  // wait for the codes.
  const int items = nr * nwb * 16;
  const auto load_pair = [&](int it, float* x2) {
    const int c = min(it, max(items - 1, 0));
    const int pr = c & 15, rb = c >> 4;
    const int rr = nwb > 0 ? rb / nwb : 0, jb = rb - rr * nwb;
    const int e0 = (b_begin + jb) * kBlock + 8 * (pr >> 2) + (pr & 3);
    const TGMEM float* xr = (const TGMEM float*)p.x + static_cast<std::size_t>(r0 + rr) * p.in;
    const bool live = it < items;
    x2[0] = live && e0 < p.in ? xr[e0] : 0.0f;
    x2[1] = live && e0 + 4 < p.in ? xr[e0 + 4] : 0.0f;
  };
  // Staging rounds of 64 items, loaded kStage at a time (all loads of a
  // batch issued before the first is used).
  constexpr int kStage = R < 2 ? 2 : R;
  const int rounds = (items + 63) >> 6;
  float xs[kStage][2];
#pragma unroll
  for (int k = 0; k < kStage; ++k)
    if (k < rounds) load_pair(lane + 64 * k, xs[k]);

  // The first chunk's code loads, unconditional (blocks past the wavefront's
  // range re-read a block of the tile; unused).
  tu32x4 cur_c[kTolChunk];
  float cur_s[kTolChunk];
#pragma unroll
  for (int j = 0; j < kTolChunk; ++j) {
    const std::size_t bc = static_cast<std::size_t>(max(0, min(b_begin + j, nblk - 1)));
    cur_c[j] = __builtin_nontemporal_load(codes + bc * kTileRows);
    cur_s[j] = __builtin_nontemporal_load(scales + bc * kTileRows);
  }

  if (lane < kZeroSlots) wl[lane] = tu32x4{0u, 0u, 0u, 0u};
  for (int r = 0; r < rounds; r += kStage) {
    if (r > 0) {
#pragma unroll
      for (int k = 0; k < kStage; ++k)
        if (r + k < rounds) load_pair(lane + 64 * (r + k), xs[k]);
    }
#pragma unroll
    for (int k = 0; k < kStage; ++k) {
      if (r + k >= rounds) break;
      const int it = lane + 64 * (r + k);
      const std::uint32_t h0 = bf16_bits_rne(xs[k][0]), h1 = bf16_bits_rne(xs[k][1]);
      const std::uint32_t l0 = bf16_bits_rne(xs[k][0] - bf16_value(h0)), l1 = bf16_bits_rne(xs[k][1] - bf16_value(h1));
      float sum = (bf16_value(h0) + bf16_value(l0)) + (bf16_value(h1) + bf16_value(l1));
      const int pr = it & 15, rb = it >> 4;
      if (it < items) {
        std::uint32_t* slot = reinterpret_cast<std::uint32_t*>(wl + kZeroSlots + rb * kSlotsPerBlock + 2 * (pr >> 2));
        slot[pr & 3] = h0 | (h1 << 16);
        slot[4 + (pr & 3)] = l0 | (l1 << 16);
      }
      // The row-block's 16 pair sums (one row of 16 lanes) by rotations within
      // the row; lane 0 of the row writes its total (a fixed order).
      sum += row_ror(sum, 8);
      sum += row_ror(sum, 4);
      sum += row_ror(sum, 2);
      sum += row_ror(sum, 1);
      if (it < items && pr == 0) wsx[rb] = 24.0f * sum;
    }
  }

  // This lane's A operand: active when its k-slice matches its m's row group;
  // part s = m & 1, input row 2t + ((m >> 1) & 1) in set t.  Slot of the
  // wavefront's block jb, word q: base[t] + jb * step[t] + 2q (inactive
  // lanes: step 0, base 0, so every slot they read is a zero slot).
  const int m = lane & 15;
  const bool active = (m >> 2) == (lane >> 4);
  const int part = m & 1, half = (m >> 1) & 1;
  int base[kSets], step[kSets];
#pragma unroll
  for (int t = 0; t < kSets; ++t) {
    const int rr = 2 * t + half;
    const bool on = active && rr < nr;
    base[t] = on ? kZeroSlots + rr * nwb * kSlotsPerBlock + part : 0;
    step[t] = on ? kSlotsPerBlock : 0;
  }
  const TolMagic mk = tol_magic();

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;

  for (int b = b_begin; b < b_end; b += kTolChunk) {
    tu32x4 nxt_c[kTolChunk];
    float nxt_s[kTolChunk];
#pragma unroll
    for (int j = 0; j < kTolChunk; ++j)
      if (b + kTolChunk + j < b_end) {
        nxt_c[j] = __builtin_nontemporal_load(codes + static_cast<std::size_t>(b + kTolChunk + j) * kTileRows);
        nxt_s[j] = __builtin_nontemporal_load(scales + static_cast<std::size_t>(b + kTolChunk + j) * kTileRows);
      }
    const int jb0 = b - b_begin;
    const tu32x4* arow[kSets];
#pragma unroll
    for (int t = 0; t < kSets; ++t) arow[t] = wl + base[t] + jb0 * step[t];
#pragma unroll
    for (int j = 0; j < kTolChunk; ++j) {
      if (b + j < b_end) {
        tf32x4 d[kSets];
#pragma unroll
        for (int t = 0; t < kSets; ++t) d[t] = tf32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const tbf16x8 bq = decode_word(cur_c[j][q], mk);
#pragma unroll
          for (int t = 0; t < kSets; ++t) {
            // Inactive lanes: step 0, so j * kSlotsPerBlock + 2q < kZeroSlots.
            const tbf16x8 aq = __builtin_bit_cast(tbf16x8, arow[t][j * kSlotsPerBlock + 2 * q]);
            d[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aq, bq, d[t], 0, 0, 0);
          }
        }
#pragma unroll
        for (int t = 0; t < kSets; ++t)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int rr = 2 * t + h;
            if (rr < R && rr < nr) {
              const float blk = __builtin_fmaf(16.0f, d[t][2 * h] + d[t][2 * h + 1], -wsx[rr * nwb + jb0 + j]);
              acc[rr] = __builtin_fmaf(blk, cur_s[j], acc[rr]);
            }
          }
      }
    }
#pragma unroll
    for (int j = 0; j < kTolChunk; ++j) {
      cur_c[j] = nxt_c[j];
      cur_s[j] = nxt_s[j];
    }
  }

  // The wavefronts' partial sums of each row, added in wavefront order.
  float* red = wsx - wave * R * bpw + nwaves * R * bpw;
  __syncthreads();
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (r < nr) red[(wave * R + r) * kTileRows + lane] = acc[r];
  __syncthreads();
  const std::size_t o = static_cast<std::size_t>(tile) * kTileRows + lane;
  for (int r = wave; r < nr; r += nwaves) {
    float v = red[r * kTileRows + lane];
    for (int w2 = 1; w2 < nwaves; ++w2) v += red[(w2 * R + r) * kTileRows + lane];
    if (o < static_cast<std::size_t>(p.out)) {
      TGMEM float* y = (TGMEM float*)p.y + static_cast<std::size_t>(r0 + r) * p.out;
      const float bias = p.bias != nullptr ? p.bias[o] : 0.0f;
      y[o] = p.accumulate ? y[o] + (v + bias) : v + bias;
    }
  }
}

// ------------------------------------------------------------ planning

constexpr std::size_t kTolLdsBudget = 32 * 1024;

// Wavefronts per tile: about kTolChunk blocks each, at most 16.
int tol_waves(std::size_t nblk) {
  return static_cast<int>(std::clamp<std::size_t>(ceil_div(nblk, kTolChunk), 1, 16));
}
// LDS of one workgroup: per wavefront its zero slots, split activations and
// block sums (R rows x bpw blocks), then the reduction area.
std::size_t tol_lds(int waves, int R, int bpw) {
  return static_cast<std::size_t>(waves) *
             ((kZeroSlots + static_cast<std::size_t>(R) * bpw * kSlotsPerBlock) * sizeof(tu32x4) +
              static_cast<std::size_t>(R) * bpw * sizeof(float)) +
         static_cast<std::size_t>(waves) * R * kTileRows * sizeof(float);
}
// Row chunk R (1, 2, 4, 8): the smallest covering `rows`, halved while the
// staged activations exceed the budget.
int tol_chunk(std::size_t rows, std::size_t nblk) {
  int r = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8;
  while (r > 1 && std::min<std::size_t>(rows, r) * nblk * kSlotsPerBlock * sizeof(tu32x4) > kTolLdsBudget) r /= 2;
  return r;
}

struct TolLaunch {
  int rchunk = 1, waves = 1, total_wgs = 0;
  std::size_t lds = 0, prob_offset = 0, map_offset = 0;
};

struct TolPlan {
  std::vector<TolProblem> probs;
  std::vector<std::uint32_t> wg_prob;
  std::vector<TolLaunch> launches;
};

int plan_tol(const GroupEntry* entries, std::size_t count, TolPlan* plan) {
  *plan = TolPlan{};
  for (std::size_t i = 0; i < count; ++i) {
    const GroupEntry& e = entries[i];
    LLMI_REQUIRE(e.m != nullptr, "tolerance matmul: null weight");
    LLMI_REQUIRE(e.x != nullptr && e.y != nullptr, "tolerance matmul: null x or y");
    LLMI_REQUIRE(e.m->type == LLMI_TYPE_Q4_0, "tolerance matmul: Q4_0 weights only");
    LLMI_REQUIRE(e.rows >= 1 && e.rows <= 8, "tolerance matmul: each product takes 1..8 input rows");
    const DeviceMatrix& m = *e.m;
    LLMI_REQUIRE(m.in > 0 && m.in <= (1u << 20) && m.out <= 0x7FFFFFFFu, "tolerance matmul: bad shape");
    LLMI_REQUIRE(tol_lds(16, 1, static_cast<int>(ceil_div(m.nblk, 16))) <= max_lds_per_block(),
                 "tolerance matmul: rows too long");
  }
  for (int R : {1, 2, 4, 8}) {
    std::vector<TolProblem> probs;
    int waves = 1;
    std::size_t biggest = 0, lds = 0;
    for (std::size_t i = 0; i < count; ++i) {
      const GroupEntry& e = entries[i];
      const DeviceMatrix& m = *e.m;
      if (m.out == 0 || tol_chunk(e.rows, m.nblk) != R) continue;
      TolProblem p{};
      p.codes = m.codes;
      p.scales = m.scales;
      p.bias = e.bias;
      p.y = e.y;
      p.x = e.x;
      p.in = static_cast<int>(m.in);
      p.nblk = static_cast<int>(m.nblk);
      p.out = static_cast<int>(m.out);
      p.rows = static_cast<int>(e.rows);
      p.ntiles = static_cast<int>(m.ntiles);
      p.accumulate = e.accumulate ? 1 : 0;
      probs.push_back(p);
      const std::size_t bytes = m.code_bytes + m.scale_bytes;
      if (bytes > biggest) {
        biggest = bytes;
        waves = tol_waves(m.nblk);
      }
    }
    if (probs.empty()) continue;
    // Longest workgroups first, as in the exact grouped launch.
    std::stable_sort(probs.begin(), probs.end(), [](const TolProblem& a, const TolProblem& b) { return a.nblk > b.nblk; });
    TolLaunch l;
    l.rchunk = R;
    l.waves = waves;
    l.prob_offset = plan->probs.size();
    l.map_offset = plan->wg_prob.size();
    std::size_t wg = 0;
    for (std::size_t j = 0; j < probs.size(); ++j) {
      TolProblem& p = probs[j];
      p.bpw = static_cast<int>(ceil_div(p.nblk, waves));
      p.first_wg = static_cast<int>(wg);
      const std::size_t wgs = static_cast<std::size_t>(p.ntiles) * ceil_div(p.rows, R);
      wg += wgs;
      LLMI_REQUIRE(wg <= 0x7FFFFFFFu, "tolerance matmul: too many workgroups");
      lds = std::max(lds, tol_lds(waves, R, p.bpw));
      plan->wg_prob.insert(plan->wg_prob.end(), wgs, static_cast<std::uint32_t>(j));
    }
    LLMI_REQUIRE(lds <= max_lds_per_block(), "tolerance matmul: a product needs more LDS than one workgroup may use");
    l.lds = lds;
    l.total_wgs = static_cast<int>(wg);
    plan->probs.insert(plan->probs.end(), probs.begin(), probs.end());
    plan->launches.push_back(l);
  }
  return LLMI_OK;
}

int launch_tol_kernel(const TolLaunch& l, const TolProblem* probs, const std::uint32_t* map, const TolProblem& single,
                      hipStream_t s) {
  if (l.total_wgs == 0) return LLMI_OK;
  const dim3 grid(static_cast<unsigned>(l.total_wgs)), block(static_cast<unsigned>(l.waves * 64));
  switch (l.rchunk) {
    case 1: qgemv_tol<1><<<grid, block, l.lds, s>>>(probs, map, single); break;
    case 2: qgemv_tol<2><<<grid, block, l.lds, s>>>(probs, map, single); break;
    case 4: qgemv_tol<4><<<grid, block, l.lds, s>>>(probs, map, single); break;
    default: qgemv_tol<8><<<grid, block, l.lds, s>>>(probs, map, single); break;
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

}  // namespace
}  // namespace llmi_hip

using namespace llmi_hip;

// A planned tolerance-mode group on the device: the problem table and the
// workgroup map.
struct llmi_hip_tol_group {
  void* table = nullptr;
  const TolProblem* probs = nullptr;
  const std::uint32_t* map = nullptr;
  TolPlan plan;
  ~llmi_hip_tol_group() {
    if (table != nullptr) (void)hipFree(table);
  }
};

namespace {

int tol_entries(const llmi_hip_weight* const* w, const float* const* x, const size_t* rows, const float* const* bias,
                float* const* y, size_t count, std::vector<GroupEntry>* entries) {
  LLMI_REQUIRE(count == 0 || (w != nullptr && x != nullptr && y != nullptr), "tolerance matmul: null array");
  entries->resize(count);
  for (size_t i = 0; i < count; ++i) {
    LLMI_REQUIRE(w[i] != nullptr, "tolerance matmul: null weight");
    (*entries)[i] = GroupEntry{&w[i]->m, x[i], bias != nullptr ? bias[i] : nullptr, y[i], rows != nullptr ? rows[i] : 1, false};
  }
  return LLMI_OK;
}

}  // namespace

extern "C" {

int llmi_hip_tol_group_create(const llmi_hip_weight* const* w, const float* const* x_dev, const size_t* rows,
                              const float* const* bias_dev, float* const* y_dev, size_t count,
                              llmi_hip_tol_group** out) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(out != nullptr, "tolerance matmul: null output handle");
  *out = nullptr;
  std::vector<GroupEntry> entries;
  if (int rc = tol_entries(w, x_dev, rows, bias_dev, y_dev, count, &entries)) return rc;
  auto g = std::make_unique<llmi_hip_tol_group>();
  if (int rc = plan_tol(entries.data(), count, &g->plan)) return rc;
  const std::size_t pb = g->plan.probs.size() * sizeof(TolProblem);
  const std::size_t mb = g->plan.wg_prob.size() * sizeof(std::uint32_t);
  if (pb + mb > 0) {
    LLMI_TRY_HIP(hipMalloc(&g->table, pb + mb));
    auto* base = static_cast<std::uint8_t*>(g->table);
    if (pb > 0) LLMI_TRY_HIP(hipMemcpy(base, g->plan.probs.data(), pb, hipMemcpyHostToDevice));
    if (mb > 0) LLMI_TRY_HIP(hipMemcpy(base + pb, g->plan.wg_prob.data(), mb, hipMemcpyHostToDevice));
    g->probs = reinterpret_cast<const TolProblem*>(base);
    g->map = reinterpret_cast<const std::uint32_t*>(base + pb);
  }
  *out = g.release();
  return LLMI_OK;
}

int llmi_hip_tol_group_launch(const llmi_hip_tol_group* g, void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(g != nullptr, "tolerance matmul: null group");
  for (const TolLaunch& l : g->plan.launches)
    if (int rc = launch_tol_kernel(l, g->probs + l.prob_offset, g->map + l.map_offset, TolProblem{}, pick(stream)))
      return rc;
  return LLMI_OK;
}

void llmi_hip_tol_group_free(llmi_hip_tol_group* g) { delete g; }

int llmi_hip_matmul_tol_dev(const llmi_hip_weight* weight, const float* x_dev, size_t rows, const float* bias_dev,
                            float* y_dev, void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(weight != nullptr, "tolerance matmul: null weight");
  const GroupEntry e{&weight->m, x_dev, bias_dev, y_dev, rows, false};
  TolPlan plan;
  if (int rc = plan_tol(&e, 1, &plan)) return rc;
  if (plan.launches.empty()) return LLMI_OK;
  // One product: its descriptor travels as a kernel argument.
  TolProblem p = plan.probs[0];
  p.first_wg = 0;
  return launch_tol_kernel(plan.launches[0], nullptr, nullptr, p, pick(stream));
}

}  // extern "C"
