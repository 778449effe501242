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
//   D                the MFMA: sum_i x'_i (1 + n_i/16) in fp32, so
//                    T = sum_i x'_i c_i = 16 D - 24 sx with sx = sum_i x'_i
//                    of the block (computed with the split).
// Then acc = fma(T, scale, acc) over a wavefront's blocks, and the
// wavefronts' partial sums of a tile are added in wavefront order, so the
// result does not depend on timing.
//
// Operand layout.  Lane l holds tile row l's 16 code bytes (the tiled layout:
// one 16-byte load).  For code word q (elements 8q..8q+7) the lane's four
// decoded registers are the MFMA's B operand at the lane's own k-slice and
// column, so the slice carries the lane's row; A[m][k] is nonzero only for k
// in the slice of m's row group, so every lane receives its own row's sums
// (lane maps: the MFMA-shape notes before a_role).  The four words
// accumulate in D (its C operand).  Inside a word, register v of B holds
// nibbles v and v + 4, so A holds x in the order 0,4,1,5,2,6,3,7.
//
// Kernels: qgemv_tol_small (batches 1-2, v_mfma_f32_16x16x32_bf16) -- each
// wavefront splits the activations of its own blocks into its own LDS region
// (two elements per lane, the block sums by DPP rotations within rows of 16
// lanes), so no workgroup barrier precedes the products, and loads the
// activations before the codes, so waiting for them does not wait for HBM;
// qgemv_tol_wide (batches 3-8, v_mfma_f32_32x32x16_bf16) -- tol_split splits
// each input once per launch and each wavefront copies one block at a time
// into its LDS region.  Lanes outside the active pattern read zero slots.
#include <algorithm>
#include <memory>
#include <utility>
#include <vector>

#include "common.hpp"

namespace llmi_hip {
namespace {

#define TGMEM __attribute__((address_space(1)))
typedef unsigned int tu32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 tbf16x8 __attribute__((ext_vector_type(8)));
typedef float tf32x4 __attribute__((ext_vector_type(4)));
typedef float tf32x16 __attribute__((ext_vector_type(16)));

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

// The split activations a batch of three to eight rows reads (tol_split's
// output for the product's input), kept apart from TolProblem so that the
// small batches' kernel carries no unused fields.
struct TolSplit {
  const tu32x4* xs;  // [row][block][word][part]
  const float* sx;   // 24 * block sums of the split activations, [row][block]
};

// One distinct activation matrix of a launch, split once by tol_split.
struct TolInput {
  const float* x;
  tu32x4* xs;
  float* sx;
  int rows, in, nblk, first_word;  // first_word: this input's first word in tol_split's grid
};

// Two floats as a bf16 pair, rounded to nearest even (v_cvt_pk_bf16_f32).
typedef __bf16 tbf16x2 __attribute__((ext_vector_type(2)));
typedef float tf32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ std::uint32_t bf16_pair(float a, float b) {
  return __builtin_bit_cast(std::uint32_t, __builtin_convertvector(tf32x2{a, b}, tbf16x2));
}
// The split of two activations: *hi = bf16 pair of (a, b), *lo = bf16 pair
// of the remainders; returns (hi_a + lo_a) + (hi_b + lo_b).
__device__ __forceinline__ float split_pair(float a, float b, std::uint32_t* hi, std::uint32_t* lo) {
  const std::uint32_t h = bf16_pair(a, b);
  const float ha = __builtin_bit_cast(float, h << 16), hb = __builtin_bit_cast(float, h & 0xFFFF0000u);
  const std::uint32_t l = bf16_pair(a - ha, b - hb);
  const float la = __builtin_bit_cast(float, l << 16), lb = __builtin_bit_cast(float, l & 0xFFFF0000u);
  *hi = h;
  *lo = l;
  return (ha + la) + (hb + lb);
}

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

// tol_split: for every row and block of each input, the two bf16 parts of
// the 32 activations in the MFMA's k order ([row][block][word][part]
// 16-byte slots) and 24 * the sum of the block's x' = hi + lo (elements past
// `in` are zero).  Used by the batches of three to eight rows, whose
// workgroups would otherwise each split eight rows again.  One thread per
// word (8 activations); a quad of lanes adds its block's four word sums in a
// fixed order.  Grid: the inputs laid end to end, each starting at a
// multiple of 256 words (inputs[i].first_word), so workgroup g splits words
// of input wg_input[g] only; `single` stands for the tables when inputs is
// null.
__global__ void __launch_bounds__(256) tol_split(const TolInput* __restrict__ inputs,
                                                 const std::uint32_t* __restrict__ wg_input, TolInput single) {
  const int gw = blockIdx.x * blockDim.x + threadIdx.x;
  const TolInput t =
      inputs != nullptr ? inputs[__builtin_amdgcn_readfirstlane(static_cast<int>(wg_input[blockIdx.x]))] : single;
  const int w = gw - t.first_word;
  const int words = t.rows * t.nblk * 4;
  const bool live = w >= 0 && w < words;
  const int rb = live ? w >> 2 : 0, q = w & 3;
  const int r = live ? rb / t.nblk : 0, b = rb - r * t.nblk;
  float sum = 0.0f;
  if (live) {
    const float* xr = t.x + static_cast<std::size_t>(r) * t.in + static_cast<std::size_t>(b) * kBlock + 8 * q;
    const int len = t.in - (b * kBlock + 8 * q);
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = i < len ? xr[i] : 0.0f;
    // k-order pair p of the word holds elements p and p + 4.
    std::uint32_t hi[4], lo[4];
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) sum += split_pair(v[pr], v[pr + 4], &hi[pr], &lo[pr]);
    tu32x4* dst = t.xs + static_cast<std::size_t>(rb) * kSlotsPerBlock + 2 * q;
    dst[0] = tu32x4{hi[0], hi[1], hi[2], hi[3]};
    dst[1] = tu32x4{lo[0], lo[1], lo[2], lo[3]};
  }
  // Inputs start at multiples of four words, so a quad is one block.
  sum += __shfl_xor(sum, 1, 64);
  sum += __shfl_xor(sum, 2, 64);
  if (live && q == 0) t.sx[rb] = 24.0f * sum;
}

// qgemv_tol_small (batches of one or two rows, v_mfma_f32_16x16x32_bf16): one
// 64-row tile of one product for input rows [r0, r0 + nr), nr <= R.  The
// workgroup's wavefronts split the tile's blocks, bpw each; each
// wavefront splits the activations of its own blocks into its own LDS region
// (no workgroup barrier before the products; LDS operations of one wavefront
// complete in order).  Region of wavefront w: kZeroSlots zero slots (the A
// operand of inactive lanes; every wavefront writes the same zeros), then
// [row][block][word][part] 16-byte slots, then 24 * sx per row and block.
template <int R>
__global__ void __launch_bounds__(1024) qgemv_tol_small(const TolProblem* __restrict__ probs,
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
      std::uint32_t hp, lp;
      float sum = split_pair(xs[k][0], xs[k][1], &hp, &lp);
      const int pr = it & 15, rb = it >> 4;
      if (it < items) {
        std::uint32_t* slot = reinterpret_cast<std::uint32_t*>(wl + kZeroSlots + rb * kSlotsPerBlock + 2 * (pr >> 2));
        slot[pr & 3] = hp;
        slot[4 + (pr & 3)] = lp;
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
            if (rr < R && (R == 1 || rr < nr)) {  // a launch's rows are at least one
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
// The MFMA shapes.  Batches of one or two rows take v_mfma_f32_16x16x32_bf16
// (rows of the tile in groups of 16, the four m of a group = two input rows x
// two activation parts); batches of three to eight take
// v_mfma_f32_32x32x16_bf16 (groups of 32 rows, the sixteen m of a group =
// eight input rows x two parts), half the A reads and MFMAs per row.
//   16x16x32: A[m][k] at lane m + 16(k/8); B[k][n] at lane n + 16(k/8);
//             D[m][n] at lane n + 16(m/4), register m%4.
//   32x32x16: A[m][k] at lane m + 32(k/8); B[k][n] at lane n + 32(k/8);
//             D[m][n] at lane n + 32((m/4)%2), register 4(m/8) + m%4.
// With B = the codes of word q of lane l's own row, k-slice g = l/16 (l/32)
// carries row 16g + n (32g + n) and A[m][k] is nonzero only for k in the
// slice of m's group, so every lane receives its own row's sums.
// This lane's A-operand role: active, its activation part and input row.
template <bool K32>
__device__ __forceinline__ void a_role(int lane, bool* active, int* part, int* row) {
  if (K32) {
    const int m = lane & 31;
    *active = ((m >> 2) & 1) == (lane >> 5);
    *part = (m >> 3) & 1;
    *row = 4 * (m >> 4) + (m & 3);
  } else {
    const int m = lane & 15;
    *active = (m >> 2) == (lane >> 4);
    *part = m & 1;
    *row = (m >> 1) & 1;
  }
}

// Blocks per chunk of qgemv_tol_wide: one -- each block's MFMAs, sixteen
// accumulators and a batch's partial sums fill the registers, and fewer
// blocks in flight per wavefront buy more wavefronts per SIMD (batch 8 on
// MI355X: 43.4 us per SmolLM2 step with two, 35.5 with one).
constexpr int wide_chunk(int) { return 1; }

// qgemv_tol_wide (batches of three to eight rows, v_mfma_f32_32x32x16_bf16):
// one 64-row tile of one product for input rows [r0, r0 + nr), nr <= R.  The
// workgroup's wavefronts split the tile's blocks, bpw each, and walk them in
// chunks of kTolChunk.  Each wavefront copies the current chunk's split
// activations (tol_split's) into its own LDS region -- no workgroup barrier
// before the products; LDS operations of one wavefront complete in order --
// and loads the next chunk's activations and codes while it computes this
// one.  Region of a wavefront: kZeroSlots zero slots (the A operand of
// inactive lanes; every wavefront writes the same zeros), the chunk's
// [row][block][word][part] 16-byte slots, then 24 * sx per row and block of
// the chunk.
template <int R>
__global__ void __launch_bounds__(1024) qgemv_tol_wide(const TolProblem* __restrict__ probs,
                                                       const TolSplit* __restrict__ splits,
                                                       const std::uint32_t* __restrict__ wg_prob, TolProblem single,
                                                       TolSplit single_split) {
  static_assert(R == 4 || R == 8, "batches of three to eight rows");
  constexpr int kC = wide_chunk(R);  // blocks per chunk (registers: eight rows keep fewer in flight)
  // A row's kC * 8 slots are followed by one slot of padding: the active
  // lanes of an A read fetch one slot of each of 8 rows, which at a stride
  // of 8 slots (128 bytes) fall into the same LDS banks.
  constexpr int kRowSlots = kC * kSlotsPerBlock + 1;
  constexpr int kRegionSlots = kZeroSlots + R * kRowSlots;
  extern __shared__ tu32x4 lds[];
  const int wg = blockIdx.x;
  TolProblem p = single;
  TolSplit sp = single_split;
  if (probs != nullptr) {
    const int idx = __builtin_amdgcn_readfirstlane(static_cast<int>(wg_prob[wg]));
    p = probs[idx];
    sp = splits[idx];
  }
  const int local = wg - p.first_wg;
  const int tile = local % p.ntiles;
  const int r0 = (local / p.ntiles) * R;
  const int nr = min(R, p.rows - r0);
  const int nblk = p.nblk, bpw = p.bpw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int nwaves = blockDim.x >> 6;
  const int b_begin = wave * bpw, b_end = min(nblk, b_begin + bpw);

  const std::size_t tbase = static_cast<std::size_t>(tile) * nblk * kTileRows + lane;
  const TGMEM tu32x4* codes = (const TGMEM tu32x4*)p.codes + tbase;
  const TGMEM float* scales = (const TGMEM float*)p.scales + tbase;
  const TGMEM tu32x4* xsrc = (const TGMEM tu32x4*)sp.xs + static_cast<std::size_t>(r0) * nblk * kSlotsPerBlock;
  const TGMEM float* sxsrc = (const TGMEM float*)sp.sx + static_cast<std::size_t>(r0) * nblk;

  tu32x4* wl = lds + static_cast<std::size_t>(wave) * kRegionSlots;
  float* wsx = reinterpret_cast<float*>(lds + static_cast<std::size_t>(nwaves) * kRegionSlots) + wave * R * kC;
  float* red = reinterpret_cast<float*>(lds + static_cast<std::size_t>(nwaves) * kRegionSlots) + nwaves * R * kC;

  // Copy of a chunk starting at block c: slot i (of R rows x kC blocks
  // x 8) = row i / 32, slot i % 32 of the row's chunk (contiguous in
  // tol_split's layout); lane l copies slots l + 64 k, and lane l < 4R one
  // block sum.  Blocks past the wavefront's range are not read (their slots
  // are never used).
  constexpr int kChunkSlots = R * kC * kSlotsPerBlock;
  constexpr int kCopy = (kChunkSlots + 63) / 64;
  tu32x4 xs[kCopy];
  float sxv;
  const auto load_chunk_x = [&](int c) {
#pragma unroll
    for (int k = 0; k < kCopy; ++k) {
      const int i = lane + 64 * k, r = i / (kC * kSlotsPerBlock), off = i % (kC * kSlotsPerBlock);
      const bool ok = i < kChunkSlots && r < nr && c + (off >> 3) < b_end;
      xs[k] = ok ? xsrc[(static_cast<std::size_t>(r) * nblk + c) * kSlotsPerBlock + off] : tu32x4{0u, 0u, 0u, 0u};
    }
    const int r = lane / kC, jb = lane % kC;
    sxv = (lane < kC * R && r < nr && c + jb < b_end) ? sxsrc[static_cast<std::size_t>(r) * nblk + c + jb] : 0.0f;
  };
  const auto stage_chunk = [&]() {
#pragma unroll
    for (int k = 0; k < kCopy; ++k)
      if (lane + 64 * k < kChunkSlots) {
        const int i = lane + 64 * k, r = i / (kC * kSlotsPerBlock);
        wl[kZeroSlots + r * kRowSlots + (i - r * kC * kSlotsPerBlock)] = xs[k];
      }
    if (lane < kC * R) wsx[lane] = sxv;
  };

  // This lane's A operand: slot base + jb * step + 2q of the chunk's block
  // jb, word q (inactive lanes: step 0, base 0 -- a zero slot).
  bool active;
  int part, arow;
  a_role<true>(lane, &active, &part, &arow);
  const bool on = active && arow < nr;
  const int base = on ? kZeroSlots + arow * kRowSlots + part : 0;
  const int step = on ? kSlotsPerBlock : 0;
  const TolMagic mk = tol_magic();

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;

  if (b_begin < b_end) {
    // The first chunk: activations first, then codes (loads complete in
    // order, so waiting for the activations does not wait for HBM).
    load_chunk_x(b_begin);
    tu32x4 cur_c[kC];
    float cur_s[kC];
#pragma unroll
    for (int j = 0; j < kC; ++j) {
      const std::size_t bc = static_cast<std::size_t>(min(b_begin + j, b_end - 1));
      cur_c[j] = __builtin_nontemporal_load(codes + bc * kTileRows);
      cur_s[j] = __builtin_nontemporal_load(scales + bc * kTileRows);
    }
    if (lane < kZeroSlots) wl[lane] = tu32x4{0u, 0u, 0u, 0u};
    for (int b = b_begin; b < b_end; b += kC) {
      stage_chunk();
      // The next chunk's activations, then its codes.
      const int bn = b + kC;
      tu32x4 nxt_c[kC];
      float nxt_s[kC];
      if (bn < b_end) {
        load_chunk_x(bn);
#pragma unroll
        for (int j = 0; j < kC; ++j) {
          const std::size_t bc = static_cast<std::size_t>(min(bn + j, b_end - 1));
          nxt_c[j] = __builtin_nontemporal_load(codes + bc * kTileRows);
          nxt_s[j] = __builtin_nontemporal_load(scales + bc * kTileRows);
        }
      }
#pragma unroll
      for (int j = 0; j < kC; ++j) {
        if (b + j >= b_end) break;
        tf32x16 d{};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const tbf16x8 bq = decode_word(cur_c[j][q], mk);
          const tbf16x8 aq = __builtin_bit_cast(tbf16x8, wl[base + j * step + 2 * q]);
          d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq, bq, d, 0, 0, 0);
        }
        // Every row, also those past nr: their A slots and block sums are
        // zeros (so their sums stay zero and are never stored), and the
        // loop keeps no branch per row.
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int rh = 8 * (r >> 2) + (r & 3);
          const float blk = __builtin_fmaf(16.0f, d[rh] + d[rh + 4], -wsx[r * kC + j]);
          acc[r] = __builtin_fmaf(blk, cur_s[j], acc[r]);
        }
      }
      if (bn < b_end) {
#pragma unroll
        for (int j = 0; j < kC; ++j) {
          cur_c[j] = nxt_c[j];
          cur_s[j] = nxt_s[j];
        }
      }
    }
  }

  // The wavefronts' partial sums of each row, added in wavefront order.
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

// Wavefronts per tile: about kTolChunk blocks each, at most 16.
int tol_waves(std::size_t nblk) {
  return static_cast<int>(std::clamp<std::size_t>(ceil_div(nblk, kTolChunk), 1, 16));
}
// LDS of one workgroup.  qgemv_tol_small: per wavefront its zero slots and
// the split activations and block sums of its bpw blocks; qgemv_tol_wide: per
// wavefront its zero slots and one chunk's (kTolChunk blocks); both then the
// reduction area.
std::size_t tol_lds(int waves, int R, int bpw) {
  const std::size_t blocks = R <= 2 ? static_cast<std::size_t>(bpw) : static_cast<std::size_t>(wide_chunk(R));
  // qgemv_tol_wide pads each row of its chunk by one slot.
  const std::size_t pad = R <= 2 ? 0 : static_cast<std::size_t>(R);
  return static_cast<std::size_t>(waves) *
         ((kZeroSlots + static_cast<std::size_t>(R) * blocks * kSlotsPerBlock + pad) * sizeof(tu32x4) +
          static_cast<std::size_t>(R) * blocks * sizeof(float) + static_cast<std::size_t>(R) * kTileRows * sizeof(float));
}
// Row chunk R (1, 2, 4, 8): the smallest covering `rows`.
int tol_chunk(std::size_t rows) { return rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8; }

struct TolLaunch {
  int rchunk = 1, waves = 1, total_wgs = 0;
  std::size_t lds = 0, prob_offset = 0, map_offset = 0;
};

struct TolPlan {
  std::vector<TolInput> inputs;  // inputs of the batches of 3..8 (xs / sx: scratch offsets until bound)
  std::vector<TolProblem> probs;
  std::vector<TolSplit> splits;  // parallel to probs
  std::vector<std::uint32_t> wg_prob;
  std::vector<TolLaunch> launches;
  std::size_t scratch_bytes = 0;
  std::size_t split_words = 0;            // tol_split's grid, in words
  std::vector<std::uint32_t> split_wg;     // tol_split's workgroup -> input
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
    LLMI_REQUIRE(tol_lds(16, 2, static_cast<int>(ceil_div(m.nblk, 16))) <= max_lds_per_block(),
                 "tolerance matmul: rows too long");
  }
  // Distinct inputs of the batches of three to eight rows, split once.
  std::vector<std::size_t> input_of(count, 0);
  for (std::size_t i = 0; i < count; ++i) {
    const GroupEntry& e = entries[i];
    if (tol_chunk(e.rows) <= 2 || e.m->out == 0) continue;
    std::size_t k = plan->inputs.size();
    for (std::size_t j = 0; j < plan->inputs.size(); ++j)
      if (plan->inputs[j].x == e.x) {
        LLMI_REQUIRE(plan->inputs[j].rows == static_cast<int>(e.rows) && plan->inputs[j].in == static_cast<int>(e.m->in),
                     "tolerance matmul: one x used with two shapes");
        k = j;
      }
    if (k == plan->inputs.size()) {
      TolInput t{};
      t.x = e.x;
      t.rows = static_cast<int>(e.rows);
      t.in = static_cast<int>(e.m->in);
      t.nblk = static_cast<int>(e.m->nblk);
      t.first_word = static_cast<int>(plan->split_words);
      plan->split_words += ceil_div(e.rows * e.m->nblk * 4, 256) * 256;
      LLMI_REQUIRE(plan->split_words <= 0x7FFFFFFFu, "tolerance matmul: activations too large");
      plan->split_wg.insert(plan->split_wg.end(), (plan->split_words - t.first_word) / 256,
                            static_cast<std::uint32_t>(plan->inputs.size()));
      const std::size_t slots = e.rows * e.m->nblk;
      t.xs = reinterpret_cast<tu32x4*>(plan->scratch_bytes);
      plan->scratch_bytes += slots * kSlotsPerBlock * sizeof(tu32x4);
      t.sx = reinterpret_cast<float*>(plan->scratch_bytes);
      plan->scratch_bytes += (slots * sizeof(float) + 255) & ~std::size_t{255};
      plan->inputs.push_back(t);
    }
    input_of[i] = k;
  }
  for (int R : {1, 2, 4, 8}) {
    std::vector<std::pair<TolProblem, TolSplit>> probs;
    int waves = 1;
    std::size_t biggest = 0, lds = 0;
    for (std::size_t i = 0; i < count; ++i) {
      const GroupEntry& e = entries[i];
      const DeviceMatrix& m = *e.m;
      if (m.out == 0 || tol_chunk(e.rows) != R) continue;
      TolProblem p{};
      p.codes = m.codes;
      p.scales = m.scales;
      p.bias = e.bias;
      p.y = e.y;
      p.x = e.x;
      TolSplit sp{};
      if (R > 2) sp = TolSplit{plan->inputs[input_of[i]].xs, plan->inputs[input_of[i]].sx};
      p.in = static_cast<int>(m.in);
      p.nblk = static_cast<int>(m.nblk);
      p.out = static_cast<int>(m.out);
      p.rows = static_cast<int>(e.rows);
      p.ntiles = static_cast<int>(m.ntiles);
      p.accumulate = e.accumulate ? 1 : 0;
      probs.emplace_back(p, sp);
      const std::size_t bytes = m.code_bytes + m.scale_bytes;
      if (bytes > biggest) {
        biggest = bytes;
        waves = tol_waves(m.nblk);
      }
    }
    if (probs.empty()) continue;
    // Longest workgroups first, as in the exact grouped launch.
    std::stable_sort(probs.begin(), probs.end(),
                     [](const auto& a, const auto& b) { return a.first.nblk > b.first.nblk; });
    TolLaunch l;
    l.rchunk = R;
    l.waves = waves;
    l.prob_offset = plan->probs.size();
    l.map_offset = plan->wg_prob.size();
    std::size_t wg = 0;
    for (std::size_t j = 0; j < probs.size(); ++j) {
      TolProblem& p = probs[j].first;
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
    for (const auto& [p, sp] : probs) {
      plan->probs.push_back(p);
      plan->splits.push_back(sp);
    }
    plan->launches.push_back(l);
  }
  return LLMI_OK;
}

// Scratch offsets -> device addresses.
void bind_tol(TolPlan* plan, std::uint8_t* scratch) {
  const auto at = [scratch](const void* off) { return scratch + reinterpret_cast<std::size_t>(off); };
  for (TolInput& t : plan->inputs) {
    t.xs = reinterpret_cast<tu32x4*>(at(t.xs));
    t.sx = reinterpret_cast<float*>(at(t.sx));
  }
  for (std::size_t i = 0; i < plan->splits.size(); ++i)
    if (plan->probs[i].rows > 2) {  // tol_chunk > 2: the split is read
      TolSplit& sp = plan->splits[i];
      sp.xs = reinterpret_cast<const tu32x4*>(at(sp.xs));
      sp.sx = reinterpret_cast<const float*>(at(sp.sx));
    }
}

int launch_tol_kernel(const TolLaunch& l, const TolProblem* probs, const TolSplit* splits, const std::uint32_t* map,
                      const TolProblem& single, const TolSplit& single_split, hipStream_t s) {
  if (l.total_wgs == 0) return LLMI_OK;
  const dim3 grid(static_cast<unsigned>(l.total_wgs)), block(static_cast<unsigned>(l.waves * 64));
  switch (l.rchunk) {
    case 1: qgemv_tol_small<1><<<grid, block, l.lds, s>>>(probs, map, single); break;
    case 2: qgemv_tol_small<2><<<grid, block, l.lds, s>>>(probs, map, single); break;
    case 4: qgemv_tol_wide<4><<<grid, block, l.lds, s>>>(probs, splits, map, single, single_split); break;
    default: qgemv_tol_wide<8><<<grid, block, l.lds, s>>>(probs, splits, map, single, single_split); break;
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
  std::uint8_t* scratch = nullptr;  // split activations of the batches of 3..8
  const TolInput* inputs = nullptr;
  const TolProblem* probs = nullptr;
  const TolSplit* splits = nullptr;
  const std::uint32_t* map = nullptr;
  const std::uint32_t* split_wg = nullptr;
  TolPlan plan;
  ~llmi_hip_tol_group() {
    if (table != nullptr) (void)hipFree(table);
    if (scratch != nullptr) (void)hipFree(scratch);
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

// The single-product entry keeps its split activations here (grow-only).
struct TolWorkspace {
  std::uint8_t* scratch = nullptr;
  std::size_t bytes = 0;
};
TolWorkspace g_tol_ws;

}  // namespace

namespace llmi_hip {
void release_tol_workspace() {
  if (g_tol_ws.scratch != nullptr) (void)hipFree(g_tol_ws.scratch);
  g_tol_ws = TolWorkspace{};
}
}  // namespace llmi_hip

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
  if (g->plan.scratch_bytes > 0) {
    LLMI_TRY_HIP(hipMalloc(reinterpret_cast<void**>(&g->scratch), g->plan.scratch_bytes));
    bind_tol(&g->plan, g->scratch);
  }
  const std::size_t ib = g->plan.inputs.size() * sizeof(TolInput);
  const std::size_t pb = g->plan.probs.size() * sizeof(TolProblem);
  const std::size_t sb = g->plan.splits.size() * sizeof(TolSplit);
  const std::size_t mb = g->plan.wg_prob.size() * sizeof(std::uint32_t);
  const std::size_t xb = g->plan.split_wg.size() * sizeof(std::uint32_t);
  if (ib + pb + sb + mb + xb > 0) {
    LLMI_TRY_HIP(hipMalloc(&g->table, ib + pb + sb + mb + xb));
    auto* base = static_cast<std::uint8_t*>(g->table);
    if (ib > 0) LLMI_TRY_HIP(hipMemcpy(base, g->plan.inputs.data(), ib, hipMemcpyHostToDevice));
    if (pb > 0) LLMI_TRY_HIP(hipMemcpy(base + ib, g->plan.probs.data(), pb, hipMemcpyHostToDevice));
    if (sb > 0) LLMI_TRY_HIP(hipMemcpy(base + ib + pb, g->plan.splits.data(), sb, hipMemcpyHostToDevice));
    if (mb > 0) LLMI_TRY_HIP(hipMemcpy(base + ib + pb + sb, g->plan.wg_prob.data(), mb, hipMemcpyHostToDevice));
    g->inputs = reinterpret_cast<const TolInput*>(base);
    g->probs = reinterpret_cast<const TolProblem*>(base + ib);
    g->splits = reinterpret_cast<const TolSplit*>(base + ib + pb);
    g->map = reinterpret_cast<const std::uint32_t*>(base + ib + pb + sb);
    if (xb > 0)
      LLMI_TRY_HIP(hipMemcpy(base + ib + pb + sb + mb, g->plan.split_wg.data(), xb, hipMemcpyHostToDevice));
    g->split_wg = reinterpret_cast<const std::uint32_t*>(base + ib + pb + sb + mb);
  }
  *out = g.release();
  return LLMI_OK;
}

int llmi_hip_tol_group_launch(const llmi_hip_tol_group* g, void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(g != nullptr, "tolerance matmul: null group");
  if (!g->plan.inputs.empty()) {
    tol_split<<<static_cast<unsigned>(g->plan.split_words / 256), 256, 0, pick(stream)>>>(g->inputs, g->split_wg,
                                                                                          TolInput{});
    LLMI_TRY_HIP(hipGetLastError());
  }
  for (const TolLaunch& l : g->plan.launches)
    if (int rc = launch_tol_kernel(l, g->probs + l.prob_offset, g->splits + l.prob_offset, g->map + l.map_offset,
                                   TolProblem{}, TolSplit{}, pick(stream)))
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
  // One product: its descriptor (and the split's) travel as kernel arguments.
  const hipStream_t s = pick(stream);
  if (plan.scratch_bytes > 0) {
    if (plan.scratch_bytes > g_tol_ws.bytes) {
      LLMI_TRY_HIP(hipStreamSynchronize(s));
      release_tol_workspace();
      LLMI_TRY_HIP(hipMalloc(reinterpret_cast<void**>(&g_tol_ws.scratch), plan.scratch_bytes));
      g_tol_ws.bytes = plan.scratch_bytes;
    }
    bind_tol(&plan, g_tol_ws.scratch);
    tol_split<<<static_cast<unsigned>(plan.split_words / 256), 256, 0, s>>>(nullptr, nullptr, plan.inputs[0]);
    LLMI_TRY_HIP(hipGetLastError());
  }
  TolProblem p = plan.probs[0];
  p.first_wg = 0;
  return launch_tol_kernel(plan.launches[0], nullptr, nullptr, nullptr, p, plan.splits[0], s);
}

}  // extern "C"
