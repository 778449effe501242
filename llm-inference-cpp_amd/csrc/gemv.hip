// Quantized matrix-vector / small-batch product for gfx950.
//
// Reference: src/model/quant.cpp:119-153.  For each output o and input row r
// the reference computes, with the compiler's fused multiply-adds,
//     part_b = fma(x[k], code[k], part_b)   over the block's elements in order
//     acc    = fma(part_b, scale_b, acc)    over the blocks in order
//     y      = acc + bias[o]                (bias 0.0f when absent)
// These kernels perform exactly those operations, so y is bit-identical.
//
// All kernels read the tiled layout (common.hpp): lane l of a wavefront owns
// output row tile*64 + l, so one block of 64 rows is a single coalesced
// 16-byte load per lane (two for Q8_0), and the activations x[k] are the
// same for every lane -- they are read with scalar loads into SGPRs and
// broadcast to the fused multiply-adds.  Every code byte and scale is read
// from HBM once; the kernels are HBM-bound at batch 1.
//
// qgemv_tile (batch 1..8): one workgroup per (64-row tile, chunk of up to R
// input rows).  Its W wavefronts split the tile's blocks into contiguous
// ranges; each decodes a block once and forms the block sums of every input
// row of the chunk, which it parks in LDS together with the block scales.
// After one barrier the wavefronts run the sequential chains over all blocks
// (one chain per input row), add the bias and store y.  Splitting the blocks
// over wavefronts is what fills the GPU when a matrix has few tiles.
//
// qgemv_narrow (batch 1, matrices with few rows): 16-row tiles, 4x the
// workgroups of qgemv_tile.
//
// qgemv_group: a fixed list of products (each batch 1..8) launched together
// (one kernel per row chunk R present); each workgroup runs one tile of one
// product with the same tile functions.
//
// qgemm_exact (batch > 8 on matrices with many tiles, e.g. an lm_head over
// every position): 64 input rows x 64 outputs per workgroup, 4 x 4 chains
// per thread, operands from LDS.
//
// qgemm_split (batch > 8 on matrices with few tiles, the prefill's
// projections): a tile's blocks spread over the workgroup's wavefronts,
// activations from scalar loads, block sums and scales through LDS.
//
// fp32 weights take kernels::matmul instead (f32.hip).
#include <algorithm>
#include <type_traits>
#include <vector>

#include "common.hpp"
#include "glue_math.hpp"

namespace llmi_hip {

namespace {

// Signed bit-field extract (v_bfe_i32).  The builtin is declared with an
// unsigned result, so the value is reinterpreted as int before any
// conversion to float.
__device__ __forceinline__ int sfield(std::uint32_t w, int offset, int width) {
  return static_cast<int>(__builtin_amdgcn_sbfe(w, offset, width));
}

// Global-memory pointers.  The grouped kernel reads its pointers from a
// table, where the compiler cannot see that they point to global memory;
// typing them keeps global (not flat) loads for the weights and scalar
// loads for the activations.
#define GMEM __attribute__((address_space(1)))
template <typename T>
__device__ __forceinline__ const GMEM T* gmem(const T* p) {
  return (const GMEM T*)p;
}
template <typename T>
__device__ __forceinline__ GMEM T* gmem_out(T* p) {
  return (GMEM T*)p;
}

template <int TYPE>
struct Block {
  static constexpr int kU = TYPE == LLMI_TYPE_Q8_0 ? 2 : 1;  // 16-byte loads per lane per block
  uint4 c[kU];
};

// Weights are streamed through once per product, so the batch 1..8 kernels
// load them with the nontemporal hint (they are not kept in the caches for
// reuse); the multi-row prefill kernel re-reads a tile per row chunk and uses
// ordinary loads.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
template <bool NT>
__device__ __forceinline__ uint4 load16(const GMEM uint4* p) {
  const GMEM u32x4* q = reinterpret_cast<const GMEM u32x4*>(p);
  const u32x4 v = NT ? __builtin_nontemporal_load(q) : *q;
  return uint4{v.x, v.y, v.z, v.w};
}
template <bool NT>
__device__ __forceinline__ float loadf(const GMEM float* p) {
  if (NT) return __builtin_nontemporal_load(p);
  return *p;
}

template <int TYPE, bool NT>
__device__ __forceinline__ Block<TYPE> load_block(const GMEM uint4* __restrict__ codes, std::size_t slot, int lane) {
  Block<TYPE> b;
#pragma unroll
  for (int u = 0; u < Block<TYPE>::kU; ++u) b.c[u] = load16<NT>(codes + (slot * Block<TYPE>::kU + u) * kTileRows + lane);
  return b;
}

// The code of element i of a block as float, exactly.
//   Q4_0: element i is nibble i%8 of word i/8 with +8 bias; XOR-ing every
//         nibble with 8 turns it into the 4-bit two's complement of n - 8.
//   Q8_0: element i is signed byte i%4 of word i/4.
template <int TYPE>
__device__ __forceinline__ float code_of(const std::uint32_t* w, int i) {
  if (TYPE == LLMI_TYPE_Q4_0) return static_cast<float>(sfield(w[i >> 3], (i & 7) * 4, 4));
  return static_cast<float>(sfield(w[i >> 2], (i & 3) * 8, 8));
}

template <int TYPE>
__device__ __forceinline__ void unpack_words(const Block<TYPE>& b, std::uint32_t* w) {
  if (TYPE == LLMI_TYPE_Q4_0) {
    w[0] = b.c[0].x ^ 0x88888888u;
    w[1] = b.c[0].y ^ 0x88888888u;
    w[2] = b.c[0].z ^ 0x88888888u;
    w[3] = b.c[0].w ^ 0x88888888u;
  } else {
    w[0] = b.c[0].x; w[1] = b.c[0].y; w[2] = b.c[0].z; w[3] = b.c[0].w;
    w[4] = b.c[Block<TYPE>::kU - 1].x; w[5] = b.c[Block<TYPE>::kU - 1].y;
    w[6] = b.c[Block<TYPE>::kU - 1].z; w[7] = b.c[Block<TYPE>::kU - 1].w;
  }
}

// Q4_0 decode constants, kept in VGPRs (v_and_or_b32 takes no literal).
// Two 4-bit codes n (element value n - 8) are moved into the mantissas of an
// f16 pair whose exponent makes the pair (1024 + n) (nibble at bits 0-3 of a
// half) or (64 + n) (bits 4-7); one packed f16 subtraction of 1032 or 72
// then gives n - 8 exactly, and v_fma_mix_f32 takes the f16 operand into an
// fp32 fused multiply-add with no separate conversion.  The products and
// sums are the same fp32 operations as with an fp32 code operand.
struct Q4Magic {
  std::uint32_t lo_mask, hi_mask, lo_exp, hi_exp;
};
__device__ __forceinline__ Q4Magic q4_magic() {
  Q4Magic k{0x000F000Fu, 0x00F000F0u, 0x64006400u, 0x54005400u};
  asm("" : "+v"(k.lo_mask), "+v"(k.hi_mask), "+v"(k.lo_exp), "+v"(k.hi_exp));
  return k;
}
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ half2_t f16_pair(std::uint32_t w, std::uint32_t mask, std::uint32_t exp_bits) {
  std::uint32_t d;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(d) : "v"(w), "v"(mask), "v"(exp_bits));
  return __builtin_bit_cast(half2_t, d);
}

// Block sum of one full block: part = fma(x[i], code[i], part), i = 0..31;
// XP points to the block's 32 activations (global memory or LDS).  For one
// input row Q4_0 codes go to v_fma_mix_f32 as f16 pairs; the multi-row
// kernels instead convert each code to fp32 once (block_codes) and use it in
// R v_fmac_f32, which issue at twice the rate of the mixed-precision FMA on
// gfx950.
template <int TYPE, typename XP>
__device__ __forceinline__ float full_block_dot(const Block<TYPE>& b, XP __restrict__ xr, const Q4Magic& k) {
  float part = 0.0f;
  if (TYPE == LLMI_TYPE_Q8_0) {
    const std::uint32_t w[8] = {b.c[0].x, b.c[0].y, b.c[0].z, b.c[0].w, b.c[Block<TYPE>::kU - 1].x,
                                b.c[Block<TYPE>::kU - 1].y, b.c[Block<TYPE>::kU - 1].z, b.c[Block<TYPE>::kU - 1].w};
#pragma unroll
    for (int i = 0; i < kBlock; ++i) part = __builtin_fmaf(xr[i], code_of<TYPE>(w, i), part);
    return part;
  }
  // Word j holds elements 8j..8j+7 as nibbles 0..7 (element 8j+2m in the low
  // nibble of byte m, 8j+2m+1 in the high nibble).
  const half2_t lo_off = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
  const half2_t hi_off = {static_cast<_Float16>(-72.0f), static_cast<_Float16>(-72.0f)};
  const std::uint32_t w[4] = {b.c[0].x, b.c[0].y, b.c[0].z, b.c[0].w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const std::uint32_t s = w[j] >> 8;
    const half2_t e04 = f16_pair(w[j], k.lo_mask, k.lo_exp) + lo_off;  // elements 0, 4 of the word
    const half2_t e15 = f16_pair(w[j], k.hi_mask, k.hi_exp) + hi_off;  // 1, 5
    const half2_t e26 = f16_pair(s, k.lo_mask, k.lo_exp) + lo_off;     // 2, 6
    const half2_t e37 = f16_pair(s, k.hi_mask, k.hi_exp) + hi_off;     // 3, 7
    const XP xj = xr + 8 * j;
    part = __builtin_fmaf(xj[0], static_cast<float>(e04.x), part);
    part = __builtin_fmaf(xj[1], static_cast<float>(e15.x), part);
    part = __builtin_fmaf(xj[2], static_cast<float>(e26.x), part);
    part = __builtin_fmaf(xj[3], static_cast<float>(e37.x), part);
    part = __builtin_fmaf(xj[4], static_cast<float>(e04.y), part);
    part = __builtin_fmaf(xj[5], static_cast<float>(e15.y), part);
    part = __builtin_fmaf(xj[6], static_cast<float>(e26.y), part);
    part = __builtin_fmaf(xj[7], static_cast<float>(e37.y), part);
  }
  return part;
}

// The 32 codes of a full block as fp32 (for the multi-row kernels).
template <int TYPE>
__device__ __forceinline__ void block_codes(const Block<TYPE>& b, float* c) {
  std::uint32_t w[8];
  unpack_words<TYPE>(b, w);
#pragma unroll
  for (int i = 0; i < kBlock; ++i) c[i] = code_of<TYPE>(w, i);
}

template <typename XP>
__device__ __forceinline__ float codes_dot(const float* c, XP __restrict__ xr) {
  float part = 0.0f;
#pragma unroll
  for (int i = 0; i < kBlock; ++i) part = __builtin_fmaf(xr[i], c[i], part);
  return part;
}

// Block sum of the final partial block (len < 32 elements).
template <int TYPE, typename XP>
__device__ __noinline__ float tail_block_dot(const Block<TYPE> blk, XP __restrict__ xr, int len) {
  std::uint32_t w[8];
  unpack_words<TYPE>(blk, w);
  float part = 0.0f;
#pragma unroll
  for (int i = 0; i < kBlock; ++i)
    if (i < len) part = __builtin_fmaf(xr[i], code_of<TYPE>(w, i), part);
  return part;
}

// Block sums of blocks [b_begin, b_end) of one tile for input rows [0, nr)
// (nr <= R; row r starts at x + r*in) into part[(r*nblk + b)*64 + lane], and
// the blocks' scales into scl[b*64 + lane].  Loads run CH blocks ahead.
template <int TYPE, int R, int CH>
__device__ __forceinline__ void block_sums(const GMEM uint4* __restrict__ codes, const GMEM float* __restrict__ scales,
                                           const GMEM float* __restrict__ x, std::size_t tile, int in, int nblk, int nr,
                                           int b_begin, int b_end, int lane, float* part, float* scl) {
  const Q4Magic k = q4_magic();
  const int nfull = in / kBlock;
  const int f_end = min(b_end, nfull);
  const std::size_t base = tile * nblk;
  Block<TYPE> cur[CH];
  float cur_s[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    if (b_begin + j < f_end) {
      cur[j] = load_block<TYPE, true>(codes, base + b_begin + j, lane);
      cur_s[j] = loadf<true>(scales + (base + b_begin + j) * kTileRows + lane);
    }
  }
  for (int b = b_begin; b < f_end; b += CH) {
    Block<TYPE> nxt[CH];
    float nxt_s[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (b + CH + j < f_end) {
        nxt[j] = load_block<TYPE, true>(codes, base + b + CH + j, lane);
        nxt_s[j] = loadf<true>(scales + (base + b + CH + j) * kTileRows + lane);
      }
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (b + j < f_end) {
        if (R == 1) {
          part[(b + j) * kTileRows + lane] = full_block_dot<TYPE>(cur[j], x + (b + j) * kBlock, k);
        } else {
          float c[kBlock];
          block_codes<TYPE>(cur[j], c);
#pragma unroll
          for (int r = 0; r < R; ++r) {
            if (r < nr)
              part[(r * nblk + b + j) * kTileRows + lane] =
                  codes_dot(c, x + static_cast<std::size_t>(r) * in + (b + j) * kBlock);
          }
        }
        scl[(b + j) * kTileRows + lane] = cur_s[j];
      }
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      cur[j] = nxt[j];
      cur_s[j] = nxt_s[j];
    }
  }
  if (nfull < nblk && nfull >= b_begin && nfull < b_end) {
    const Block<TYPE> blk = load_block<TYPE, true>(codes, base + nfull, lane);
    for (int r = 0; r < nr; ++r)
      part[(r * nblk + nfull) * kTileRows + lane] =
          tail_block_dot<TYPE>(blk, x + static_cast<std::size_t>(r) * in + nfull * kBlock, in - nfull * kBlock);
    scl[nfull * kTileRows + lane] = loadf<true>(scales + (base + nfull) * kTileRows + lane);
  }
}

// The sequential chain over all blocks of one row of a tile, from LDS
// (stride `stride` floats between blocks).  Two register sets of
// kChainRound blocks: the reads of one are issued before the fused
// multiply-adds of the other, so LDS latency overlaps the chain.  The reads
// walk two pointers with constant offsets (an index clamped to the last
// block puts the next address in a register an outstanding read still
// targets, and every round then waits for all reads in flight).  A round's
// look-ahead may read up to kChainRound blocks past the row: inside the
// next row or the scales, or in the padding wide_lds adds after them; those
// values are never used.
constexpr int kChainRound = 4;
__device__ __forceinline__ float chain_lds(const float* part, const float* scl, int nblk, int lane, int stride) {
  const float* pp = part + lane;
  const float* sp = scl + lane;
  float pa[kChainRound], sa[kChainRound], pb[kChainRound], sb[kChainRound];
  const auto read = [&](float* p, float* q, const float* ps, const float* ss) {
#pragma unroll
    for (int u = 0; u < kChainRound; ++u) {
      p[u] = ps[u * stride];
      q[u] = ss[u * stride];
    }
  };
  float acc = 0.0f;
  const auto steps = [&](const float* p, const float* q) {
#pragma unroll
    for (int u = 0; u < kChainRound; ++u) acc = __builtin_fmaf(p[u], q[u], acc);
  };
  read(pa, sa, pp, sp);
  int b = 0;
  for (; b + 2 * kChainRound <= nblk; b += 2 * kChainRound) {
    read(pb, sb, pp + kChainRound * stride, sp + kChainRound * stride);
    __builtin_amdgcn_sched_barrier(0);
    steps(pa, sa);
    read(pa, sa, pp + 2 * kChainRound * stride, sp + 2 * kChainRound * stride);
    __builtin_amdgcn_sched_barrier(0);
    steps(pb, sb);
    pp += 2 * kChainRound * stride;
    sp += 2 * kChainRound * stride;
  }
  // pa holds blocks b .. b + 3 (those below nblk); the rest one by one.
#pragma unroll
  for (int u = 0; u < kChainRound; ++u)
    if (b + u < nblk) acc = __builtin_fmaf(pa[u], sa[u], acc);
  for (int c = b + kChainRound; c < nblk; ++c) acc = __builtin_fmaf(part[c * stride + lane], scl[c * stride + lane], acc);
  return acc;
}

__device__ __forceinline__ void store_out(GMEM float* __restrict__ y, std::size_t o, float v, int accumulate) {
  y[o] = accumulate ? y[o] + v : v;
}

// Load chunk (blocks in flight per wavefront) of the 64-row tile kernels,
// from launch-shape sweeps on MI355X: Q4_0 takes up to 4 blocks (one 16-byte
// load each), Q8_0 one block (two loads).
template <int TYPE>
constexpr int wide_chunk() {
  return TYPE == LLMI_TYPE_Q8_0 ? 1 : 4;
}

// One 64-row tile for input rows [0, nr), nr <= R (x, y already point at the
// chunk's first row).  The workgroup's wavefronts split the blocks, bpw
// each, and park block sums and scales in LDS (part[nr][nblk][64] then
// scale[nblk][64]); wavefront w then runs the chains of rows w, w + W, ...
// Every thread of the workgroup must call it (it has a barrier).
template <int TYPE, int R>
__device__ __forceinline__ void wide_tile(const GMEM uint4* __restrict__ codes, const GMEM float* __restrict__ scales,
                                          const GMEM float* __restrict__ x, const GMEM float* __restrict__ bias,
                                          GMEM float* __restrict__ y, int in, int nblk, int out, int nr, int bpw,
                                          int accumulate, std::size_t tile, float* lds) {
  float* part = lds;
  float* scl = lds + static_cast<std::size_t>(nr) * nblk * kTileRows;
  const int lane = threadIdx.x & (kTileRows - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int b_begin = wave * bpw;
  const int b_end = min(nblk, b_begin + bpw);
  block_sums<TYPE, R, wide_chunk<TYPE>()>(codes, scales, x, tile, in, nblk, nr, b_begin, b_end, lane, part, scl);
  __syncthreads();
  const std::size_t o = tile * kTileRows + lane;
  for (int r = wave; r < nr; r += nwaves) {
    const float acc = chain_lds(part + static_cast<std::size_t>(r) * nblk * kTileRows, scl, nblk, lane, kTileRows);
    if (o < static_cast<std::size_t>(out))
      store_out(y + static_cast<std::size_t>(r) * out, o, acc + (bias != nullptr ? bias[o] : 0.0f), accumulate);
  }
}

// Stages the activations of a 16-row tile in LDS, applying the prologue
// (see kPlain, kRmsNorm, kSiluUp).  Every thread of the workgroup calls it;
// it ends with a barrier.
// Elements each thread loads per round of stage_x: a round's loads are all
// issued before the first one is used, so a row of `in` activations costs
// one memory round trip while in <= kStageBatch * blockDim.x.
constexpr int kStageBatch = 8;

__device__ __forceinline__ void stage_x(const GMEM float* __restrict__ x, int in, int prologue,
                                        const GMEM float* __restrict__ pw, float eps, float* xs) {
  __shared__ double red[64];
  __shared__ std::uint64_t tab[32];
  const int tid = threadIdx.x, nthreads = blockDim.x;

  const bool one_round = in <= nthreads * kStageBatch;
  float v[kStageBatch], w[kStageBatch];
  double part = 0.0;
  const auto round = [&](int i0) {
#pragma unroll
    for (int u = 0; u < kStageBatch; ++u) {
      const int i = i0 + u * nthreads + tid;
      v[u] = i < in ? x[i] : 0.0f;
      w[u] = prologue != kPlain && i < in ? pw[i] : 0.0f;
    }
    if (prologue == kSiluUp && i0 == 0) {
      if (tid < 32) tab[tid] = exact::kExp2Tab[tid];
      __syncthreads();
    }
#pragma unroll
    for (int u = 0; u < kStageBatch; ++u) {
      const int i = i0 + u * nthreads + tid;
      if (i < in) {
        if (prologue == kSiluUp) {
          xs[i] = silu_exact(v[u], tab) * w[u];
        } else {
          xs[i] = v[u];
          const double d = static_cast<double>(v[u]);
          part = __builtin_fma(d, d, part);
        }
      }
    }
  };
  // The first round outside the loop: a loop header makes the compiler wait
  // for every load in flight (the caller's weight loads, issued just
  // before), which would put the activations' round trip after theirs.
  round(0);
  for (int i0 = nthreads * kStageBatch; i0 < in; i0 += nthreads * kStageBatch) round(i0);
  if (prologue != kRmsNorm) {
    __syncthreads();
    return;
  }
  // RMSNorm: the double sum of squares in any order, taken when the error
  // bound proves the reference's sequential sum gives the same float scale
  // (else summed sequentially), then y = w * (x * scale).
  part = row_sum16_f64(part);
  if ((tid & 15) == 15) red[tid >> 4] = part;
  __syncthreads();
  // Every wave sums the (up to 64) row partials with its lanes, as a tree,
  // and evaluates the three scales of the bound check -- at ss - slack, ss
  // and ss + slack -- on lanes 0, 1 and 2 at once (one double division and
  // square root deep, not three).
  const int lane = tid & 63;
  double rs = lane < (nthreads >> 4) ? red[lane] : 0.0;
  rs = row_sum16_f64(rs);
  const double ss = (readlane_f64(rs, 15) + readlane_f64(rs, 31)) + (readlane_f64(rs, 47) + readlane_f64(rs, 63));
  const double slack = sum_slack(in) * ss;
  const float mine = rms_scale(lane == 0 ? ss - slack : lane == 2 ? ss + slack : ss, in, eps);
  float sc = readlane_f32(mine, 1);
  if (readlane_f32(mine, 0) != readlane_f32(mine, 2)) {
    double seq = 0.0;  // every x is in LDS (the barrier above)
    for (int i = 0; i < in; ++i) {
      const double d = static_cast<double>(xs[i]);
      seq = __builtin_fma(d, d, seq);
    }
    sc = rms_scale(seq, in, eps);
    __syncthreads();  // (uniform branch) xs is read before it is scaled
  }
  if (one_round) {
    // This thread's x and w are still in registers.
#pragma unroll
    for (int u = 0; u < kStageBatch; ++u) {
      const int i = u * nthreads + tid;
      if (i < in) xs[i] = w[u] * (v[u] * sc);
    }
  } else {
    // Each thread scales the elements it staged.
    for (int i = tid; i < in; i += nthreads) xs[i] = pw[i] * (xs[i] * sc);
  }
  __syncthreads();
}

// LDS row stride (floats) of a 16-row tile's (block sum, scale) pairs: nblk
// pairs rounded up to 16, plus 4 floats, so the 16 rows start 4 banks apart.
__host__ __device__ __forceinline__ int pair_stride(int nblk) { return 2 * ((nblk + 15) & ~15) + 4; }

// The sequential chain over the (block sum, scale) pairs of one row, two
// blocks per 16-byte LDS read, eight reads (16 blocks) per round.  Two
// register sets: the reads of one round are issued before the fused
// multiply-adds of the other, and whole rounds run without per-block
// conditions (only the last, partial round has them).  The reads walk one
// pointer with constant offsets; a look-ahead may read up to 15 pairs past
// nblk -- inside the next row, or in the padding narrow_lds adds after the
// last row -- and those values are never used.
constexpr int kPairPad = 32;  // floats of look-ahead padding after the last row
__device__ __forceinline__ float chain_pairs(const float* row, int nblk) {
  const float4* pr = reinterpret_cast<const float4*>(row);
  float4 a[8], c[8];
  const auto read = [&](float4* v, const float4* src) {
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = src[u];
  };
  float acc = 0.0f;
  const auto steps = [&](const float4* v) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      acc = __builtin_fmaf(v[u].x, v[u].y, acc);
      acc = __builtin_fmaf(v[u].z, v[u].w, acc);
    }
  };
  read(a, pr);
  int b = 0;
  for (; b + 32 <= nblk; b += 32) {
    read(c, pr + 8);
    __builtin_amdgcn_sched_barrier(0);
    steps(a);
    read(a, pr + 16);
    __builtin_amdgcn_sched_barrier(0);
    steps(c);
    pr += 16;
  }
  // a holds pairs b .. b + 15; fewer than 32 remain.
  if (b + 16 <= nblk) {
    read(c, pr + 8);
    __builtin_amdgcn_sched_barrier(0);
    steps(a);
#pragma unroll
    for (int u = 0; u < 8; ++u) a[u] = c[u];
    b += 16;
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    if (b + 2 * u < nblk) acc = __builtin_fmaf(a[u].x, a[u].y, acc);
    if (b + 2 * u + 1 < nblk) acc = __builtin_fmaf(a[u].z, a[u].w, acc);
  }
  return acc;
}

// One 16-row tile (batch 1), for matrices with few rows.  Lane l of a
// wavefront owns row tile16*16 + (l & 15) and one of 4 block groups (l >> 4);
// the W wavefronts give 4W groups of bpg contiguous blocks.  The 16 rows of
// one block are a contiguous 256-byte piece of the 64-row layout, so loads
// stay coalesced.  The first kHoist blocks of a lane are loaded before the
// activations are staged (the two round trips overlap).  The activations sit
// in LDS and are read with broadcast loads (16 lanes per address); block
// sums and scales go to LDS as pairs, and lanes 0-15 run the chains.  LDS:
// x[in (padded to 4)], then 16 rows of pair_stride(nblk) floats.
template <int TYPE>
__device__ __forceinline__ void narrow_tile(const GMEM uint4* __restrict__ codes, const GMEM float* __restrict__ scales,
                                            const GMEM float* __restrict__ x, const GMEM float* __restrict__ bias,
                                            GMEM float* __restrict__ y, int in, int nblk, int out, int bpg, int accumulate,
                                            std::size_t tile16, float* lds, int prologue = kPlain,
                                            const GMEM float* __restrict__ pw = nullptr, float eps = 0.0f) {
  constexpr int kHoist = 4;
  const Q4Magic k = q4_magic();
  float* xs = lds;
  const int stride = pair_stride(nblk);
  float* pairs = lds + ((in + 3) & ~3);
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int group = (threadIdx.x >> 6) * 4 + (lane >> 4);
  const std::size_t row = tile16 * 16 + r;
  const std::size_t tile = row / kTileRows;
  const int sub = static_cast<int>(row % kTileRows);
  const int nfull = in / kBlock;
  const int b_begin = group * bpg;
  const int b_end = min(nblk, b_begin + bpg);
  Block<TYPE> pre[kHoist];
  float pre_s[kHoist];
#pragma unroll
  for (int j = 0; j < kHoist; ++j) {
    const int b = b_begin + j;
    if (b < b_end) {
      pre[j] = load_block<TYPE, true>(codes, tile * nblk + b, sub);
      pre_s[j] = loadf<true>(scales + (tile * nblk + b) * kTileRows + sub);
    }
  }
  // The chain lanes fetch their bias and (accumulating) old y now, so that
  // the store at the end does not wait for them.  y is this product's
  // output only, so reading it early is safe.
  float add = 0.0f, old = 0.0f;
  const bool owner = threadIdx.x < 16 && row < static_cast<std::size_t>(out);
  if (owner) {
    if (bias != nullptr) add = bias[row];
    if (accumulate) old = y[row];
  }
  stage_x(x, in, prologue, pw, eps, xs);
  float2* mine = reinterpret_cast<float2*>(pairs + r * stride);
#pragma unroll
  for (int j = 0; j < kHoist; ++j) {
    const int b = b_begin + j;
    if (b < b_end) {
      const float part = b < nfull ? full_block_dot<TYPE>(pre[j], xs + b * kBlock, k)
                                   : tail_block_dot<TYPE>(pre[j], xs + b * kBlock, in - b * kBlock);
      mine[b] = make_float2(part, pre_s[j]);
    }
  }
  for (int b = b_begin + kHoist; b < b_end; ++b) {
    const Block<TYPE> blk = load_block<TYPE, true>(codes, tile * nblk + b, sub);
    const float sc = loadf<true>(scales + (tile * nblk + b) * kTileRows + sub);
    const float part = b < nfull ? full_block_dot<TYPE>(blk, xs + b * kBlock, k)
                                 : tail_block_dot<TYPE>(blk, xs + b * kBlock, in - b * kBlock);
    mine[b] = make_float2(part, sc);
  }
  __syncthreads();
  if (owner) {
    const float v = chain_pairs(pairs + r * stride, nblk) + add;
    y[row] = accumulate ? old + v : v;
  }
}

// grid (ntiles, ceil(rows / R)).
template <int TYPE, int R>
__global__ void __launch_bounds__(1024) qgemv_tile(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                   const float* __restrict__ x, const float* __restrict__ bias,
                                                   float* __restrict__ y, int in, int nblk, int out, int rows, int bpw,
                                                   int accumulate) {
  extern __shared__ float lds[];
  const int r0 = blockIdx.y * R;
  const int nr = min(R, rows - r0);
  wide_tile<TYPE, R>(gmem(codes), gmem(scales), gmem(x + static_cast<std::size_t>(r0) * in), gmem(bias),
                     gmem_out(y + static_cast<std::size_t>(r0) * out), in, nblk, out, nr, bpw, accumulate, blockIdx.x,
                     lds);
}

template <int TYPE>
__global__ void __launch_bounds__(1024) qgemv_narrow(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                     const float* __restrict__ x, const float* __restrict__ bias,
                                                     float* __restrict__ y, int in, int nblk, int out, int bpg,
                                                     int accumulate) {
  extern __shared__ float4 lds4[];  // 16-byte aligned: the chains read float4
  narrow_tile<TYPE>(gmem(codes), gmem(scales), gmem(x), gmem(bias), gmem_out(y), in, nblk, out, bpg, accumulate,
                    blockIdx.x, reinterpret_cast<float*>(lds4));
}

// One launch over a group's products that share the weight type and the row
// chunk R (64-row tiles).  Workgroup w runs workgroup (w - first_wg) of
// problem wg_prob[w].
template <int TYPE, int R>
__global__ void __launch_bounds__(1024) qgemv_group(const GroupProblem* __restrict__ probs,
                                                    const std::uint32_t* __restrict__ wg_prob) {
  extern __shared__ float lds[];
  const int wg = blockIdx.x;
  // Uniform by construction; readfirstlane keeps the descriptor in SGPRs.
  const int idx = __builtin_amdgcn_readfirstlane(static_cast<int>(wg_prob[wg]));
  const GroupProblem p = probs[idx];
  const int local = wg - p.first_wg;
  const GMEM uint4* codes = gmem(reinterpret_cast<const uint4*>(p.codes));
  const GMEM float* scales = gmem(p.scales);
  const GMEM float* bias = gmem(p.bias);
  const int tile = local % p.ntiles;
  const int r0 = (local / p.ntiles) * R;
  const int nr = min(R, p.rows - r0);
  const GMEM float* x = gmem(p.x + static_cast<std::size_t>(r0) * p.in);
  GMEM float* y = gmem_out(p.y + static_cast<std::size_t>(r0) * p.out);
  wide_tile<TYPE, R>(codes, scales, x, bias, y, p.in, p.nblk, p.out, nr, p.bpw, p.accumulate, tile, lds);
}

// The 16-row tiles of a group (batch 1, optional prologue), in a kernel of
// their own so that their staging registers do not lower the occupancy of
// qgemv_group.
template <int TYPE>
__global__ void __launch_bounds__(1024) qgemv_group_narrow(const GroupProblem* __restrict__ probs,
                                                           const std::uint32_t* __restrict__ wg_prob) {
  extern __shared__ float4 lds4[];  // 16-byte aligned: the chains read float4
  const int wg = blockIdx.x;
  const int idx = __builtin_amdgcn_readfirstlane(static_cast<int>(wg_prob[wg]));
  const GroupProblem p = probs[idx];
  narrow_tile<TYPE>(gmem(reinterpret_cast<const uint4*>(p.codes)), gmem(p.scales), gmem(p.x), gmem(p.bias),
                    gmem_out(p.y), p.in, p.nblk, p.out, p.bpw, p.accumulate, wg - p.first_wg,
                    reinterpret_cast<float*>(lds4), p.prologue, gmem(p.pw), p.eps);
}

// The same 16-row tiles for a launch of at most kFewProblems products whose
// descriptors travel as kernel arguments: the kernel starts without the two
// dependent memory reads (workgroup -> product, then the product) of the
// table-driven launch, which sit in front of every load of the one-token
// step's short kernels.
constexpr int kFewProblems = 3;
struct FewProblems {
  GroupProblem p[kFewProblems];
  int count;
};
template <int TYPE>
__global__ void __launch_bounds__(1024) qgemv_few_narrow(FewProblems f) {
  extern __shared__ float4 lds4[];
  const int wg = blockIdx.x;
  // The product by comparisons (uniform), each field by selects, so the
  // argument block is never indexed dynamically.
  const int i = (f.count > 2 && wg >= f.p[2].first_wg) ? 2 : (f.count > 1 && wg >= f.p[1].first_wg) ? 1 : 0;
#define LLMI_PICK(fld) (i == 2 ? f.p[2].fld : i == 1 ? f.p[1].fld : f.p[0].fld)
  narrow_tile<TYPE>(gmem(reinterpret_cast<const uint4*>(LLMI_PICK(codes))), gmem(LLMI_PICK(scales)),
                    gmem(LLMI_PICK(x)), gmem(LLMI_PICK(bias)), gmem_out(LLMI_PICK(y)), LLMI_PICK(in), LLMI_PICK(nblk),
                    LLMI_PICK(out), LLMI_PICK(bpw), LLMI_PICK(accumulate), wg - LLMI_PICK(first_wg),
                    reinterpret_cast<float*>(lds4), LLMI_PICK(prologue), gmem(LLMI_PICK(pw)), LLMI_PICK(eps));
#undef LLMI_PICK
}

// One 16-row-tile product with its descriptor as scalar arguments, ordered
// so that what the first loads need (the weight pointers and shape, x and
// the prologue operand) is among the first 14 dwords, which arrive
// preloaded in SGPRs (-amdgpu-kernarg-preload-count); the one-token step's
// launches of one product take it.
template <int TYPE>
__global__ void __launch_bounds__(1024)
    qgemv_one_narrow(const uint4* __restrict__ codes, const float* __restrict__ scales, const float* __restrict__ x,
                     const float* __restrict__ pw, int nblk, int bpw, int in, int prologue, float eps, int out,
                     const float* __restrict__ bias, float* __restrict__ y, int accumulate) {
  extern __shared__ float4 lds4[];
  narrow_tile<TYPE>(gmem(codes), gmem(scales), gmem(x), gmem(bias), gmem_out(y), in, nblk, out, bpw, accumulate,
                    blockIdx.x, reinterpret_cast<float*>(lds4), prologue, gmem(pw), eps);
}

// The tolerance-mode one-token product split over K (SplitProduct):
// workgroup (tile, split), one wavefront, computes rows tile * 64 + lane over
// blocks [split * BPS, ...): the prologue's loads (the range's activations,
// and for RMSNorm the row's first batch of squares, for the combine the
// chunk partials) are issued first and the weights of all its blocks right
// after them -- loads complete in issue order, so the prologue then waits for
// its own data only and its arithmetic overlaps the weights' trip from HBM;
// the activations of its range are staged in LDS under the prologue, the
// block sums and the chain over its blocks are the exact kernels', and the
// partial sums go to y by atomic adds.
constexpr int kSplitMaxHeads = 8;  // kAttnCombine: whole heads per split (16 blocks of head_dim 64)
// What the first loads' addresses need comes first in the arguments: their
// first 14 dwords arrive preloaded in SGPRs.
template <int TYPE, int PRO, int BPS>
__global__ void __launch_bounds__(64) tsplit_gemv(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                  const float* __restrict__ x, const float* __restrict__ pw, int nblk,
                                                  int in, int out, int comb_hd, float eps, int comb_nch,
                                                  const float* __restrict__ bias, float* __restrict__ y,
                                                  float* __restrict__ zero, int nzero,
                                                  const int* __restrict__ npos_dev) {
  __shared__ __attribute__((aligned(16))) float xs[BPS * kBlock];
  __shared__ float wgt[PRO == kAttnCombine ? kSplitMaxHeads * kAttnMaxChunks : 1];
  const int lane = threadIdx.x;
  const int tile = blockIdx.x;
  const int b0 = blockIdx.y * BPS;
  const int nb = min(BPS, nblk - b0);
  const GMEM uint4* cg = gmem(codes);
  const GMEM float* sg = gmem(scales);
  Block<TYPE> blk[BPS];
  float sc[BPS];
  const auto load_weights = [&]() {
    __builtin_amdgcn_sched_barrier(0);  // the prologue's loads stay in front
#pragma unroll
    for (int j = 0; j < BPS; ++j) {
      // Past the range: the range's last block again (unused).
      const std::size_t slot = static_cast<std::size_t>(tile) * nblk + static_cast<std::size_t>(b0 + min(j, nb - 1));
      blk[j] = load_block<TYPE, true>(cg, slot, lane);
      sc[j] = loadf<true>(sg + slot * kTileRows + lane);
    }
  };
  // x' over the range [k0, k0 + n): each lane's elements (and, for
  // RMSNorm, its share of the whole row's squares) are loaded in batches
  // before any is used, so the staging costs one memory round trip per
  // batch rather than one per element.
  constexpr int kPer = (BPS * kBlock + 63) / 64;  // range elements per lane
  static_assert(kPer * 64 == BPS * kBlock, "every lane's slots lie inside xs");
  const int k0 = b0 * kBlock, n = min(nb * kBlock, in - k0);
  const GMEM float* xg = gmem(x);
  const GMEM float* pg = gmem(pw);
  // Every load is unconditional, from an index clamped into the row (a load
  // behind a per-lane condition becomes a branch, and the compiler may then
  // wait for it on the spot); values past the range are never stored.
  if constexpr (PRO == kRmsNorm || PRO == kSiluUp || PRO == kPlain) {
    float xv[kPer], pv[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = min(k0 + u * 64 + lane, in - 1);
      xv[u] = xg[i];
      if constexpr (PRO != kPlain) pv[u] = pg[i];
    }
    if constexpr (PRO == kRmsNorm) {
      // The row's squares in batches of kBatch per lane; the first batch's
      // loads go out before the weights'.
      constexpr int kBatch = 16;
      float v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int i = u * 64 + lane;
        const float t = xg[min(i, in - 1)];
        v[u] = i < in ? t : 0.0f;
      }
      load_weights();
      float ss = 0.0f;
#pragma unroll
      for (int u = 0; u < kBatch; ++u) ss = __builtin_fmaf(v[u], v[u], ss);
      for (int i0 = 64 * kBatch; i0 < in; i0 += 64 * kBatch) {
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
          const int i = i0 + u * 64 + lane;
          const float t = xg[min(i, in - 1)];
          v[u] = i < in ? t : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) ss = __builtin_fmaf(v[u], v[u], ss);
      }
      ss = wave_sum_dpp(ss);
      const float scale = 1.0f / __builtin_sqrtf(ss / static_cast<float>(in) + eps);
#pragma unroll
      for (int u = 0; u < kPer; ++u) xv[u] = pv[u] * (xv[u] * scale);
    } else {
      load_weights();
      if constexpr (PRO == kSiluUp) {
#pragma unroll
        for (int u = 0; u < kPer; ++u) xv[u] = xv[u] / (1.0f + __expf(-xv[u])) * pv[u];
      }
    }
    // Every slot is stored (xs holds kPer * 64 = BPS * kBlock floats; the
    // block sums read the first n), so no load is sunk behind a condition.
#pragma unroll
    for (int u = 0; u < kPer; ++u) xs[u * 64 + lane] = xv[u];
  } else {
    // kAttnCombine: the range is whole heads h0 .. h0 + nhh - 1; lanes 16r ..
    // 16r + 15 form the chunk weights of head hb + r.  Every chunk slot's
    // partials are loaded (slots past the step's chunks hold finite values
    // -- zeros or an earlier step's -- and get weight 0), so no load waits
    // for the chunk count, which a graph-replayed step reads from memory.
    // From a graph, comb_nch carries the run's chunk length and the count
    // follows from the positions (read after every load is issued).
    const int hd = comb_hd, nh_all = in / hd, h0 = k0 / hd, nhh = n / hd;
    const GMEM float* ms = xg + static_cast<std::size_t>(kAttnMaxChunks) * nh_all * hd;
    const GMEM float* ls = ms + kAttnMaxChunks * nh_all;
    float ov[kPer][kAttnMaxChunks];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = u * 64 + lane;
      const int hh = i / hd, d = i - hh * hd;
      const GMEM float* oh = xg + static_cast<std::size_t>(h0 + min(hh, nhh - 1)) * kAttnMaxChunks * hd + d;
#pragma unroll
      for (int c = 0; c < kAttnMaxChunks; ++c) ov[u][c] = oh[c * hd];  // a clamped head's for i >= n (unused)
    }
    // m and l of both groups of four heads (at most kSplitMaxHeads = 8),
    // then the weights.
    static_assert(kSplitMaxHeads <= 8, "two groups of four heads");
    float m_all[2], l_all[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int t = (h0 + min(4 * g + (lane >> 4), nhh - 1)) * kAttnMaxChunks + (lane & 15);
      m_all[g] = ms[t];
      l_all[g] = ls[t];
    }
    load_weights();
    if (npos_dev != nullptr) comb_nch = (__builtin_amdgcn_readfirstlane(*npos_dev) + comb_nch - 1) / comb_nch;
    // Both groups always (a lane whose head is past the range is not live
    // and stores nothing), so the loads above have a use on every path.
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int hb = 4 * g;
      const int hh = hb + (lane >> 4), c = lane & 15;
      const bool live = hh < nhh && c < comb_nch;
      const float mv = live ? m_all[g] : -__builtin_inff();
      const float lv = live ? l_all[g] : 0.0f;
      const float mx = row_last_bcast(row_max16_f32(mv), lane);
      const float w = live ? __expf(mv - mx) : 0.0f;
      const float den = row_last_bcast(row_sum16_f32(w * lv), lane);
      if (hh < nhh) wgt[hh * kAttnMaxChunks + c] = live ? w / den : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int i = u * 64 + lane;
      const float* wh = wgt + min(i / hd, nhh - 1) * kAttnMaxChunks;  // past n: a clamped head's (unused)
      float acc_c = 0.0f;
#pragma unroll
      for (int c = 0; c < kAttnMaxChunks; ++c) acc_c = __builtin_fmaf(wh[c], ov[u][c], acc_c);
      xs[i] = acc_c;
    }
  }
  __syncthreads();
  const Q4Magic k = q4_magic();
  const int nfull = in / kBlock - b0;  // whole blocks of the range
  float acc = 0.0f;
  if (nb == BPS && nfull >= BPS) {
    // A range of BPS whole blocks (uniform): no condition per block, so every
    // block's loads have a use on this path and none is sunk past the prologue.
#pragma unroll
    for (int j = 0; j < BPS; ++j) acc = __builtin_fmaf(full_block_dot<TYPE>(blk[j], xs + j * kBlock, k), sc[j], acc);
  } else {
#pragma unroll
    for (int j = 0; j < BPS; ++j) {
      if (j < nb) {
        const float part = j < nfull ? full_block_dot<TYPE>(blk[j], xs + j * kBlock, k)
                                     : tail_block_dot<TYPE>(blk[j], xs + j * kBlock, in - (b0 + j) * kBlock);
        acc = __builtin_fmaf(part, sc[j], acc);
      }
    }
  }
  const int row = tile * kTileRows + lane;
  if (row < out) {
    if (blockIdx.y == 0 && bias != nullptr) acc += bias[row];
    unsafeAtomicAdd(y + row, acc);
  }
  // Clearing the next product's output (a buffer this launch does not
  // read): last, so that its stores are not ahead of any load in the
  // counter the waits above use.
  if (zero != nullptr) {
    const int wg = static_cast<int>(blockIdx.y * gridDim.x + blockIdx.x);
    const int stride = static_cast<int>(gridDim.x * gridDim.y) * 64;
    for (int i = wg * 64 + lane; i < nzero; i += stride) zero[i] = 0.0f;
  }
}

// ------------------------------------------------------------ batch > 8
// The exact multi-row product on many tiles: one workgroup per MR = 64
// input rows x one 64-row tile of the matrix (64 outputs).  Per quantization
// block the workgroup stages the block's activations of its MR rows and the
// block's codes of its 64 outputs, converted to fp32 once, in LDS --
// transposed, [k][row] and [k][output], so one read gives a thread its 4
// rows (or 4 outputs) at one k -- plus the 64 scales; double-buffered: the
// next block's loads go to registers before this block's arithmetic and to
// LDS after it.  Thread (tr, to) holds the 4 x 4 chains of rows 4tr.. and
// outputs 4to..4to+3: part = fma(x[k], code[k], part) over the block's k in
// order, then acc = fma(part, scale, acc) -- the reference's chains, so y is
// bit-identical.  The final partial block runs only its len elements.
constexpr int kExactRows = 64;

template <int TYPE>
__global__ void __launch_bounds__(256) qgemm_exact(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                   const float* __restrict__ x, const float* __restrict__ bias,
                                                   float* __restrict__ y, int in, int nblk, int out, int rows,
                                                   int accumulate) {
  constexpr int MR = kExactRows;
  constexpr int RT = MR / 16;          // rows per thread
  constexpr int XS = MR + 4;           // LDS floats per k of the activations
  constexpr int CSTRIDE = kTileRows + 4;
  constexpr int XPT = MR * kBlock / 256;  // activations staged per thread
  __shared__ __attribute__((aligned(16))) float xs[2][kBlock * XS];
  __shared__ __attribute__((aligned(16))) float cs[2][kBlock * CSTRIDE];
  __shared__ float ss[2][kTileRows];
  const std::size_t tile = blockIdx.x;
  const int r0 = blockIdx.y * MR;
  const int tid = threadIdx.x;
  const int tr = tid >> 4, to = tid & 15;
  // Staging: activations of row xr, elements XPT*xq..+XPT-1 of the block;
  // codes of output cr (= lane of the tile), elements 8*cq..8*cq+7.
  // Addresses are clamped into x (rows past `rows`, and elements past `in`
  // of the final block, are never used), so no load sits behind a branch.
  const int xr = tid / (kBlock / XPT), xq = tid % (kBlock / XPT);
  const int cr = tid >> 2, cq = tid & 3;
  const float* xrow = x + static_cast<std::size_t>(min(r0 + xr, rows - 1)) * in;
  const GMEM uint4* cg = gmem(codes);
  struct Staged {
    float xv[XPT];
    Block<TYPE> blk;
    float sc;
  };
  const auto load = [&](Staged& st, int b) {
    const int k0 = b * kBlock + XPT * xq;
#pragma unroll
    for (int u = 0; u < XPT; ++u) st.xv[u] = xrow[min(k0 + u, in - 1)];
    st.blk = load_block<TYPE, false>(cg, tile * nblk + b, cr);
    st.sc = scales[(tile * nblk + b) * kTileRows + (tid & (kTileRows - 1))];
  };
  const auto store = [&](const Staged& st, int buf) {
    std::uint32_t w[8];
    unpack_words<TYPE>(st.blk, w);
#pragma unroll
    for (int u = 0; u < XPT; ++u) xs[buf][(XPT * xq + u) * XS + xr] = st.xv[u];
#pragma unroll
    for (int u = 0; u < 8; ++u) cs[buf][(8 * cq + u) * CSTRIDE + cr] = code_of<TYPE>(w, 8 * cq + u);
    if (tid < kTileRows) ss[buf][tid] = st.sc;
  };
  float acc[RT][4];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  // Two register sets carry the staged blocks two iterations ahead: set A
  // the odd blocks, set B the even ones past block 0.  Iteration b computes
  // block b from LDS, stores block b + 1 (loaded two iterations earlier)
  // into the other LDS buffer and loads block b + 3 into the set it freed,
  // so a block's global loads have two blocks of arithmetic to arrive.
  Staged A, B;
  load(B, 0);
  store(B, 0);
  if (nblk > 1) load(A, 1);
  if (nblk > 2) load(B, 2);
  __syncthreads();
  const auto iteration = [&](int b, Staged& next) {
    const int buf = b & 1;
    const int len = min(kBlock, in - b * kBlock);
    const float* xb = xs[buf] + RT * tr;
    const float* cb = cs[buf] + 4 * to;
    float part[RT][4];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) part[i][j] = 0.0f;
    const auto step = [&](int k) {
      const float4 xv = *reinterpret_cast<const float4*>(xb + k * XS);
      const float xa[RT] = {xv.x, xv.y, xv.z, xv.w};
      const float4 cv = *reinterpret_cast<const float4*>(cb + k * CSTRIDE);
      const float ca[4] = {cv.x, cv.y, cv.z, cv.w};
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) part[i][j] = __builtin_fmaf(xa[i], ca[j], part[i][j]);
    };
    if (len == kBlock) {
#pragma unroll 8
      for (int k = 0; k < kBlock; ++k) step(k);
    } else {
      for (int k = 0; k < len; ++k) step(k);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float sc = ss[buf][4 * to + j];
#pragma unroll
      for (int i = 0; i < RT; ++i) acc[i][j] = __builtin_fmaf(part[i][j], sc, acc[i][j]);
    }
    if (b + 1 < nblk) {
      store(next, buf ^ 1);
      if (b + 3 < nblk) load(next, b + 3);
    }
    __syncthreads();
  };
  for (int b = 0; b < nblk; b += 2) {
    iteration(b, A);
    if (b + 1 < nblk) iteration(b + 1, B);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const std::size_t o = tile * kTileRows + 4 * to + j;
    if (o >= static_cast<std::size_t>(out)) continue;
    const float add = bias != nullptr ? bias[o] : 0.0f;
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const int r = r0 + RT * tr + i;
      if (r < rows) {
        float* dst = y + static_cast<std::size_t>(r) * out + o;
        const float v = acc[i][j] + add;
        *dst = accumulate ? *dst + v : v;
      }
    }
  }
}

// qgemm_split (batch > 8, matrices with few 64-row tiles): one workgroup per
// (tile, chunk of kSplitRows input rows) whose kSplitWaves wavefronts take
// the tile's blocks round-robin, two per round each (W = kSplitWaves).  In
// each round wavefront w decodes blocks 2W * round + w and 2W * round + W + w
// once each (lane l: output tile*64 + l) and forms their block sums for
// every row of the chunk, with the activations read by scalar loads; the
// sums and scales go to LDS (two buffers, one barrier per round), and
// wavefront w then advances the chains of rows w, w + W over the round's 2W
// blocks in order: acc = fma(part, scale, acc).  (Two blocks per round
// halve the barriers: Qwen2.5's down_proj at 512 rows 109 -> 102 us.)
// The block sums are the reference's per-block chains and the chain over
// blocks runs in block order, so y is bit-identical; splitting the blocks
// fills the GPU where a 64-row tile per row chunk gives too few workgroups.
// Small row chunks (2 or 4 rows) measured fastest: the chunk's activations
// are scalar loads per block and row, and more workgroups hide them.
template <int TYPE, int kSplitRows, int kSplitWaves, class Epi>
__device__ __forceinline__ void split_tile(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                           const float* __restrict__ x, const float* __restrict__ bias, int in,
                                           int nblk, int out, int rows, std::size_t tile, int chunk, const Epi& epi) {
  constexpr int RW = (kSplitRows + kSplitWaves - 1) / kSplitWaves;  // chains per lane
  __shared__ float part[2][kSplitRows][2 * kSplitWaves][kTileRows];
  __shared__ float scl[2][2 * kSplitWaves][kTileRows];
  const int r0 = chunk * kSplitRows;
  const int nr = min(kSplitRows, rows - r0);
  const int lane = threadIdx.x & (kTileRows - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const GMEM uint4* cg = gmem(codes);
  const GMEM float* sg = gmem(scales);
  const GMEM float* xg = gmem(x) + static_cast<std::size_t>(r0) * in;
  const int nfull = in / kBlock;
  const std::size_t base = tile * nblk;
  float acc[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) acc[i] = 0.0f;
  const int nround = (nblk + 2 * kSplitWaves - 1) / (2 * kSplitWaves);
  Block<TYPE> cur[2]{};
  float cur_s[2] = {0.0f, 0.0f};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int bb = h * kSplitWaves + wave;
    if (bb < nblk) {
      cur[h] = load_block<TYPE, false>(cg, base + bb, lane);
      cur_s[h] = sg[(base + bb) * kTileRows + lane];
    }
  }
  for (int rd = 0; rd < nround; ++rd) {
    const int buf = rd & 1;
    Block<TYPE> nxt[2]{};
    float nxt_s[2] = {0.0f, 0.0f};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int bn = (rd + 1) * 2 * kSplitWaves + h * kSplitWaves + wave;
      if (bn < nblk) {
        nxt[h] = load_block<TYPE, false>(cg, base + bn, lane);
        nxt_s[h] = sg[(base + bn) * kTileRows + lane];
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int b = rd * 2 * kSplitWaves + h * kSplitWaves + wave;
      const int j = h * kSplitWaves + wave;
      if (b < nfull) {
        float c[kBlock];
        block_codes<TYPE>(cur[h], c);
#pragma unroll
        for (int r = 0; r < kSplitRows; ++r)
          if (r < nr) part[buf][r][j][lane] = codes_dot(c, xg + static_cast<std::size_t>(r) * in + b * kBlock);
      } else if (b < nblk) {
        for (int r = 0; r < nr; ++r)
          part[buf][r][j][lane] =
              tail_block_dot<TYPE>(cur[h], xg + static_cast<std::size_t>(r) * in + b * kBlock, in - b * kBlock);
      }
      if (b < nblk) scl[buf][j][lane] = cur_s[h];
    }
    __syncthreads();
    const int nb = min(2 * kSplitWaves, nblk - rd * 2 * kSplitWaves);
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      const int r = wave + kSplitWaves * i;
      if (r < kSplitRows && r < nr) {
        float a = acc[i];
        for (int j = 0; j < nb; ++j) a = __builtin_fmaf(part[buf][r][j][lane], scl[buf][j][lane], a);
        acc[i] = a;
      }
    }
    cur[0] = nxt[0];
    cur[1] = nxt[1];
    cur_s[0] = nxt_s[0];
    cur_s[1] = nxt_s[1];
  }
  // The epilogue runs on whole wavefronts (row conditions are per wavefront),
  // so it may exchange values between the lanes of a row.
  const std::size_t o = tile * kTileRows + lane;
  const bool o_ok = o < static_cast<std::size_t>(out);
  const float add = bias != nullptr && o_ok ? bias[o] : 0.0f;
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const int r = wave + kSplitWaves * i;
    if (r < kSplitRows && r < nr) epi(r0 + r, o, o_ok, acc[i] + add);
  }
}

// y[row][o] = v (or += v).
struct StoreOut {
  float* y;
  int out, accumulate;
  __device__ __forceinline__ void operator()(int row, std::size_t o, bool o_ok, float v) const {
    if (!o_ok) return;
    float* dst = y + static_cast<std::size_t>(row) * out + o;
    *dst = accumulate ? *dst + v : v;
  }
};

template <int TYPE, int R, int W>
__global__ void __launch_bounds__(W * 64) qgemm_split(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                      const float* __restrict__ x, const float* __restrict__ bias,
                                                      float* __restrict__ y, int in, int nblk, int out, int rows,
                                                      int accumulate) {
  split_tile<TYPE, R, W>(codes, scales, x, bias, in, nblk, out, rows, blockIdx.x, blockIdx.y,
                         StoreOut{y, out, accumulate});
}

// The gate and up projections of an MLP in one split-block tile: each round
// a wavefront decodes block b of the gate matrix and forms its block sums for
// every input row, then the same for the up matrix, the chains run side by
// side, and the epilogue writes
// silu(gate) * up as the reference's MLP does after its two matmuls
// (kernels.cpp:148, transformer.cpp:288-290): v = gate + 0.0f (the matmul's
// absent bias), v / (1 + expf(-v)) * (up + 0.0f), with the exact expf.
template <int TYPE, int kSplitRows, int kSplitWaves>
__global__ void __launch_bounds__(kSplitWaves * 64) qgemm_split_gate_up(
    const uint4* __restrict__ codes_g, const float* __restrict__ scales_g, const uint4* __restrict__ codes_u,
    const float* __restrict__ scales_u, const float* __restrict__ x, float* __restrict__ y, int in, int nblk, int out,
    int rows) {
  constexpr int RW = (kSplitRows + kSplitWaves - 1) / kSplitWaves;  // chains per lane and product
  __shared__ float part[2][2][kSplitRows][kSplitWaves][kTileRows];  // [buffer][gate, up]
  __shared__ float scl[2][2][kSplitWaves][kTileRows];
  const std::size_t tile = blockIdx.x;
  const int r0 = blockIdx.y * kSplitRows;
  const int nr = min(kSplitRows, rows - r0);
  const int lane = threadIdx.x & (kTileRows - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const GMEM uint4* cgg = gmem(codes_g);
  const GMEM uint4* cgu = gmem(codes_u);
  const GMEM float* sgg = gmem(scales_g);
  const GMEM float* sgu = gmem(scales_u);
  const GMEM float* xg = gmem(x) + static_cast<std::size_t>(r0) * in;
  const int nfull = in / kBlock;
  const std::size_t base = tile * nblk;
  float acc_g[RW], acc_u[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) acc_g[i] = acc_u[i] = 0.0f;
  const int nround = (nblk + kSplitWaves - 1) / kSplitWaves;
  Block<TYPE> cur_g{}, cur_u{};
  float sc_g = 0.0f, sc_u = 0.0f;
  if (wave < nblk) {
    cur_g = load_block<TYPE, false>(cgg, base + wave, lane);
    cur_u = load_block<TYPE, false>(cgu, base + wave, lane);
    sc_g = sgg[(base + wave) * kTileRows + lane];
    sc_u = sgu[(base + wave) * kTileRows + lane];
  }
  for (int rd = 0; rd < nround; ++rd) {
    const int buf = rd & 1;
    const int b = rd * kSplitWaves + wave;
    Block<TYPE> nxt_g{}, nxt_u{};
    float nsc_g = 0.0f, nsc_u = 0.0f;
    if (b + kSplitWaves < nblk) {
      nxt_g = load_block<TYPE, false>(cgg, base + b + kSplitWaves, lane);
      nxt_u = load_block<TYPE, false>(cgu, base + b + kSplitWaves, lane);
      nsc_g = sgg[(base + b + kSplitWaves) * kTileRows + lane];
      nsc_u = sgu[(base + b + kSplitWaves) * kTileRows + lane];
    }
    if (b < nfull) {
      // One product's block at a time: a single set of 32 decoded codes
      // stays live, which keeps the kernel at the split kernel's occupancy.
      {
        float c[kBlock];
        block_codes<TYPE>(cur_g, c);
#pragma unroll
        for (int r = 0; r < kSplitRows; ++r)
          if (r < nr) part[buf][0][r][wave][lane] = codes_dot(c, xg + static_cast<std::size_t>(r) * in + b * kBlock);
      }
      __builtin_amdgcn_sched_barrier(0);
      {
        float c[kBlock];
        block_codes<TYPE>(cur_u, c);
#pragma unroll
        for (int r = 0; r < kSplitRows; ++r)
          if (r < nr) part[buf][1][r][wave][lane] = codes_dot(c, xg + static_cast<std::size_t>(r) * in + b * kBlock);
      }
    } else if (b < nblk) {
      for (int r = 0; r < nr; ++r) {
        const GMEM float* xr = xg + static_cast<std::size_t>(r) * in + b * kBlock;
        part[buf][0][r][wave][lane] = tail_block_dot<TYPE>(cur_g, xr, in - b * kBlock);
        part[buf][1][r][wave][lane] = tail_block_dot<TYPE>(cur_u, xr, in - b * kBlock);
      }
    }
    if (b < nblk) {
      scl[buf][0][wave][lane] = sc_g;
      scl[buf][1][wave][lane] = sc_u;
    }
    __syncthreads();
    const int nb = min(kSplitWaves, nblk - rd * kSplitWaves);
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      const int r = wave + kSplitWaves * i;
      if (r < kSplitRows && r < nr) {
        float ag = acc_g[i], au = acc_u[i];
        for (int j = 0; j < nb; ++j) {
          ag = __builtin_fmaf(part[buf][0][r][j][lane], scl[buf][0][j][lane], ag);
          au = __builtin_fmaf(part[buf][1][r][j][lane], scl[buf][1][j][lane], au);
        }
        acc_g[i] = ag;
        acc_u[i] = au;
      }
    }
    cur_g = nxt_g;
    cur_u = nxt_u;
    sc_g = nsc_g;
    sc_u = nsc_u;
  }
  const std::size_t o = tile * kTileRows + lane;
  if (o < static_cast<std::size_t>(out)) {
#pragma unroll
    for (int i = 0; i < RW; ++i) {
      const int r = wave + kSplitWaves * i;
      if (r < kSplitRows && r < nr) {
        const float v = acc_g[i] + 0.0f;
        const float u = acc_u[i] + 0.0f;
        y[static_cast<std::size_t>(r0 + r) * out + o] = v / (1.0f + exact::expf(-v)) * u;
      }
    }
  }
}

// Up to kMaxShared products of one weight type and input size that share x
// and rows (the prefill's q/k/v, gate/up) in one launch: workgroup column
// blockIdx.x is tile blockIdx.x - tile_end[p - 1] of the product p whose
// tile range holds it.
constexpr int kMaxShared = 3;
struct SplitGroup {
  const uint4* codes[kMaxShared];
  const float* scales[kMaxShared];
  const float* bias[kMaxShared];
  float* y[kMaxShared];
  int out[kMaxShared];
  int tile_end[kMaxShared];
  int mode[kMaxShared];  // a SharedEpilogue
  int count;
  RopeCache rope;
};

// A product's output in a grouped launch: y as computed, RoPE'd in place (q),
// RoPE'd into the KV cache (k), or copied into it (v).  The RoPE modes take a
// head size of 64, one head per 64-output tile, and rotate elements (i, i+32)
// of a head with the host tables: v[i] = fma(a, c, -(b * s)),
// v[i + 32] = fma(b, c, a * s) (kernels.cpp:122-134).
struct GroupStore {
  const SplitGroup& g;
  int p;
  __device__ __forceinline__ void operator()(int row, std::size_t o, bool o_ok, float v) const {
    const int mode = g.mode[p];
    if (mode == kStorePlain) {
      if (o_ok) g.y[p][static_cast<std::size_t>(row) * g.out[p] + o] = v;
      return;
    }
    const int lane = static_cast<int>(o & 63);
    const int pos = g.rope.base + row;
    if (mode != kStoreCache) {
      const float partner = __shfl_xor(v, 32, 64);
      const float c = g.rope.cos_t[static_cast<std::size_t>(pos) * 32 + (lane & 31)];
      const float sn = g.rope.sin_t[static_cast<std::size_t>(pos) * 32 + (lane & 31)];
      v = lane < 32 ? __builtin_fmaf(v, c, -(partner * sn)) : __builtin_fmaf(v, c, partner * sn);
    }
    if (!o_ok) return;
    if (mode == kStoreRope) {
      g.y[p][static_cast<std::size_t>(row) * g.out[p] + o] = v;
    } else {
      const std::size_t head = o >> 6;
      g.y[p][(head * g.rope.cap + pos) * 64 + lane] = v;
    }
  }
};

template <int TYPE, int R, int W>
__global__ void __launch_bounds__(W * 64) qgemm_split_group(SplitGroup g, const float* __restrict__ x, int in,
                                                            int nblk, int rows) {
  const int t = static_cast<int>(blockIdx.x);
  int p = 0;
  while (p + 1 < g.count && t >= g.tile_end[p]) ++p;
  const int t0 = p == 0 ? 0 : g.tile_end[p - 1];
  split_tile<TYPE, R, W>(g.codes[p], g.scales[p], x, g.bias[p], in, nblk, g.out[p], rows,
                         static_cast<std::size_t>(t - t0), blockIdx.y, GroupStore{g, p});
}

// ------------------------------------------------------------ planning
// LDS bytes of one workgroup of each kind.
// part[nr][nblk][64], scale[nblk][64], then the chain's look-ahead padding.
std::size_t wide_lds(std::size_t nblk, std::size_t nr) {
  return ((nr + 1) * nblk + 2 * kChainRound) * kTileRows * sizeof(float);
}
// x[in (padded to 4)], 16 rows of pairs, then chain_pairs' look-ahead padding.
std::size_t narrow_lds(std::size_t in, std::size_t nblk) {
  return (((in + 3) & ~std::size_t{3}) + 16 * static_cast<std::size_t>(pair_stride(static_cast<int>(nblk))) +
          kPairPad) *
         sizeof(float);
}

// LDS a wide workgroup aims to stay within, so that several workgroups share
// a CU; longer rows may use up to the per-workgroup maximum.
constexpr std::size_t kLdsTarget = 64 * 1024;

// Row chunk R (a template size: 1, 2, 4, 8) of a wide workgroup: the
// smallest one covering `rows`, halved until its LDS fits `budget`; 0 if not
// even one row fits.
int pick_chunk(std::size_t rows, std::size_t nblk, std::size_t budget) {
  const int want = rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : 8;
  for (int r = want; r >= 1; r /= 2)
    if (wide_lds(nblk, std::min<std::size_t>(rows, r)) <= budget) return r;
  return 0;
}

// Wavefronts per 64-row tile: each takes about kBlocksPerWave blocks (4 for
// Q4_0, 2 for Q8_0: about 4 KB of codes and scales in flight per
// wavefront), at most 16.  Measured on MI355X over the 151936x896 lm_head.
int wide_waves(std::size_t nblk, int type) {
  const std::size_t per = type == LLMI_TYPE_Q8_0 ? 2 : 4;
  return static_cast<int>(std::clamp<std::size_t>(ceil_div(nblk, per), 1, 16));
}

// Wavefronts of a 16-row tile: about two blocks per lane group (4 groups per
// wavefront), at most 64 groups.
int narrow_waves(std::size_t nblk) {
  constexpr std::size_t kBlocksPerGroup = 2;
  const std::size_t groups = std::clamp<std::size_t>(ceil_div(nblk, kBlocksPerGroup), 1, 64);
  return static_cast<int>(ceil_div(groups, 4));
}

struct TilePlan {
  int kind = 0;  // 0: qgemm_exact; GroupProblem::kNarrow; or the row chunk R of qgemv_tile
  int waves = 1;
  int bpw = 1;
  std::size_t lds = 0;
};

// Launch shape of a single product.  Batch 1 matrices with fewer than
// kNarrowTiles 64-row tiles use 16-row tiles (more workgroups); otherwise
// the wide tile.
TilePlan plan_single(const DeviceMatrix& m, std::size_t rows) {
  constexpr std::size_t kNarrowTiles = 128;
  const std::size_t nblk = std::max<std::size_t>(m.nblk, 1);
  TilePlan p;
  if (rows > 8) return p;  // qgemm_exact
  if (rows == 1 && m.ntiles < kNarrowTiles && narrow_lds(m.in, nblk) <= max_lds_per_block()) {
    p.kind = GroupProblem::kNarrow;
    p.waves = narrow_waves(nblk);
    p.bpw = static_cast<int>(ceil_div(nblk, static_cast<std::size_t>(p.waves) * 4));
    p.lds = narrow_lds(m.in, nblk);
    return p;
  }
  int r = pick_chunk(rows, nblk, kLdsTarget);
  if (r == 0) r = pick_chunk(1, nblk, max_lds_per_block());
  if (r == 0) return p;  // rows too long for LDS staging: qgemm_exact
  p.kind = r;
  p.bpw = static_cast<int>(ceil_div(nblk, wide_waves(nblk, m.type)));
  p.waves = static_cast<int>(ceil_div(nblk, p.bpw));
  p.lds = wide_lds(nblk, std::min<std::size_t>(rows, r));
  return p;
}

template <int TYPE, int R>
void launch_tile(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y, int acc,
                 const TilePlan& p, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(m.ntiles), static_cast<unsigned>(ceil_div(rows, R)));
  qgemv_tile<TYPE, R><<<grid, static_cast<unsigned>(p.waves * 64), p.lds, s>>>(
      reinterpret_cast<const uint4*>(m.codes), m.scales, x, bias, y, static_cast<int>(m.in), static_cast<int>(m.nblk),
      static_cast<int>(m.out), static_cast<int>(rows), p.bpw, acc);
}

template <int TYPE, int R, int W>
void launch_split(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y, int acc,
                  hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(m.ntiles), static_cast<unsigned>(ceil_div(rows, R)));
  qgemm_split<TYPE, R, W><<<grid, W * 64, 0, s>>>(reinterpret_cast<const uint4*>(m.codes), m.scales, x, bias, y,
                                                  static_cast<int>(m.in), static_cast<int>(m.nblk),
                                                  static_cast<int>(m.out), static_cast<int>(rows), acc);
}

// Multi-row products.  qgemm_exact when its 64-row chunks alone give about
// 1024 workgroups (an lm_head over every position); otherwise qgemm_split
// with the row chunk and wavefront count measured fastest on MI355X for the
// launch's size: 4 rows x 4 wavefronts from ~6K wavefronts up, 4 x 8 from
// ~4K, else 2 x 8 (SmolLM2-135M and Qwen2.5-0.5B projections at 128 and 512
// rows; Qwen2.5's gate/up 92 us split against 109 on qgemm_exact, its
// 151936-row lm_head 2.46 ms split against 2.14).
template <int TYPE>
void launch_rows(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y, int acc,
                 hipStream_t s) {
  constexpr std::size_t kExactMin = 1024;
  if (m.ntiles * ceil_div(rows, kExactRows) >= kExactMin) {
    const dim3 grid(static_cast<unsigned>(m.ntiles), static_cast<unsigned>(ceil_div(rows, kExactRows)));
    qgemm_exact<TYPE><<<grid, 256, 0, s>>>(reinterpret_cast<const uint4*>(m.codes), m.scales, x, bias, y,
                                           static_cast<int>(m.in), static_cast<int>(m.nblk), static_cast<int>(m.out),
                                           static_cast<int>(rows), acc);
    return;
  }
  // Here ntiles * ceil(rows / 64) < 1024, so rows < 65536 and every split
  // launch's grid y (ceil(rows / R), R >= 2) stays below 32768.
  const auto waves = [&](std::size_t r, std::size_t w) { return m.ntiles * ceil_div(rows, r) * w; };
  if (waves(4, 4) >= 6144) launch_split<TYPE, 4, 4>(m, x, rows, bias, y, acc, s);
  else if (waves(4, 8) >= 4096) launch_split<TYPE, 4, 8>(m, x, rows, bias, y, acc, s);
  else launch_split<TYPE, 2, 8>(m, x, rows, bias, y, acc, s);
}

template <int TYPE, int R, int W>
void launch_split_group(const SplitGroup& g, std::size_t tiles, const float* x, std::size_t in, std::size_t nblk,
                        std::size_t rows, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(ceil_div(rows, R)));
  qgemm_split_group<TYPE, R, W><<<grid, W * 64, 0, s>>>(g, x, static_cast<int>(in), static_cast<int>(nblk),
                                                        static_cast<int>(rows));
}

// The grouped split launch of launch_matmul_shared: the row chunk and
// wavefront count by the launch's total size, as for one product.
template <int TYPE>
void launch_group_rows(const SplitGroup& g, std::size_t tiles, const float* x, std::size_t in, std::size_t nblk,
                       std::size_t rows, hipStream_t s) {
  const auto waves = [&](std::size_t r, std::size_t w) { return tiles * ceil_div(rows, r) * w; };
  if (waves(4, 4) >= 6144) launch_split_group<TYPE, 4, 4>(g, tiles, x, in, nblk, rows, s);
  else if (waves(4, 8) >= 4096) launch_split_group<TYPE, 4, 8>(g, tiles, x, in, nblk, rows, s);
  else launch_split_group<TYPE, 2, 8>(g, tiles, x, in, nblk, rows, s);
}

template <int TYPE>
void launch_typed(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y, int acc,
                  hipStream_t s) {
  const TilePlan p = plan_single(m, rows);
  switch (p.kind) {
    case 0: launch_rows<TYPE>(m, x, rows, bias, y, acc, s); break;
    case GroupProblem::kNarrow:
      qgemv_narrow<TYPE><<<static_cast<unsigned>(ceil_div(m.out, 16)), static_cast<unsigned>(p.waves * 64), p.lds, s>>>(
          reinterpret_cast<const uint4*>(m.codes), m.scales, x, bias, y, static_cast<int>(m.in),
          static_cast<int>(m.nblk), static_cast<int>(m.out), p.bpw, acc);
      break;
    case 1: launch_tile<TYPE, 1>(m, x, rows, bias, y, acc, p, s); break;
    case 2: launch_tile<TYPE, 2>(m, x, rows, bias, y, acc, p, s); break;
    case 4: launch_tile<TYPE, 4>(m, x, rows, bias, y, acc, p, s); break;
    default: launch_tile<TYPE, 8>(m, x, rows, bias, y, acc, p, s); break;
  }
}

int check_shape(const DeviceMatrix& m, std::size_t rows) {
  LLMI_REQUIRE(m.in > 0, "matmul: in must be positive");
  LLMI_REQUIRE(m.in <= 0x7FFFFFFFu && m.out <= 0x7FFFFFFFu, "matmul: shape too large");
  LLMI_REQUIRE(ceil_div(rows, 8) <= 65535, "matmul: too many input rows for one launch");
  return LLMI_OK;
}

}  // namespace

int launch_matmul(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y, hipStream_t s,
                  bool accumulate) {
  if (rows == 0 || m.out == 0) return LLMI_OK;
  if (m.type == LLMI_TYPE_F32) {
    LLMI_REQUIRE(x != nullptr && y != nullptr, "matmul: null pointer");
    return launch_matmul_f32(m, x, rows, bias, y, s, accumulate);
  }
  if (int rc = check_shape(m, rows)) return rc;
  LLMI_REQUIRE(x != nullptr && y != nullptr, "matmul: null pointer");
  const int acc = accumulate ? 1 : 0;
  if (m.type == LLMI_TYPE_Q8_0) launch_typed<LLMI_TYPE_Q8_0>(m, x, rows, bias, y, acc, s);
  else launch_typed<LLMI_TYPE_Q4_0>(m, x, rows, bias, y, acc, s);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int launch_gate_up_silu(const DeviceMatrix& gate, const DeviceMatrix& up, const float* x, std::size_t rows,
                        float* y, hipStream_t s, bool* fused) {
  *fused = false;
  if (rows <= 8 || gate.type == LLMI_TYPE_F32 || gate.type != up.type || gate.in != up.in || gate.out != up.out ||
      gate.out == 0 || gate.ntiles * ceil_div(rows, kExactRows) >= 1024)
    return LLMI_OK;
  if (int rc = check_shape(gate, rows)) return rc;
  LLMI_REQUIRE(x != nullptr && y != nullptr, "gate_up: null pointer");
  const auto waves = [&](std::size_t r, std::size_t w) { return gate.ntiles * ceil_div(rows, r) * w; };
  const auto launch = [&](auto tag_r, auto tag_w) {
    constexpr int R = decltype(tag_r)::value, W = decltype(tag_w)::value;
    const dim3 grid(static_cast<unsigned>(gate.ntiles), static_cast<unsigned>(ceil_div(rows, R)));
    const int in = static_cast<int>(gate.in), nblk = static_cast<int>(gate.nblk), out = static_cast<int>(gate.out);
    const int nr = static_cast<int>(rows);
    const auto* cg = reinterpret_cast<const uint4*>(gate.codes);
    const auto* cu = reinterpret_cast<const uint4*>(up.codes);
    if (gate.type == LLMI_TYPE_Q8_0)
      qgemm_split_gate_up<LLMI_TYPE_Q8_0, R, W><<<grid, W * 64, 0, s>>>(cg, gate.scales, cu, up.scales, x, y, in, nblk,
                                                                        out, nr);
    else
      qgemm_split_gate_up<LLMI_TYPE_Q4_0, R, W><<<grid, W * 64, 0, s>>>(cg, gate.scales, cu, up.scales, x, y, in, nblk,
                                                                        out, nr);
  };
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  using I8 = std::integral_constant<int, 8>;
  if (waves(4, 4) >= 6144) launch(I4{}, I4{});
  else if (waves(4, 8) >= 4096) launch(I4{}, I8{});
  else launch(I2{}, I8{});
  LLMI_TRY_HIP(hipGetLastError());
  *fused = true;
  return LLMI_OK;
}

int launch_matmul_shared(const DeviceMatrix* const* ms, const float* const* biases, float* const* ys, int count,
                         const float* x, std::size_t rows, hipStream_t s, const RopeCache* rope, bool* roped) {
  if (roped != nullptr) *roped = false;
  LLMI_REQUIRE(count >= 1 && count <= kMaxShared, "matmul_shared: 1..3 products");
  std::size_t tiles = 0;
  bool grouped = count > 1 && rows > 8;
  for (int i = 0; i < count && grouped; ++i) {
    const DeviceMatrix& m = *ms[i];
    // One launch only where each product alone would take qgemm_split.
    grouped = m.type != LLMI_TYPE_F32 && m.type == ms[0]->type && m.in == ms[0]->in && m.out > 0 &&
              m.ntiles * ceil_div(rows, kExactRows) < 1024;
    tiles += m.ntiles;
  }
  if (!grouped) {
    for (int i = 0; i < count; ++i)
      if (int rc = launch_matmul(*ms[i], x, rows, biases[i], ys[i], s)) return rc;
    return LLMI_OK;
  }
  if (int rc = check_shape(*ms[0], rows)) return rc;
  LLMI_REQUIRE(x != nullptr, "matmul_shared: null x");
  SplitGroup g{};
  int end = 0;
  for (int i = 0; i < count; ++i) {
    LLMI_REQUIRE(ys[i] != nullptr, "matmul_shared: null y");
    g.codes[i] = reinterpret_cast<const uint4*>(ms[i]->codes);
    g.scales[i] = ms[i]->scales;
    g.bias[i] = biases[i];
    g.y[i] = ys[i];
    g.out[i] = static_cast<int>(ms[i]->out);
    end += static_cast<int>(ms[i]->ntiles);
    g.tile_end[i] = end;
    g.mode[i] = kStorePlain;
  }
  g.count = count;
  // RoPE and the cache writes ride along for q, k, v of head size 64.
  if (rope != nullptr && roped != nullptr && count == 3 && ms[0]->out % 64 == 0 && ms[1]->out % 64 == 0 &&
      ms[2]->out % 64 == 0) {
    g.rope = *rope;
    g.mode[0] = kStoreRope;
    g.mode[1] = kStoreRopeCache;
    g.mode[2] = kStoreCache;
    g.y[1] = rope->kc;
    g.y[2] = rope->vc;
    *roped = true;
  }
  const DeviceMatrix& m0 = *ms[0];
  if (m0.type == LLMI_TYPE_Q8_0) launch_group_rows<LLMI_TYPE_Q8_0>(g, tiles, x, m0.in, m0.nblk, rows, s);
  else launch_group_rows<LLMI_TYPE_Q4_0>(g, tiles, x, m0.in, m0.nblk, rows, s);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int plan_group(const GroupEntry* entries, std::size_t count, GroupPlan* plan) {
  // Narrow 16-row tiles for batch-1 products only when the 64-row tiles would
  // leave the GPU mostly idle (fewer than ~4 workgroups per CU), and for long
  // rows (more than kNarrowMaxBlocks blocks) only below one 64-row workgroup
  // per CU: 24 Qwen2.5 down_proj matrices (896 x 4864, 336 64-row tiles) in
  // one launch stream about twice as fast on 64-row tiles, one alone (14
  // tiles) about 1.6x faster on 16-row tiles (measured on MI355X).  A
  // prologue always needs them.
  constexpr std::size_t kNarrowBelow = 1024;
  constexpr std::size_t kNarrowMaxBlocks = 64;
  constexpr std::size_t kLongRowsNarrowBelow = 256;
  *plan = GroupPlan{};
  std::size_t wide_total = 0;
  for (std::size_t i = 0; i < count; ++i) {
    const GroupEntry& e = entries[i];
    LLMI_REQUIRE(e.m != nullptr, "group: null weight");
    LLMI_REQUIRE(e.m->type != LLMI_TYPE_F32, "group: fp32 weights are not part of grouped launches");
    LLMI_REQUIRE(e.rows >= 1 && e.rows <= 8, "group: each product takes 1..8 input rows");
    LLMI_REQUIRE(e.x != nullptr && e.y != nullptr, "group: null x or y");
    if (int rc = check_shape(*e.m, e.rows)) return rc;
    wide_total += e.m->ntiles * ceil_div(e.rows, 8);
  }
  // Products are launched by weight type and row chunk R (one kernel
  // instance each).
  for (int type : {LLMI_TYPE_Q8_0, LLMI_TYPE_Q4_0})
  for (int R : {int{GroupProblem::kNarrow}, 1, 2, 4, 8}) {
    std::vector<GroupProblem> probs;
    std::size_t biggest = 0;
    int waves = 1;
    for (std::size_t i = 0; i < count; ++i) {
      const GroupEntry& e = entries[i];
      const DeviceMatrix& m = *e.m;
      if (m.out == 0) continue;
      const bool fits = narrow_lds(m.in, m.nblk) <= max_lds_per_block();
      const bool narrow =
          e.rows == 1 && fits &&
          (e.prologue != kPlain ||
           (wide_total < kNarrowBelow && (m.nblk <= kNarrowMaxBlocks || wide_total < kLongRowsNarrowBelow)));
      LLMI_REQUIRE(e.prologue == kPlain || narrow, "group: a prologue needs batch 1 and in <= ~20k");
      LLMI_REQUIRE(e.prologue == kPlain || e.prologue == kRmsNorm || e.prologue == kSiluUp,
                   "group: unknown prologue");
      int r = narrow ? int{GroupProblem::kNarrow} : pick_chunk(e.rows, m.nblk, kLdsTarget);
      if (r == 0) r = pick_chunk(1, m.nblk, max_lds_per_block());
      LLMI_REQUIRE(r != 0, "group: rows too long for the grouped GEMV (in above ~10k)");
      if (r != R || m.type != type) continue;
      GroupProblem p{};
      p.codes = m.codes;
      p.scales = m.scales;
      p.x = e.x;
      p.bias = e.bias;
      p.y = e.y;
      p.type = m.type;
      p.kind = r;
      p.in = static_cast<int>(m.in);
      p.nblk = static_cast<int>(m.nblk);
      p.out = static_cast<int>(m.out);
      p.rows = static_cast<int>(e.rows);
      p.ntiles = static_cast<int>(m.ntiles);
      p.accumulate = e.accumulate ? 1 : 0;
      p.prologue = e.prologue;
      p.pw = e.pw;
      p.eps = e.eps;
      probs.push_back(p);
      // The launch's wavefront count: the most any 16-row tile wants, or
      // what the largest product wants for 64-row tiles.
      const std::size_t bytes = m.code_bytes + m.scale_bytes;
      if (narrow) {
        waves = std::max(waves, narrow_waves(m.nblk));
      } else if (bytes > biggest) {
        biggest = bytes;
        waves = wide_waves(m.nblk, m.type);
      }
    }
    if (probs.empty()) continue;
    // Longest workgroups first (most blocks per tile): they start while the
    // short ones fill the GPU around them, and the launch ends on short
    // workgroups.  (Qwen2.5's 24 MLP layers in one launch: 61% / 81% of HBM
    // peak for Q4_0 / Q8_0 against 50% / 71% in layer order.)
    std::stable_sort(probs.begin(), probs.end(),
                     [](const GroupProblem& a, const GroupProblem& b) { return a.nblk > b.nblk; });
    GroupLaunch l;
    l.type = type;
    l.rchunk = R;
    l.waves = waves;
    l.prob_offset = plan->probs.size();
    l.map_offset = plan->wg_prob.size();
    std::size_t wg = 0;
    for (std::size_t j = 0; j < probs.size(); ++j) {
      GroupProblem& p = probs[j];
      std::size_t wgs = 0, need = 0;
      if (p.kind == GroupProblem::kNarrow) {
        p.bpw = static_cast<int>(ceil_div(p.nblk, static_cast<std::size_t>(waves) * 4));
        wgs = ceil_div(p.out, 16);
        need = narrow_lds(p.in, p.nblk);
      } else {
        p.bpw = static_cast<int>(ceil_div(p.nblk, waves));
        wgs = static_cast<std::size_t>(p.ntiles) * ceil_div(p.rows, R);
        need = wide_lds(p.nblk, std::min(p.rows, R));
      }
      p.first_wg = static_cast<int>(wg);
      wg += wgs;
      LLMI_REQUIRE(wg <= 0x7FFFFFFFu, "group: too many workgroups");
      l.lds = std::max(l.lds, need);
      plan->wg_prob.insert(plan->wg_prob.end(), wgs, static_cast<std::uint32_t>(j));
    }
    LLMI_REQUIRE(l.lds <= max_lds_per_block(), "group: a product needs more LDS than one workgroup may use");
    l.total_wgs = static_cast<int>(wg);
    l.nprob = static_cast<int>(probs.size());
    plan->probs.insert(plan->probs.end(), probs.begin(), probs.end());
    plan->launches.push_back(l);
  }
  return LLMI_OK;
}

int launch_group(const GroupProblem* probs_dev, const std::uint32_t* map_dev, const GroupLaunch& l, hipStream_t s) {
  if (l.total_wgs == 0) return LLMI_OK;
  const dim3 grid(static_cast<unsigned>(l.total_wgs)), block(static_cast<unsigned>(l.waves * 64));
  const GroupProblem* probs = probs_dev + l.prob_offset;
  const std::uint32_t* map = map_dev + l.map_offset;
  if (l.rchunk == GroupProblem::kNarrow) {
    if (l.type == LLMI_TYPE_Q8_0) qgemv_group_narrow<LLMI_TYPE_Q8_0><<<grid, block, l.lds, s>>>(probs, map);
    else qgemv_group_narrow<LLMI_TYPE_Q4_0><<<grid, block, l.lds, s>>>(probs, map);
  } else if (l.type == LLMI_TYPE_Q8_0) {
    switch (l.rchunk) {
      case 1: qgemv_group<LLMI_TYPE_Q8_0, 1><<<grid, block, l.lds, s>>>(probs, map); break;
      case 2: qgemv_group<LLMI_TYPE_Q8_0, 2><<<grid, block, l.lds, s>>>(probs, map); break;
      case 4: qgemv_group<LLMI_TYPE_Q8_0, 4><<<grid, block, l.lds, s>>>(probs, map); break;
      default: qgemv_group<LLMI_TYPE_Q8_0, 8><<<grid, block, l.lds, s>>>(probs, map); break;
    }
  } else {
    switch (l.rchunk) {
      case 1: qgemv_group<LLMI_TYPE_Q4_0, 1><<<grid, block, l.lds, s>>>(probs, map); break;
      case 2: qgemv_group<LLMI_TYPE_Q4_0, 2><<<grid, block, l.lds, s>>>(probs, map); break;
      case 4: qgemv_group<LLMI_TYPE_Q4_0, 4><<<grid, block, l.lds, s>>>(probs, map); break;
      default: qgemv_group<LLMI_TYPE_Q4_0, 8><<<grid, block, l.lds, s>>>(probs, map); break;
    }
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int DeviceGroup::build(const GroupEntry* entries, std::size_t count) {
  release();
  GroupPlan plan;
  if (int rc = plan_group(entries, count, &plan)) return rc;
  launches = plan.launches;
  host_probs = plan.probs;
  const std::size_t pbytes = plan.probs.size() * sizeof(GroupProblem);
  const std::size_t mbytes = plan.wg_prob.size() * sizeof(std::uint32_t);
  if (pbytes + mbytes == 0) return LLMI_OK;
  LLMI_TRY_HIP(hipMalloc(&table, pbytes + mbytes));
  auto* base = static_cast<std::uint8_t*>(table);
  LLMI_TRY_HIP(hipMemcpy(base, plan.probs.data(), pbytes, hipMemcpyHostToDevice));
  if (mbytes > 0) LLMI_TRY_HIP(hipMemcpy(base + pbytes, plan.wg_prob.data(), mbytes, hipMemcpyHostToDevice));
  probs = reinterpret_cast<const GroupProblem*>(base);
  map = reinterpret_cast<const std::uint32_t*>(base + pbytes);
  return LLMI_OK;
}

int DeviceGroup::launch(hipStream_t s) const {
  for (const GroupLaunch& l : launches) {
    if (l.rchunk == GroupProblem::kNarrow && l.nprob >= 1 && l.nprob <= kFewProblems && l.total_wgs > 0) {
      // Few products: descriptors by value (qgemv_few_narrow).
      FewProblems f{};
      f.count = l.nprob;
      for (int k = 0; k < l.nprob; ++k) f.p[k] = host_probs[l.prob_offset + static_cast<std::size_t>(k)];
      const dim3 grid(static_cast<unsigned>(l.total_wgs)), block(static_cast<unsigned>(l.waves * 64));
      if (l.nprob == 1) {
        // One product: scalar arguments (preloaded), qgemv_one_narrow.
        const GroupProblem& p = f.p[0];
        const auto* codes = reinterpret_cast<const uint4*>(p.codes);
#define LLMI_ONE_ARGS \
  codes, p.scales, p.x, p.pw, p.nblk, p.bpw, p.in, p.prologue, p.eps, p.out, p.bias, p.y, p.accumulate
        if (l.type == LLMI_TYPE_Q8_0) {
          qgemv_one_narrow<LLMI_TYPE_Q8_0><<<grid, block, l.lds, s>>>(LLMI_ONE_ARGS);
        } else {
          qgemv_one_narrow<LLMI_TYPE_Q4_0><<<grid, block, l.lds, s>>>(LLMI_ONE_ARGS);
        }
#undef LLMI_ONE_ARGS
        LLMI_TRY_HIP(hipGetLastError());
        continue;
      }
      if (l.type == LLMI_TYPE_Q8_0) {
        qgemv_few_narrow<LLMI_TYPE_Q8_0><<<grid, block, l.lds, s>>>(f);
      } else {
        qgemv_few_narrow<LLMI_TYPE_Q4_0><<<grid, block, l.lds, s>>>(f);
      }
      LLMI_TRY_HIP(hipGetLastError());
      continue;
    }
    if (int rc = launch_group(probs, map, l, s)) return rc;
  }
  return LLMI_OK;
}

// Splits of a SplitProduct: about kSplitTarget workgroups, BPS (the
// kernel's blocks per split) one of 2, 4, 8, 16, and the power of two is
// taken below max(nblk / (kSplitTarget / tiles), nblk / kSplitMaxPerOutput):
// the atomic adds into one cache line of y are applied one after another
// (152 per output cost ~3 us more than plain stores on MI355X), so long rows
// take wider splits.
constexpr int kSplitTarget = 1024;
constexpr int kSplitMaxPerOutput = 40;

int plan_split(SplitProduct* p) {
  LLMI_REQUIRE(p->m != nullptr && p->x != nullptr && p->y != nullptr, "split product: null operand");
  const DeviceMatrix& m = *p->m;
  LLMI_REQUIRE(m.type == LLMI_TYPE_Q8_0 || m.type == LLMI_TYPE_Q4_0, "split product: Q8_0 or Q4_0 weights only");
  LLMI_REQUIRE(p->prologue == kRmsNorm || p->prologue == kSiluUp || p->prologue == kAttnCombine ||
                   p->prologue == kPlain,
               "split product: unknown prologue");
  LLMI_REQUIRE(p->prologue == kPlain || p->pw != nullptr, "split product: null prologue operand");
  const int nblk = static_cast<int>(m.nblk), ntiles = static_cast<int>(m.ntiles);
  LLMI_REQUIRE(nblk >= 1 && ntiles >= 1, "split product: empty matrix");
  const int want = std::max(1, kSplitTarget / ntiles);
  int bps = static_cast<int>(ceil_div(static_cast<std::size_t>(nblk), static_cast<std::size_t>(want)));
  bps = std::max(bps, static_cast<int>(ceil_div(static_cast<std::size_t>(nblk),
                                                static_cast<std::size_t>(kSplitMaxPerOutput))));
  int unit = 1;
  if (p->prologue == kAttnCombine) {
    LLMI_REQUIRE(p->comb_hd >= 32 && p->comb_hd % kBlock == 0 && m.in % static_cast<std::size_t>(p->comb_hd) == 0,
                 "split product: an attention-combine product needs in = heads * head_dim, head_dim % 32 == 0");
    unit = p->comb_hd / kBlock;
  }
  int pick = 2;
  while (pick < 16 && (2 * pick <= bps || pick % unit != 0)) pick *= 2;
  LLMI_REQUIRE(pick % unit == 0 && (p->prologue != kAttnCombine || pick * kBlock / p->comb_hd <= kSplitMaxHeads),
               "split product: head_dim too large for a split");
  p->bps = pick;
  p->splits = static_cast<int>(ceil_div(static_cast<std::size_t>(nblk), static_cast<std::size_t>(pick)));
  return LLMI_OK;
}

namespace {

template <int TYPE, int PRO>
void launch_split_bps(const SplitProduct& p, hipStream_t s, int comb_nch, const int* npos_dev) {
  const DeviceMatrix& m = *p.m;
  const dim3 grid(static_cast<unsigned>(m.ntiles), static_cast<unsigned>(p.splits));
#define LLMI_SPLIT_ARGS                                                                                            \
  reinterpret_cast<const uint4*>(m.codes), m.scales, p.x, p.pw, static_cast<int>(m.nblk), static_cast<int>(m.in), \
      static_cast<int>(m.out), p.comb_hd, p.eps, comb_nch, p.bias, p.y, p.zero, p.nzero, npos_dev
  switch (p.bps) {
    case 2: tsplit_gemv<TYPE, PRO, 2><<<grid, 64, 0, s>>>(LLMI_SPLIT_ARGS); break;
    case 4: tsplit_gemv<TYPE, PRO, 4><<<grid, 64, 0, s>>>(LLMI_SPLIT_ARGS); break;
    case 8: tsplit_gemv<TYPE, PRO, 8><<<grid, 64, 0, s>>>(LLMI_SPLIT_ARGS); break;
    default: tsplit_gemv<TYPE, PRO, 16><<<grid, 64, 0, s>>>(LLMI_SPLIT_ARGS); break;
  }
#undef LLMI_SPLIT_ARGS
}

template <int TYPE>
void launch_split_type(const SplitProduct& p, hipStream_t s, int comb_nch, const int* npos_dev) {
  switch (p.prologue) {
    case kRmsNorm: launch_split_bps<TYPE, kRmsNorm>(p, s, comb_nch, nullptr); break;
    case kSiluUp: launch_split_bps<TYPE, kSiluUp>(p, s, comb_nch, nullptr); break;
    case kAttnCombine: launch_split_bps<TYPE, kAttnCombine>(p, s, comb_nch, npos_dev); break;
    default: launch_split_bps<TYPE, kPlain>(p, s, comb_nch, nullptr); break;
  }
}

}  // namespace

int launch_split(const SplitProduct& p, hipStream_t s, int comb_nch, const int* npos_dev) {
  LLMI_REQUIRE(p.m != nullptr && p.splits >= 1 && (p.bps == 2 || p.bps == 4 || p.bps == 8 || p.bps == 16),
               "split product: not planned");
  LLMI_REQUIRE(p.prologue != kAttnCombine || npos_dev != nullptr || (comb_nch >= 1 && comb_nch <= kAttnMaxChunks),
               "split product: attention chunks out of range");
  if (p.m->type == LLMI_TYPE_Q8_0) launch_split_type<LLMI_TYPE_Q8_0>(p, s, comb_nch, npos_dev);
  else launch_split_type<LLMI_TYPE_Q4_0>(p, s, comb_nch, npos_dev);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

void DeviceGroup::release() {
  if (table != nullptr) (void)hipFree(table);
  table = nullptr;
  probs = nullptr;
  map = nullptr;
  launches.clear();
  host_probs.clear();
}

}  // namespace llmi_hip
