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
// qgemv_group: a fixed list of products (each batch 1..8) as one launch; each
// workgroup runs one tile of one problem with the same tile functions.
//
// qgemv_rows (batch > 8, the exact prefill path): one wavefront per tile
// walks all blocks in order with the chains in registers.
#include <algorithm>
#include <vector>

#include "common.hpp"

namespace llmi_hip {

namespace {

// Signed bit-field extract (v_bfe_i32).  The builtin is declared with an
// unsigned result, so the value is reinterpreted as int before any
// conversion to float.
__device__ __forceinline__ int sfield(std::uint32_t w, int offset, int width) {
  return static_cast<int>(__builtin_amdgcn_sbfe(w, offset, width));
}

template <int TYPE>
struct Block {
  static constexpr int kU = TYPE == LLMI_TYPE_Q8_0 ? 2 : 1;  // 16-byte loads per lane per block
  uint4 c[kU];
};

template <int TYPE>
__device__ __forceinline__ Block<TYPE> load_block(const uint4* __restrict__ codes, std::size_t slot, int lane) {
  Block<TYPE> b;
#pragma unroll
  for (int u = 0; u < Block<TYPE>::kU; ++u) b.c[u] = codes[(slot * Block<TYPE>::kU + u) * kTileRows + lane];
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

// Block sum of one full block: part = fma(x[i], code[i], part), i = 0..31.
template <int TYPE>
__device__ __forceinline__ float full_block_dot(const std::uint32_t* w, const float* __restrict__ xr) {
  float part = 0.0f;
#pragma unroll
  for (int i = 0; i < kBlock; ++i) part = __builtin_fmaf(xr[i], code_of<TYPE>(w, i), part);
  return part;
}

// Block sum of the final partial block (len < 32 elements).
template <int TYPE>
__device__ __noinline__ float tail_block_dot(const Block<TYPE> blk, const float* __restrict__ xr, int len) {
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
__device__ __forceinline__ void block_sums(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                           const float* __restrict__ x, std::size_t tile, int in, int nblk, int nr,
                                           int b_begin, int b_end, int lane, float* part, float* scl) {
  const int nfull = in / kBlock;
  const int f_end = min(b_end, nfull);
  const std::size_t base = tile * nblk;
  Block<TYPE> cur[CH];
  float cur_s[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    if (b_begin + j < f_end) {
      cur[j] = load_block<TYPE>(codes, base + b_begin + j, lane);
      cur_s[j] = scales[(base + b_begin + j) * kTileRows + lane];
    }
  }
  for (int b = b_begin; b < f_end; b += CH) {
    Block<TYPE> nxt[CH];
    float nxt_s[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (b + CH + j < f_end) {
        nxt[j] = load_block<TYPE>(codes, base + b + CH + j, lane);
        nxt_s[j] = scales[(base + b + CH + j) * kTileRows + lane];
      }
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (b + j < f_end) {
        std::uint32_t w[8];
        unpack_words<TYPE>(cur[j], w);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r < nr)
            part[(r * nblk + b + j) * kTileRows + lane] =
                full_block_dot<TYPE>(w, x + static_cast<std::size_t>(r) * in + (b + j) * kBlock);
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
    const Block<TYPE> blk = load_block<TYPE>(codes, base + nfull, lane);
    for (int r = 0; r < nr; ++r)
      part[(r * nblk + nfull) * kTileRows + lane] =
          tail_block_dot<TYPE>(blk, x + static_cast<std::size_t>(r) * in + nfull * kBlock, in - nfull * kBlock);
    scl[nfull * kTileRows + lane] = scales[(base + nfull) * kTileRows + lane];
  }
}

// The sequential chain over all blocks of one row of a tile, from LDS
// (stride `stride` floats between blocks).
__device__ __forceinline__ float chain_lds(const float* part, const float* scl, int nblk, int lane, int stride) {
  float acc = 0.0f;
  int b = 0;
  for (; b + 4 <= nblk; b += 4) {
    const float p0 = part[(b + 0) * stride + lane], s0 = scl[(b + 0) * stride + lane];
    const float p1 = part[(b + 1) * stride + lane], s1 = scl[(b + 1) * stride + lane];
    const float p2 = part[(b + 2) * stride + lane], s2 = scl[(b + 2) * stride + lane];
    const float p3 = part[(b + 3) * stride + lane], s3 = scl[(b + 3) * stride + lane];
    acc = __builtin_fmaf(p0, s0, acc);
    acc = __builtin_fmaf(p1, s1, acc);
    acc = __builtin_fmaf(p2, s2, acc);
    acc = __builtin_fmaf(p3, s3, acc);
  }
  for (; b < nblk; ++b) acc = __builtin_fmaf(part[b * stride + lane], scl[b * stride + lane], acc);
  return acc;
}

__device__ __forceinline__ void store_out(float* __restrict__ y, std::size_t o, float v, int accumulate) {
  y[o] = accumulate ? y[o] + v : v;
}

// One 64-row tile for input rows [0, nr), nr <= R (x, y already point at the
// chunk's first row).  The workgroup's wavefronts split the blocks, bpw
// each, and park block sums and scales in LDS (part[nr][nblk][64] then
// scale[nblk][64]); wavefront w then runs the chains of rows w, w + W, ...
// Every thread of the workgroup must call it (it has a barrier).
template <int TYPE, int R, int CH>
__device__ __forceinline__ void wide_tile(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                          const float* __restrict__ x, const float* __restrict__ bias,
                                          float* __restrict__ y, int in, int nblk, int out, int nr, int bpw,
                                          int accumulate, std::size_t tile, float* lds) {
  float* part = lds;
  float* scl = lds + static_cast<std::size_t>(nr) * nblk * kTileRows;
  const int lane = threadIdx.x & (kTileRows - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int b_begin = wave * bpw;
  const int b_end = min(nblk, b_begin + bpw);
  block_sums<TYPE, R, CH>(codes, scales, x, tile, in, nblk, nr, b_begin, b_end, lane, part, scl);
  __syncthreads();
  const std::size_t o = tile * kTileRows + lane;
  for (int r = wave; r < nr; r += nwaves) {
    const float acc = chain_lds(part + static_cast<std::size_t>(r) * nblk * kTileRows, scl, nblk, lane, kTileRows);
    if (o < static_cast<std::size_t>(out))
      store_out(y + static_cast<std::size_t>(r) * out, o, acc + (bias != nullptr ? bias[o] : 0.0f), accumulate);
  }
}

// One 16-row tile (batch 1), for matrices with few rows.  Lane l of a
// wavefront owns row tile16*16 + (l & 15) and one of 4 block groups (l >> 4);
// the W wavefronts give 4W groups of bpg contiguous blocks.  The 16 rows of
// one block are a contiguous 256-byte piece of the 64-row layout, so loads
// stay coalesced.  The activations are staged in LDS once and read with
// broadcast loads (16 lanes per address); block sums and scales go to LDS,
// and lanes 0-15 run the chain.  LDS: x[in (padded to 4)], part[nblk][16],
// scale[nblk][16].
template <int TYPE>
__device__ __forceinline__ void narrow_tile(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                            const float* __restrict__ x, const float* __restrict__ bias,
                                            float* __restrict__ y, int in, int nblk, int out, int bpg, int accumulate,
                                            std::size_t tile16, float* lds) {
  float* xs = lds;
  float* part = lds + ((in + 3) & ~3);
  float* scl = part + nblk * 16;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int group = (threadIdx.x >> 6) * 4 + (lane >> 4);
  const std::size_t row = tile16 * 16 + r;
  const std::size_t tile = row / kTileRows;
  const int sub = static_cast<int>(row % kTileRows);
  for (int i = threadIdx.x; i < in; i += blockDim.x) xs[i] = x[i];
  __syncthreads();
  const int nfull = in / kBlock;
  const int b_begin = group * bpg;
  const int b_end = min(nblk, b_begin + bpg);
  for (int b = b_begin; b < b_end; ++b) {
    const Block<TYPE> blk = load_block<TYPE>(codes, tile * nblk + b, sub);
    const float sc = scales[(tile * nblk + b) * kTileRows + sub];
    std::uint32_t w[8];
    unpack_words<TYPE>(blk, w);
    float p;
    if (b < nfull) {
      p = full_block_dot<TYPE>(w, xs + b * kBlock);
    } else {
      p = 0.0f;
      const int len = in - b * kBlock;
      for (int i = 0; i < len; ++i) p = __builtin_fmaf(xs[b * kBlock + i], code_of<TYPE>(w, i), p);
    }
    part[b * 16 + r] = p;
    scl[b * 16 + r] = sc;
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const float acc = chain_lds(part, scl, nblk, r, 16);
    if (row < static_cast<std::size_t>(out)) store_out(y, row, acc + (bias != nullptr ? bias[row] : 0.0f), accumulate);
  }
}

constexpr int chunk_for(int type) { return type == LLMI_TYPE_Q8_0 ? 2 : 4; }

// grid (ntiles, ceil(rows / R)).
template <int TYPE, int R>
__global__ void __launch_bounds__(1024) qgemv_tile(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                   const float* __restrict__ x, const float* __restrict__ bias,
                                                   float* __restrict__ y, int in, int nblk, int out, int rows, int bpw,
                                                   int accumulate) {
  extern __shared__ float lds[];
  const int r0 = blockIdx.y * R;
  const int nr = min(R, rows - r0);
  wide_tile<TYPE, R, chunk_for(TYPE)>(codes, scales, x + static_cast<std::size_t>(r0) * in, bias,
                                      y + static_cast<std::size_t>(r0) * out, in, nblk, out, nr, bpw, accumulate,
                                      blockIdx.x, lds);
}

template <int TYPE>
__global__ void __launch_bounds__(1024) qgemv_narrow(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                     const float* __restrict__ x, const float* __restrict__ bias,
                                                     float* __restrict__ y, int in, int nblk, int out, int bpg,
                                                     int accumulate) {
  extern __shared__ float lds[];
  narrow_tile<TYPE>(codes, scales, x, bias, y, in, nblk, out, bpg, accumulate, blockIdx.x, lds);
}

// Workgroup w runs workgroup (w - first_wg) of the problem whose range holds
// w, found by binary search over the table (sorted by first_wg).
__global__ void __launch_bounds__(kGroupThreads) qgemv_group(const GroupProblem* __restrict__ probs, int nprob) {
  extern __shared__ float lds[];
  const int wg = blockIdx.x;
  int lo = 0, hi = nprob - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (probs[mid].first_wg <= wg) lo = mid;
    else hi = mid - 1;
  }
  const GroupProblem p = probs[lo];
  const int local = wg - p.first_wg;
  const uint4* codes = reinterpret_cast<const uint4*>(p.codes);
  if (p.kind == GroupProblem::kNarrow) {
    if (p.type == LLMI_TYPE_Q8_0)
      narrow_tile<LLMI_TYPE_Q8_0>(codes, p.scales, p.x, p.bias, p.y, p.in, p.nblk, p.out, p.bpw, p.accumulate, local, lds);
    else
      narrow_tile<LLMI_TYPE_Q4_0>(codes, p.scales, p.x, p.bias, p.y, p.in, p.nblk, p.out, p.bpw, p.accumulate, local, lds);
    return;
  }
  const int tile = local % p.ntiles;
  const int r0 = (local / p.ntiles) * p.kind;
  const int nr = min(p.kind, p.rows - r0);
  const float* x = p.x + static_cast<std::size_t>(r0) * p.in;
  float* y = p.y + static_cast<std::size_t>(r0) * p.out;
#define LLMI_GROUP_WIDE(T, RR)                                                                                  \
  wide_tile<T, RR, chunk_for(T)>(codes, p.scales, x, p.bias, y, p.in, p.nblk, p.out, nr, p.bpw, p.accumulate, \
                                 tile, lds)
  if (p.type == LLMI_TYPE_Q8_0) {
    switch (p.kind) {
      case 1: LLMI_GROUP_WIDE(LLMI_TYPE_Q8_0, 1); break;
      case 2: LLMI_GROUP_WIDE(LLMI_TYPE_Q8_0, 2); break;
      case 4: LLMI_GROUP_WIDE(LLMI_TYPE_Q8_0, 4); break;
      default: LLMI_GROUP_WIDE(LLMI_TYPE_Q8_0, 8); break;
    }
  } else {
    switch (p.kind) {
      case 1: LLMI_GROUP_WIDE(LLMI_TYPE_Q4_0, 1); break;
      case 2: LLMI_GROUP_WIDE(LLMI_TYPE_Q4_0, 2); break;
      case 4: LLMI_GROUP_WIDE(LLMI_TYPE_Q4_0, 4); break;
      default: LLMI_GROUP_WIDE(LLMI_TYPE_Q4_0, 8); break;
    }
  }
#undef LLMI_GROUP_WIDE
}

// ------------------------------------------------------------ batch > 8
// One wavefront per tile (4 tiles per 256-thread workgroup), R input rows
// per workgroup row (grid.y), chains in registers.
template <int TYPE, int R, int CH>
__global__ void __launch_bounds__(256) qgemv_rows(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                  const float* __restrict__ x, const float* __restrict__ bias,
                                                  float* __restrict__ y, int in, int nblk, int out, int rows,
                                                  int ntiles, int accumulate) {
  const int lane = threadIdx.x & (kTileRows - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const std::size_t tile = static_cast<std::size_t>(blockIdx.x) * 4 + wave;
  if (tile >= static_cast<std::size_t>(ntiles)) return;
  const int r0 = blockIdx.y * R;
  const int nr = min(R, rows - r0);
  const int nfull = in / kBlock;
  const float* xb = x + static_cast<std::size_t>(r0) * in;

  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;

  Block<TYPE> cur[CH];
  float cur_s[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    if (j < nfull) {
      cur[j] = load_block<TYPE>(codes, tile * nblk + j, lane);
      cur_s[j] = scales[(tile * nblk + j) * kTileRows + lane];
    }
  }
  for (int b = 0; b < nfull; b += CH) {
    Block<TYPE> nxt[CH];
    float nxt_s[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (b + CH + j < nfull) {
        nxt[j] = load_block<TYPE>(codes, tile * nblk + b + CH + j, lane);
        nxt_s[j] = scales[(tile * nblk + b + CH + j) * kTileRows + lane];
      }
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (b + j < nfull) {
        std::uint32_t w[8];
        unpack_words<TYPE>(cur[j], w);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (r < nr) {
            const float p = full_block_dot<TYPE>(w, xb + static_cast<std::size_t>(r) * in + (b + j) * kBlock);
            acc[r] = __builtin_fmaf(p, cur_s[j], acc[r]);
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      cur[j] = nxt[j];
      cur_s[j] = nxt_s[j];
    }
  }
  if (nfull < nblk) {
    const Block<TYPE> blk = load_block<TYPE>(codes, tile * nblk + nfull, lane);
    const float s = scales[(tile * nblk + nfull) * kTileRows + lane];
    for (int r = 0; r < nr; ++r) {
      const float p = tail_block_dot<TYPE>(blk, xb + static_cast<std::size_t>(r) * in + nfull * kBlock, in - nfull * kBlock);
#pragma unroll
      for (int rr = 0; rr < R; ++rr)
        if (rr == r) acc[rr] = __builtin_fmaf(p, s, acc[rr]);
    }
  }
  const std::size_t o = tile * kTileRows + lane;
  if (o < static_cast<std::size_t>(out)) {
    const float add = bias != nullptr ? bias[o] : 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (r < nr) {
        float* dst = y + static_cast<std::size_t>(r0 + r) * out + o;
        const float v = acc[r] + add;
        *dst = accumulate ? *dst + v : v;
      }
    }
  }
}

// ------------------------------------------------------------ planning
// LDS bytes of one workgroup of each kind.
std::size_t wide_lds(std::size_t nblk, std::size_t nr) { return (nr + 1) * nblk * kTileRows * sizeof(float); }
std::size_t narrow_lds(std::size_t in, std::size_t nblk) { return (((in + 3) & ~std::size_t{3}) + 2 * nblk * 16) * sizeof(float); }

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

struct TilePlan {
  int kind = 0;  // 0: qgemv_rows; GroupProblem::kNarrow; or the row chunk R of qgemv_tile
  int waves = 1;
  int bpw = 1;
  std::size_t lds = 0;
};

// Launch shape of a single product.  Batch 1 matrices with fewer than
// kNarrowTiles 64-row tiles use 16-row tiles; otherwise the wide tile with
// enough wavefronts per workgroup to put ~kTargetWaves in the grid.
TilePlan plan_single(const DeviceMatrix& m, std::size_t rows) {
  constexpr std::size_t kTargetWaves = 8192;
  constexpr std::size_t kNarrowTiles = 128;
  constexpr std::size_t kBlocksPerGroup = 2;
  const std::size_t nblk = std::max<std::size_t>(m.nblk, 1);
  TilePlan p;
  if (rows > 8) return p;  // qgemv_rows
  if (rows == 1 && m.ntiles < kNarrowTiles && narrow_lds(m.in, nblk) <= max_lds_per_block()) {
    p.kind = GroupProblem::kNarrow;
    const std::size_t groups = std::min<std::size_t>(64, ceil_div(nblk, kBlocksPerGroup));
    p.waves = static_cast<int>(ceil_div(groups, 4));
    p.bpw = static_cast<int>(ceil_div(nblk, static_cast<std::size_t>(p.waves) * 4));
    p.lds = narrow_lds(m.in, nblk);
    return p;
  }
  int r = pick_chunk(rows, nblk, kLdsTarget);
  if (r == 0) r = pick_chunk(1, nblk, max_lds_per_block());
  if (r == 0) return p;  // rows too long for LDS staging: qgemv_rows
  const std::size_t wgs = m.ntiles * ceil_div(rows, r);
  const std::size_t per_wg = std::max<std::size_t>(1, ceil_div(kTargetWaves, wgs));
  const std::size_t waves = std::max<std::size_t>(1, std::min<std::size_t>({16, nblk, per_wg}));
  p.kind = r;
  p.bpw = static_cast<int>(ceil_div(nblk, waves));
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

template <int TYPE>
void launch_rows(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y, int acc,
                 hipStream_t s) {
  constexpr int R = 8, CH = TYPE == LLMI_TYPE_Q8_0 ? 2 : 4;
  const dim3 grid(static_cast<unsigned>(ceil_div(m.ntiles, 4)), static_cast<unsigned>(ceil_div(rows, R)));
  qgemv_rows<TYPE, R, CH><<<grid, 256, 0, s>>>(reinterpret_cast<const uint4*>(m.codes), m.scales, x, bias, y,
                                               static_cast<int>(m.in), static_cast<int>(m.nblk),
                                               static_cast<int>(m.out), static_cast<int>(rows),
                                               static_cast<int>(m.ntiles), acc);
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
  if (int rc = check_shape(m, rows)) return rc;
  LLMI_REQUIRE(x != nullptr && y != nullptr, "matmul: null pointer");
  const int acc = accumulate ? 1 : 0;
  if (m.type == LLMI_TYPE_Q8_0) launch_typed<LLMI_TYPE_Q8_0>(m, x, rows, bias, y, acc, s);
  else launch_typed<LLMI_TYPE_Q4_0>(m, x, rows, bias, y, acc, s);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int plan_group(const GroupEntry* entries, std::size_t count, std::vector<GroupProblem>* probs, int* total_wgs,
               std::size_t* lds) {
  constexpr std::size_t kWaves = kGroupThreads / 64;
  // Narrow 16-row tiles only when the wide tiles would leave the GPU mostly
  // idle (fewer than ~4 workgroups per CU).
  constexpr std::size_t kNarrowBelow = 1024;
  std::size_t wide_total = 0;
  for (std::size_t i = 0; i < count; ++i) {
    const GroupEntry& e = entries[i];
    LLMI_REQUIRE(e.m != nullptr, "group: null weight");
    LLMI_REQUIRE(e.rows >= 1 && e.rows <= 8, "group: each product takes 1..8 input rows");
    LLMI_REQUIRE(e.x != nullptr && e.y != nullptr, "group: null x or y");
    if (int rc = check_shape(*e.m, e.rows)) return rc;
    wide_total += e.m->ntiles * ceil_div(e.rows, 8);
  }
  probs->clear();
  std::size_t wg = 0, max_lds = 0;
  for (std::size_t i = 0; i < count; ++i) {
    const GroupEntry& e = entries[i];
    const DeviceMatrix& m = *e.m;
    if (m.out == 0) continue;
    GroupProblem p{};
    p.codes = m.codes;
    p.scales = m.scales;
    p.x = e.x;
    p.bias = e.bias;
    p.y = e.y;
    p.type = m.type;
    p.in = static_cast<int>(m.in);
    p.nblk = static_cast<int>(m.nblk);
    p.out = static_cast<int>(m.out);
    p.rows = static_cast<int>(e.rows);
    p.ntiles = static_cast<int>(m.ntiles);
    p.accumulate = e.accumulate ? 1 : 0;
    std::size_t wgs = 0, need = 0;
    if (e.rows == 1 && wide_total < kNarrowBelow && narrow_lds(m.in, m.nblk) <= max_lds_per_block()) {
      p.kind = GroupProblem::kNarrow;
      p.bpw = static_cast<int>(ceil_div(m.nblk, kWaves * 4));
      wgs = ceil_div(m.out, 16);
      need = narrow_lds(m.in, m.nblk);
    } else {
      int r = pick_chunk(e.rows, m.nblk, kLdsTarget);
      if (r == 0) r = pick_chunk(1, m.nblk, max_lds_per_block());
      LLMI_REQUIRE(r != 0, "group: rows too long for the grouped GEMV (in above ~10k)");
      p.kind = r;
      p.bpw = static_cast<int>(ceil_div(m.nblk, kWaves));
      wgs = m.ntiles * ceil_div(e.rows, r);
      need = wide_lds(m.nblk, std::min<std::size_t>(e.rows, r));
    }
    p.first_wg = static_cast<int>(wg);
    wg += wgs;
    LLMI_REQUIRE(wg <= 0x7FFFFFFFu, "group: too many workgroups");
    max_lds = std::max(max_lds, need);
    probs->push_back(p);
  }
  *total_wgs = static_cast<int>(wg);
  *lds = max_lds;
  return LLMI_OK;
}

int launch_group(const GroupProblem* probs_dev, int nprob, int total_wgs, std::size_t lds, hipStream_t s) {
  if (nprob == 0 || total_wgs == 0) return LLMI_OK;
  qgemv_group<<<static_cast<unsigned>(total_wgs), kGroupThreads, lds, s>>>(probs_dev, nprob);
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

}  // namespace llmi_hip
