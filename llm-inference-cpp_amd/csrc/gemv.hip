// Quantized matrix-vector / small-batch product for gfx950.
//
// Reference: src/model/quant.cpp:119-153.  For each output o and input row r
// the reference computes, with the compiler's fused multiply-adds,
//     part_b = fma(x[k], code[k], part_b)   over the block's elements in order
//     acc    = fma(part_b, scale_b, acc)    over the blocks in order
//     y      = acc + bias[o]                (bias 0.0f when absent)
// These kernels perform exactly those operations, so y is bit-identical.
//
// Both kernels read the tiled layout (common.hpp): lane l of a wavefront owns
// output row tile*64 + l, so one block of 64 rows is a single coalesced
// 16-byte load per lane (two for Q8_0), and the activations x[k] are the
// same for every lane -- they are read with scalar loads into SGPRs and
// broadcast to the fused multiply-adds for free.  Every code byte and scale
// is read from HBM once; the kernels are HBM-bound at batch 1.
//
// qgemv_r1 (decode, one input row): the W wavefronts of a workgroup split
// the tile's blocks into contiguous ranges and compute block sums
// independently (so even a matrix with few tiles fills the GPU); the sums
// and the block scales are parked in LDS and wavefront 0 runs the sequential
// chain over all blocks, adds the bias and stores y.
//
// qgemv_rows (R = 2..8 input rows, and the exact prefill path): one
// wavefront per tile walks all blocks in order with the chain in registers,
// prefetching the next chunk of blocks while it computes the current one;
// each decoded code is used for all R rows.
#include <algorithm>

#include "common.hpp"

namespace llmi_hip {

// Launch shape of the batch-1 GEMV.  Matrices with many 64-row tiles use
// qgemv_r1 (one workgroup per tile, activations in SGPRs) with enough
// wavefronts per tile to put ~kTargetWaves in the grid.  Matrices with fewer
// tiles than kNarrowTiles use qgemv_narrow (16-row tiles), whose 4W block
// groups per workgroup take ~kBlocksPerGroup blocks each.
GemvPlan plan_gemv(const DeviceMatrix& m) {
  constexpr std::size_t kTargetWaves = 8192;
  constexpr std::size_t kNarrowTiles = 128;
  constexpr std::size_t kBlocksPerGroup = 2;
  GemvPlan p;
  const std::size_t nblk = std::max<std::size_t>(m.nblk, 1);
  if (m.ntiles < kNarrowTiles) {
    p.narrow = true;
    const std::size_t groups = std::min<std::size_t>(64, ceil_div(nblk, kBlocksPerGroup));
    p.waves = static_cast<int>(ceil_div(groups, 4));
    p.bpw = static_cast<int>(ceil_div(nblk, static_cast<std::size_t>(p.waves) * 4));  // blocks per group
    return p;
  }
  const std::size_t per_tile = std::max<std::size_t>(1, ceil_div(kTargetWaves, m.ntiles));
  std::size_t waves = std::max<std::size_t>(1, std::min<std::size_t>({16, nblk, per_tile}));
  p.bpw = static_cast<int>(ceil_div(nblk, waves));
  p.waves = static_cast<int>(ceil_div(nblk, p.bpw));
  return p;
}

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

// ---------------------------------------------------------------- batch 1
// One workgroup per tile.  Dynamic LDS: part[nblk][64] then scale[nblk][64].
template <int TYPE, int CH>
__global__ void __launch_bounds__(1024) qgemv_r1(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                 const float* __restrict__ x, const float* __restrict__ bias,
                                                 float* __restrict__ y, int in, int nblk, int out, int bpw,
                                                 int accumulate);

// Block sums of this wavefront's blocks [b_begin, b_end) of one tile into
// part[] (stride 64 floats per block), scales into scl[] when non-null.
template <int TYPE, int CH>
__device__ __forceinline__ void block_sums(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                           const float* __restrict__ x, std::size_t tile, int in, int nblk, int b_begin,
                                           int b_end, int lane, float* part, float* scl) {
  const int nfull = in / kBlock;
  const int f_end = min(b_end, nfull);
  Block<TYPE> cur[CH];
  float cur_s[CH];
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    if (b_begin + j < f_end) {
      cur[j] = load_block<TYPE>(codes, tile * nblk + b_begin + j, lane);
      if (scl != nullptr) cur_s[j] = scales[(tile * nblk + b_begin + j) * kTileRows + lane];
    }
  }
  for (int b = b_begin; b < f_end; b += CH) {
    Block<TYPE> nxt[CH];
    float nxt_s[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (b + CH + j < f_end) {
        nxt[j] = load_block<TYPE>(codes, tile * nblk + b + CH + j, lane);
        if (scl != nullptr) nxt_s[j] = scales[(tile * nblk + b + CH + j) * kTileRows + lane];
      }
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if (b + j < f_end) {
        std::uint32_t w[8];
        unpack_words<TYPE>(cur[j], w);
        part[(b + j) * kTileRows + lane] = full_block_dot<TYPE>(w, x + (b + j) * kBlock);
        if (scl != nullptr) scl[(b + j) * kTileRows + lane] = cur_s[j];
      }
    }
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      cur[j] = nxt[j];
      cur_s[j] = nxt_s[j];
    }
  }
  if (nfull < nblk && nfull >= b_begin && nfull < b_end) {
    const Block<TYPE> blk = load_block<TYPE>(codes, tile * nblk + nfull, lane);
    part[nfull * kTileRows + lane] = tail_block_dot<TYPE>(blk, x + nfull * kBlock, in - nfull * kBlock);
    if (scl != nullptr) scl[nfull * kTileRows + lane] = scales[(tile * nblk + nfull) * kTileRows + lane];
  }
}

// The sequential chain over all blocks of a tile (wavefront 0), from LDS.
__device__ __forceinline__ float chain_lds(const float* part, const float* scl, int nblk, int lane) {
  float acc = 0.0f;
  int b = 0;
  for (; b + 4 <= nblk; b += 4) {
    const float p0 = part[(b + 0) * kTileRows + lane], s0 = scl[(b + 0) * kTileRows + lane];
    const float p1 = part[(b + 1) * kTileRows + lane], s1 = scl[(b + 1) * kTileRows + lane];
    const float p2 = part[(b + 2) * kTileRows + lane], s2 = scl[(b + 2) * kTileRows + lane];
    const float p3 = part[(b + 3) * kTileRows + lane], s3 = scl[(b + 3) * kTileRows + lane];
    acc = __builtin_fmaf(p0, s0, acc);
    acc = __builtin_fmaf(p1, s1, acc);
    acc = __builtin_fmaf(p2, s2, acc);
    acc = __builtin_fmaf(p3, s3, acc);
  }
  for (; b < nblk; ++b) acc = __builtin_fmaf(part[b * kTileRows + lane], scl[b * kTileRows + lane], acc);
  return acc;
}

// Batch 1 for matrices with few rows (qgemv_narrow): 16-row tiles, so a
// matrix gets 4x the workgroups of the 64-row kernel.  Lane l of a
// wavefront owns row tile16*16 + (l & 15) and one of 4 block groups
// (l >> 4); the W wavefronts of the workgroup give 4W groups, each taking a
// contiguous range of blocks.  The 16 rows of one block are a contiguous
// 256-byte piece of the 64-row tiled layout, so loads stay coalesced.  The
// activations are staged in LDS once per workgroup and read with broadcast
// loads (16 lanes per address).  Block sums and scales go to LDS; lanes 0-15
// of wavefront 0 run the sequential chain.
// Dynamic LDS: x[in], part[nblk][16], scale[nblk][16].
template <int TYPE>
__global__ void __launch_bounds__(1024) qgemv_narrow(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                     const float* __restrict__ x, const float* __restrict__ bias,
                                                     float* __restrict__ y, int in, int nblk, int out, int bpg,
                                                     int accumulate) {
  extern __shared__ float lds[];
  float* xs = lds;
  float* part = lds + ((in + 3) & ~3);
  float* scl = part + nblk * 16;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int wave = threadIdx.x >> 6;
  const int group = wave * 4 + (lane >> 4);
  const std::size_t row = static_cast<std::size_t>(blockIdx.x) * 16 + r;
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
    float acc = 0.0f;
    int b = 0;
    for (; b + 4 <= nblk; b += 4) {
      const float p0 = part[(b + 0) * 16 + r], s0 = scl[(b + 0) * 16 + r];
      const float p1 = part[(b + 1) * 16 + r], s1 = scl[(b + 1) * 16 + r];
      const float p2 = part[(b + 2) * 16 + r], s2 = scl[(b + 2) * 16 + r];
      const float p3 = part[(b + 3) * 16 + r], s3 = scl[(b + 3) * 16 + r];
      acc = __builtin_fmaf(p0, s0, acc);
      acc = __builtin_fmaf(p1, s1, acc);
      acc = __builtin_fmaf(p2, s2, acc);
      acc = __builtin_fmaf(p3, s3, acc);
    }
    for (; b < nblk; ++b) acc = __builtin_fmaf(part[b * 16 + r], scl[b * 16 + r], acc);
    if (row < static_cast<std::size_t>(out)) {
      const float v = acc + (bias != nullptr ? bias[row] : 0.0f);
      y[row] = accumulate ? y[row] + v : v;
    }
  }
}

template <int TYPE, int CH>
__global__ void __launch_bounds__(1024) qgemv_r1(const uint4* __restrict__ codes, const float* __restrict__ scales,
                                                 const float* __restrict__ x, const float* __restrict__ bias,
                                                 float* __restrict__ y, int in, int nblk, int out, int bpw,
                                                 int accumulate) {
  extern __shared__ float lds[];
  float* part = lds;
  float* scl = lds + static_cast<std::size_t>(nblk) * kTileRows;
  const int lane = threadIdx.x & (kTileRows - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const std::size_t tile = blockIdx.x;
  const int b_begin = wave * bpw;
  const int b_end = min(nblk, b_begin + bpw);
  block_sums<TYPE, CH>(codes, scales, x, tile, in, nblk, b_begin, b_end, lane, part, scl);
  __syncthreads();
  if (wave == 0) {
    const float acc = chain_lds(part, scl, nblk, lane);
    const std::size_t o = tile * kTileRows + lane;
    if (o < static_cast<std::size_t>(out)) {
      const float v = acc + (bias != nullptr ? bias[o] : 0.0f);
      y[o] = accumulate ? y[o] + v : v;
    }
  }
}

// ------------------------------------------------------------ batch 2..8
// One wavefront per tile (4 tiles per 256-thread workgroup).
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

constexpr int chunk_for(int type) { return type == LLMI_TYPE_Q8_0 ? 4 : 8; }

template <int TYPE, int R>
int launch_rows(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y, int acc,
                hipStream_t s);

// Largest supported load chunk that does not exceed bpw blocks.
int chunk_le(int bpw, int type) {
  const int cap = chunk_for(type);
  int ch = 1;
  while (ch * 2 <= bpw && ch * 2 <= cap) ch *= 2;
  return ch;
}

template <int TYPE, int CH>
void launch_r1_ch(const DeviceMatrix& m, const float* x, const float* bias, float* y, int acc, int waves, int bpw,
                  std::size_t lds, hipStream_t s) {
  qgemv_r1<TYPE, CH><<<static_cast<unsigned>(m.ntiles), static_cast<unsigned>(waves * 64), lds, s>>>(
      reinterpret_cast<const uint4*>(m.codes), m.scales, x, bias, y, static_cast<int>(m.in), static_cast<int>(m.nblk),
      static_cast<int>(m.out), bpw, acc);
}

template <int TYPE>
int launch_narrow(const DeviceMatrix& m, const float* x, const float* bias, float* y, int acc, const GemvPlan& p,
                  hipStream_t s) {
  const std::size_t lds = (((m.in + 3) & ~std::size_t{3}) + 2 * m.nblk * 16) * sizeof(float);
  qgemv_narrow<TYPE><<<static_cast<unsigned>(ceil_div(m.out, 16)), static_cast<unsigned>(p.waves * 64), lds, s>>>(
      reinterpret_cast<const uint4*>(m.codes), m.scales, x, bias, y, static_cast<int>(m.in), static_cast<int>(m.nblk),
      static_cast<int>(m.out), p.bpw, acc);
  return LLMI_OK;
}

template <int TYPE>
int launch_r1(const DeviceMatrix& m, const float* x, const float* bias, float* y, int acc, hipStream_t s) {
  const GemvPlan p = plan_gemv(m);
  if (p.narrow) {
    const std::size_t lds = (((m.in + 3) & ~std::size_t{3}) + 2 * m.nblk * 16) * sizeof(float);
    if (lds <= max_lds_per_block()) return launch_narrow<TYPE>(m, x, bias, y, acc, p, s);
  }
  const std::size_t lds = 2 * m.nblk * kTileRows * sizeof(float);
  // Rows too long for the LDS staging take the one-wavefront-per-tile path.
  if (lds > max_lds_per_block()) return launch_rows<TYPE, 2>(m, x, 1, bias, y, acc, s);
  int waves = p.waves, bpw = p.bpw;
  if (p.narrow) {  // narrow plan did not fit: fall back to the 64-row kernel
    bpw = static_cast<int>(ceil_div(m.nblk, std::min<std::size_t>(16, m.nblk)));
    waves = static_cast<int>(ceil_div(m.nblk, bpw));
  }
  switch (chunk_le(bpw, TYPE)) {
    case 1: launch_r1_ch<TYPE, 1>(m, x, bias, y, acc, waves, bpw, lds, s); break;
    case 2: launch_r1_ch<TYPE, 2>(m, x, bias, y, acc, waves, bpw, lds, s); break;
    case 4: launch_r1_ch<TYPE, 4>(m, x, bias, y, acc, waves, bpw, lds, s); break;
    default: launch_r1_ch<TYPE, 8>(m, x, bias, y, acc, waves, bpw, lds, s); break;
  }
  return LLMI_OK;
}

template <int TYPE, int R>
int launch_rows(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y, int acc,
                hipStream_t s) {
  constexpr int CH = chunk_for(TYPE) / 2;
  const dim3 grid(static_cast<unsigned>(ceil_div(m.ntiles, 4)), static_cast<unsigned>(ceil_div(rows, R)));
  qgemv_rows<TYPE, R, CH><<<grid, 256, 0, s>>>(reinterpret_cast<const uint4*>(m.codes), m.scales, x, bias, y,
                                               static_cast<int>(m.in), static_cast<int>(m.nblk),
                                               static_cast<int>(m.out), static_cast<int>(rows),
                                               static_cast<int>(m.ntiles), acc);
  return LLMI_OK;
}

template <int TYPE>
int launch_typed(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y, int acc,
                 hipStream_t s) {
  if (rows == 1) return launch_r1<TYPE>(m, x, bias, y, acc, s);
  if (rows == 2) return launch_rows<TYPE, 2>(m, x, rows, bias, y, acc, s);
  if (rows <= 4) return launch_rows<TYPE, 4>(m, x, rows, bias, y, acc, s);
  return launch_rows<TYPE, 8>(m, x, rows, bias, y, acc, s);
}

}  // namespace

int launch_matmul(const DeviceMatrix& m, const float* x, std::size_t rows, const float* bias, float* y, hipStream_t s,
                  bool accumulate) {
  if (rows == 0 || m.out == 0) return LLMI_OK;
  LLMI_REQUIRE(m.in > 0, "matmul: in must be positive");
  LLMI_REQUIRE(m.in <= 0x7FFFFFFFu && m.out <= 0x7FFFFFFFu, "matmul: shape too large");
  LLMI_REQUIRE(ceil_div(rows, 8) <= 65535, "matmul: too many input rows for one launch");
  LLMI_REQUIRE(x != nullptr && y != nullptr, "matmul: null pointer");
  const int acc = accumulate ? 1 : 0;
  const int rc = m.type == LLMI_TYPE_Q8_0 ? launch_typed<LLMI_TYPE_Q8_0>(m, x, rows, bias, y, acc, s)
                                          : launch_typed<LLMI_TYPE_Q4_0>(m, x, rows, bias, y, acc, s);
  if (rc != LLMI_OK) return rc;
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

}  // namespace llmi_hip
