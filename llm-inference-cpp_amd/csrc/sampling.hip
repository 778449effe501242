// Token sampling on the GPU: the reference's sampling_probabilities and
// sample() (src/model/sampling.cpp:11-77) on logits in HBM, with the
// reference's results bit for bit.  The random number stays the caller's:
// sample() draws one std::uniform_real_distribution<double>(0, 1) number from
// its std::mt19937_64 per call (temperature > 0), and the device entry points
// take that number (`target`).
//
// The reference's arithmetic is elementwise except for four sequential double
// sums: the softmax denominator (index order), the top-p running sum and the
// renormalisation sum (both in ranking order), and the running sum that
// sample() compares with its draw (index order).  Each is taken here as a
// parallel sum P with a bound on its distance from the sequential sum S: for
// m non-negative terms both lie within (m-1)u of the exact sum (u = 2^-53,
// whatever the summation tree), so |S - P| <= sigma*P with
// sigma = 4u*(m + 65536) (the 65536 covers the empty slots of the reduction
// trees).  A decision is taken from P only when every S in
// [P(1-sigma), P(1+sigma)] gives the same decision -- the same float
// reciprocal, the same first index whose running sum reaches a threshold --
// and the sum is otherwise recomputed sequentially in the reference's order
// (by one thread, the block staging the terms through LDS).  The sequential
// passes are rare (a threshold within ~1e-11 relative of a running sum).
//
// Kernels of one sampling call (temperature > 0), all on one stream:
//   smp_max    max of logits / temperature (float division), NaN / +inf flags
//   smp_exp    e = expf(x / T - max) (the exact expf), sum -> inv = float(1/sum)
//   when 0 < top_k <= kSelectMax (the ranking's first k):
//     smp_sel_local  p = e * inv; each slice's first k, in index order
//     smp_sel_merge  the first k among those, ranked
//   else, when something is filtered (the whole ranking):
//     smp_scale  p = e * inv and the ranking keys (float bits, index)
//     smp_sort_hist / smp_sort_scan / smp_sort_scatter, four times: the
//                ranking by a stable LSD radix sort (descending p, ties in
//                index order: std::stable_sort's order)
//   (nothing filtered: the later kernels scale e on the fly)
//   smp_keep   top-k, top-p, bounds on the renormalisation sum
//   smp_draw   the filtered probabilities (bounded) and the first index whose
//              running sum reaches target
// When the renormalisation sum's bound leaves the drawn index open (rare),
// the host runs smp_seq_sum2 (the exact sum, ranking order) and smp_draw
// again.  sampling_probabilities always takes the exact sum.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "common.hpp"
#include "exact_math.hpp"
#include "glue_math.hpp"

namespace llmi_hip {
namespace {

constexpr int kSmpThreads = 256;
constexpr int kSmpWaves = kSmpThreads / 64;
constexpr int kSmpBlocks = 128;               // slices of the vocabulary, one workgroup each
constexpr int kSeqChunk = kSmpThreads * 8;    // terms per LDS stage of the sequential sums

enum : int { kFlagNaN = 1, kFlagPosInf = 2, kFlagAllNegInf = 4 };
constexpr int kFlagBad = kFlagNaN | kFlagPosInf | kFlagAllNegInf;
enum : int { kSeqSoftmax = 1, kSeqTopP = 2, kSeqDraw = 4, kSeqSum2 = 8, kSeqSelect = 16 };

struct SmpState {
  float mx;         // max of logits / temperature
  int flags;        // kFlag*
  float inv;        // float(1 / softmax sum)
  int keep;         // kept entries (top-k, top-p)
  double s2_lo;     // the renormalisation sum lies in [s2_lo, s2_hi]; equal when exact
  double s2_hi;
  float p_thr;      // kept: p > p_thr, or p == p_thr and index <= idx_last
  int idx_last;
  int id;           // the drawn index
  int decided;      // 1 when id is the reference's
  int seq_paths;    // kSeq*: which sums needed the sequential pass (diagnostics)
  unsigned counter; // last-block handshake, reset by each kernel's last block
};

struct SmpWork {
  float* p;                  // e, then p = e * inv
  std::uint32_t* keys;       // ranking keys: bits of p (p >= +0)
  std::uint32_t* keys_sorted;
  std::int32_t* idx;
  std::int32_t* idx_sorted;
  double* part_d;            // per-block partials
  int* part_i;
  float* part_f;
  SmpState* st;
};

__device__ __forceinline__ float recip_float(double s) { return static_cast<float>(1.0 / s); }
__device__ __forceinline__ double smp_sigma(int m) { return 4.0 * (static_cast<double>(m) + 65536.0) * 0x1p-53; }

struct Slice {
  int lo, hi;
};
__device__ __forceinline__ Slice slice_of(int m, int b, int blocks) {
  const int per = (m + blocks - 1) / blocks;
  const int lo = min(m, b * per);
  return Slice{lo, min(m, lo + per)};
}

__device__ __forceinline__ float block_max_f(float v, float* red) {
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < kSmpWaves; ++w) r = fmaxf(r, red[w]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ int block_or(int v, int* red) {
  for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = 0;
  for (int w = 0; w < kSmpWaves; ++w) r |= red[w];
  __syncthreads();
  return r;
}
__device__ __forceinline__ int block_min_i(int v, int* red) {
  for (int o = 32; o > 0; o >>= 1) v = min(v, __shfl_xor(v, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = red[0];
  for (int w = 1; w < kSmpWaves; ++w) r = min(r, red[w]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ int block_max_i(int v, int* red) {
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = red[0];
  for (int w = 1; w < kSmpWaves; ++w) r = max(r, red[w]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ double block_sum_d(double v, double* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = red[0];
  for (int w = 1; w < kSmpWaves; ++w) r = r + red[w];
  __syncthreads();
  return r;
}

// Thread 0 publishes the block's partials (already stored; the release half
// of the counter update makes them visible at agent scope) and learns whether
// it is the last block of the grid to do so (the acquire half).  The last
// block's other threads read the partials after a barrier with agent-scope
// atomic loads (load_relaxed); data written by earlier kernels needs nothing.
// No other fence: an agent-scope fence writes back or invalidates the whole
// L2 of the XCD, which costs microseconds per wavefront.
__device__ __forceinline__ bool arrive_last(unsigned* counter) {
  const unsigned done = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  return done == gridDim.x - 1;
}
__device__ __forceinline__ void reset_counter(unsigned* counter) {
  __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T load_relaxed(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The grid's per-block partials src[0..nb) (written by other workgroups of
// this launch) into LDS, every thread loading its share, then the running
// prefix pre[0..nb] (pre[0] = 0) by thread 0 in block order.
__device__ __forceinline__ void partial_prefix(const double* src, int stride, int nb, double* tmp, double* pre) {
  for (int b = threadIdx.x; b < nb; b += kSmpThreads) tmp[b] = load_relaxed(src + static_cast<std::size_t>(b) * stride);
  __syncthreads();
  if (threadIdx.x == 0) {
    pre[0] = 0.0;
    for (int b = 0; b < nb; ++b) pre[b + 1] = pre[b] + tmp[b];
  }
  __syncthreads();
}

// First b in [0, nb) with pre[b + 1] * factor >= t, or nb (pre in LDS).
__device__ __forceinline__ int first_block_reaching(const double* pre, int nb, double factor, double t, int* red_i) {
  int c = nb;
  for (int b = threadIdx.x; b < nb; b += kSmpThreads)
    if (pre[b + 1] * factor >= t) c = min(c, b);
  return block_min_i(c, red_i);
}

// Exclusive prefix of v over the block in thread order, as sums (wave
// shuffles, then the wave totals: no subtraction, so every prefix is a tree
// of the terms); *total = the sum.  wave_tot holds kSmpWaves doubles.
__device__ __forceinline__ double block_exclusive_scan_w(double v, double* wave_tot, double* total) {
  const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
  double incl = v;
  for (int o = 1; o < 64; o <<= 1) {
    const double u = __shfl_up(incl, o, 64);
    if (l >= o) incl = incl + u;
  }
  double excl = __shfl_up(incl, 1, 64);
  if (l == 0) excl = 0.0;
  if (l == 63) wave_tot[wv] = incl;
  __syncthreads();
  double before = 0.0, tot = 0.0;
  for (int q = 0; q < kSmpWaves; ++q) {
    if (q < wv) before = before + wave_tot[q];
    tot = tot + wave_tot[q];
  }
  __syncthreads();
  *total = tot;
  return before + excl;
}

// First j in [lo, hi) with (base + v(lo) + ... + v(j)) * factor >= t, or hi.
// Every thread of the block takes part; the running sums are a tree over the
// terms (a contiguous run per thread, then the block scan).  Runs of up to
// kHeld terms are read once, every load issued before the first use (the
// slice was written on another XCD: each dependent read would wait for HBM).
template <typename F>
__device__ int slice_first_reach(F v, int lo, int hi, double base, double factor, double t, double* sh, int* red_i) {
  constexpr int kHeld = 8;
  const int len = hi - lo;
  if (len <= 0) return hi;
  const int per = (len + kSmpThreads - 1) / kSmpThreads;
  const int a = lo + min(len, static_cast<int>(threadIdx.x) * per);
  const int e = min(hi, a + per);
  int found = hi;
  if (per <= kHeld) {
    float x[kHeld];
#pragma unroll
    for (int q = 0; q < kHeld; ++q) {
      const float val = v(min(a + q, hi - 1));
      x[q] = a + q < e ? val : 0.0f;
    }
    double cs = 0.0;
#pragma unroll
    for (int q = 0; q < kHeld; ++q) cs = cs + static_cast<double>(x[q]);
    double total;
    double run = base + block_exclusive_scan_w(cs, sh, &total);
#pragma unroll
    for (int q = 0; q < kHeld; ++q) {
      run = run + static_cast<double>(x[q]);
      if (found == hi && a + q < e && run * factor >= t) found = a + q;
    }
    return block_min_i(found, red_i);
  }
  double cs = 0.0;
  for (int j = a; j < e; ++j) cs = cs + static_cast<double>(v(j));
  double total;
  double run = base + block_exclusive_scan_w(cs, sh, &total);
  for (int j = a; j < e; ++j) {
    run = run + static_cast<double>(v(j));
    if (run * factor >= t) {
      found = j;
      break;
    }
  }
  return block_min_i(found, red_i);
}

// base + v(lo) + ... + v(hi - 1), a tree as above.
template <typename F>
__device__ double slice_sum(F v, int lo, int hi, double* red) {
  double s = 0.0;
  for (int j = lo + static_cast<int>(threadIdx.x); j < hi; j += kSmpThreads) s = s + static_cast<double>(v(j));
  return block_sum_d(s, red);
}

// The reference's own sequential double running sum of v(0), v(1), ...,
// v(m-1): thread 0 adds while waves 1..3 stage the next kSeqChunk terms into
// the other half of `stage` (2 * kSeqChunk floats).  With `has_stop`, stops at
// the first j whose running sum reaches stop_at and returns j; else returns m.
// *sum = the running sum where it stopped.  Every thread must call it.  The
// stop index goes through two LDS slots used in alternate rounds, so thread 0
// never overwrites a slot another wave has yet to read.
template <typename F>
__device__ int block_sequential_sum(F v, int m, bool has_stop, double stop_at, double* sum, float* stage,
                                    int* stop_slots) {
  const int t = threadIdx.x;
  for (int k = t; k < kSeqChunk; k += kSmpThreads) stage[k] = k < m ? v(k) : 0.0f;
  if (t == 0) {
    stop_slots[0] = -1;
    stop_slots[1] = -1;
  }
  __syncthreads();
  double run = 0.0;
  int buf = 0, stop = -1;
  for (int c0 = 0; c0 < m; c0 += kSeqChunk) {
    if (t >= 64) {
      float* nxt = stage + (buf ^ 1) * kSeqChunk;
      for (int k = t - 64; k < kSeqChunk; k += kSmpThreads - 64) {
        const int j = c0 + kSeqChunk + k;
        nxt[k] = j < m ? v(j) : 0.0f;
      }
    }
    if (t == 0) {
      const float* cur = stage + buf * kSeqChunk;
      const int len = min(kSeqChunk, m - c0);
      for (int k = 0; k < len; ++k) {
        run = run + static_cast<double>(cur[k]);
        if (has_stop && run >= stop_at) {
          stop_slots[buf] = c0 + k;
          break;
        }
      }
    }
    __syncthreads();
    stop = stop_slots[buf];
    if (stop >= 0) break;
    buf ^= 1;
  }
  if (t == 0) *sum = run;
  __syncthreads();
  return stop >= 0 ? stop : m;
}

// ------------------------------------------------------------------ kernels
__global__ void __launch_bounds__(kSmpThreads) smp_max(const float* __restrict__ logits, int n, float temp, SmpWork w,
                                                       SampleLog* __restrict__ log) {
  __shared__ float red_f[kSmpWaves];
  __shared__ int red_i[kSmpWaves];
  __shared__ bool last;
  const Slice sl = slice_of(n, blockIdx.x, gridDim.x);
  float m = -__builtin_inff();
  int fl = 0;
  for (int i = sl.lo + static_cast<int>(threadIdx.x); i < sl.hi; i += kSmpThreads) {
    const float v = logits[i] / temp;
    if (v != v) fl |= kFlagNaN;
    if (v == __builtin_inff()) fl |= kFlagPosInf;
    m = fmaxf(m, v);
  }
  m = block_max_f(m, red_f);
  fl = block_or(fl, red_i);
  if (threadIdx.x == 0) {
    w.part_f[blockIdx.x] = m;
    w.part_i[blockIdx.x] = fl;
    last = arrive_last(&w.st->counter);
  }
  __syncthreads();
  if (!last) return;
  float mm = -__builtin_inff();
  int ff = 0;
  for (int b = threadIdx.x; b < static_cast<int>(gridDim.x); b += kSmpThreads) {
    mm = fmaxf(mm, load_relaxed(w.part_f + b));
    ff |= load_relaxed(w.part_i + b);
  }
  mm = block_max_f(mm, red_f);
  ff = block_or(ff, red_i);
  if (threadIdx.x == 0) {
    if (ff == 0 && mm == -__builtin_inff()) ff = kFlagAllNegInf;
    w.st->mx = mm;
    w.st->flags = ff;
    w.st->seq_paths = 0;
    w.st->decided = 0;
    if (log != nullptr) *log = SampleLog{-1, ff << 1};  // smp_draw overwrites it when it decides
    reset_counter(&w.st->counter);
  }
}

// kernels.cpp:136-146 on x / temperature.
__global__ void __launch_bounds__(kSmpThreads) smp_exp(const float* __restrict__ logits, int n, float temp, SmpWork w) {
  __shared__ std::uint64_t tab[32];
  __shared__ double red_d[kSmpWaves];
  __shared__ float stage[2 * kSeqChunk];
  __shared__ int stop[2];
  __shared__ double seq;
  __shared__ bool last;
  if (w.st->flags & kFlagBad) return;
  if (threadIdx.x < 32) tab[threadIdx.x] = exact::kExp2Tab[threadIdx.x];
  __syncthreads();
  const float mx = w.st->mx;
  const Slice sl = slice_of(n, blockIdx.x, gridDim.x);
  double part = 0.0;
  for (int i = sl.lo + static_cast<int>(threadIdx.x); i < sl.hi; i += kSmpThreads) {
    const float e = exact::expf_with(logits[i] / temp - mx, tab);
    w.p[i] = e;
    part = part + static_cast<double>(e);
  }
  part = block_sum_d(part, red_d);
  if (threadIdx.x == 0) {
    w.part_d[blockIdx.x] = part;
    last = arrive_last(&w.st->counter);
  }
  __syncthreads();
  if (!last) return;
  __shared__ float inv_s;
  __shared__ double tmp[kSmpBlocks], pre[kSmpBlocks + 1];
  partial_prefix(w.part_d, 1, gridDim.x, tmp, pre);
  if (threadIdx.x == 0) {
    const double sum = pre[gridDim.x];
    const double slack = smp_sigma(n) * sum;
    inv_s = recip_float(sum - slack) == recip_float(sum + slack) ? recip_float(sum) : -1.0f;
  }
  __syncthreads();
  float inv = inv_s;
  if (inv < 0.0f) {
    // The bound leaves float(1/sum) open: the sequential sum, its terms
    // recomputed from the logits (other workgroups' e need not be visible).
    block_sequential_sum([=](int j) { return exact::expf_with(logits[j] / temp - mx, tab); }, n, false, 0.0, &seq,
                         stage, stop);
    inv = recip_float(seq);
    if (threadIdx.x == 0) w.st->seq_paths |= kSeqSoftmax;
  }
  if (threadIdx.x == 0) {
    w.st->inv = inv;
    reset_counter(&w.st->counter);
  }
}

__global__ void __launch_bounds__(kSmpThreads) smp_scale(int n, SmpWork w, int write_keys) {
  if (w.st->flags & kFlagBad) return;
  const int i = blockIdx.x * kSmpThreads + threadIdx.x;
  if (i >= n) return;
  const float p = w.p[i] * w.st->inv;
  w.p[i] = p;
  if (write_keys) {
    w.keys[i] = __builtin_bit_cast(std::uint32_t, p);
    w.idx[i] = i;
  }
}

// Ranking keys of p = e * inv, p left unscaled (the exact path of an
// unfiltered draw, which skipped smp_scale).
__global__ void __launch_bounds__(kSmpThreads) smp_keys(int n, SmpWork w) {
  const int i = blockIdx.x * kSmpThreads + threadIdx.x;
  if (i >= n) return;
  w.keys[i] = __builtin_bit_cast(std::uint32_t, w.p[i] * w.st->inv);
  w.idx[i] = i;
}

// First maximum of x (transformer.cpp:22-24) for temperature <= 0: slices,
// then the last workgroup combines (lowest index among equal maxima).
__device__ __forceinline__ void better_of(float& v, int& i, float v2, int i2) {
  if (i2 < 0) return;
  if (i < 0 || v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}
__device__ __forceinline__ void block_best(float& v, int& i, float* sv, int* si) {
  for (int o = 32; o > 0; o >>= 1) {
    const float v2 = __shfl_xor(v, o, 64);
    const int i2 = __shfl_xor(i, o, 64);
    better_of(v, i, v2, i2);
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = v;
    si[threadIdx.x >> 6] = i;
  }
  __syncthreads();
  v = sv[0];
  i = si[0];
  for (int w = 1; w < kSmpWaves; ++w) better_of(v, i, sv[w], si[w]);
  __syncthreads();
}
__global__ void __launch_bounds__(kSmpThreads) smp_argmax(const float* __restrict__ x, int n, SmpWork w,
                                                          std::int32_t* __restrict__ out) {
  __shared__ float sv[kSmpWaves];
  __shared__ int si[kSmpWaves];
  __shared__ bool last;
  const Slice sl = slice_of(n, blockIdx.x, gridDim.x);
  float v = 0.0f;
  int i = -1;
  for (int j = sl.lo + static_cast<int>(threadIdx.x); j < sl.hi; j += kSmpThreads) better_of(v, i, x[j], j);
  block_best(v, i, sv, si);
  if (threadIdx.x == 0) {
    w.part_f[blockIdx.x] = v;
    w.part_i[blockIdx.x] = i;
    last = arrive_last(&w.st->counter);
  }
  __syncthreads();
  if (!last) return;
  v = 0.0f;
  i = -1;
  for (int b = threadIdx.x; b < static_cast<int>(gridDim.x); b += kSmpThreads)
    better_of(v, i, load_relaxed(w.part_f + b), load_relaxed(w.part_i + b));
  block_best(v, i, sv, si);
  if (threadIdx.x == 0) {
    *out = i < 0 ? 0 : i;
    reset_counter(&w.st->counter);
  }
}

// Kept by the filters: above the last kept value, or equal to it at an index
// up to the last kept one's (the ranking breaks ties by index).
__device__ __forceinline__ bool kept(float p, int i, float p_thr, int idx_last) {
  return p > p_thr || (p == p_thr && i <= idx_last);
}
__device__ __forceinline__ float renorm(float p, double s) {
  return static_cast<float>(static_cast<double>(p) / s);
}

// ------------------------------------------------------------ top-k selection
// The first k entries of the ranking (p descending, equal p by index, the
// order std::stable_sort gives sampling.cpp:30-34) without sorting all n, for
// 0 < top_k <= kSelectMax.  Keys are the bits of p = e * inv (p >= +0, so
// their unsigned order is p's order); a select finds the k-th largest key K
// by four 8-bit radix passes over LDS histograms (integer counts: every
// decision is exact) and keeps every key above K and the lowest-index entries
// equal to it.  smp_sel_local does that per slice, writing the slice's first
// k in index order; the ranking's first k are among those candidates, which
// are then in index order overall, and smp_sel_merge selects again over them
// and ranks the k it keeps.
constexpr int kSelectMax = 64;
constexpr int kCandMax = kSmpBlocks * kSelectMax;
static_assert(kSmpThreads == 256, "one histogram bin per thread");

__device__ __forceinline__ std::uint32_t key_bits(float p) { return __builtin_bit_cast(std::uint32_t, p); }

// One radix step of a select.  hist[0..256) holds the counts of the next
// digit among the keys under the prefix sel[0]; sel[1] keys are known to be
// above that prefix.  Wave 0 finds the digit where the count from the top
// first reaches `want` and appends it (lane l owns digits 255-4l .. 252-4l).
// Call between barriers.
__device__ __forceinline__ void radix_pick(const int* hist, int want, unsigned* sel) {
  if (threadIdx.x >= 64) return;
  const int l = threadIdx.x;
  const unsigned prefix = sel[0];
  const int above = static_cast<int>(sel[1]);
  int c[4], s = 0;
  for (int j = 0; j < 4; ++j) {
    c[j] = hist[255 - 4 * l - j];
    s += c[j];
  }
  int incl = s;
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(incl, o, 64);
    if (l >= o) incl += u;
  }
  int run = above + incl - s;
  for (int j = 0; j < 4; ++j) {
    if (run < want && run + c[j] >= want) {
      sel[0] = (prefix << 8) | static_cast<unsigned>(255 - 4 * l - j);
      sel[1] = static_cast<unsigned>(run);
    }
    run += c[j];
  }
}

// Exclusive prefix over the block (kWaves wavefronts) of one count per
// thread, in thread order; *total = the sum.  wave_tot holds kWaves ints.
template <int kWaves>
__device__ __forceinline__ int block_count_prefix(int v, int* wave_tot, int* total) {
  const int l = threadIdx.x & 63, wv = threadIdx.x >> 6;
  int incl = v;
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(incl, o, 64);
    if (l >= o) incl += u;
  }
  if (l == 63) wave_tot[wv] = incl;
  __syncthreads();
  int r = incl - v, tot = 0;
  for (int q = 0; q < kWaves; ++q) {
    const int c = wave_tot[q];
    if (q < wv) r += c;
    tot += c;
  }
  __syncthreads();
  *total = tot;
  return r;
}

// Scales the slice (p = e * inv, the work of smp_scale) and writes its first
// min(k, slice) entries of the ranking, in index order, to
// keys / idx [b * kSelectMax, ...); their count to part_i[b].
__global__ void __launch_bounds__(kSmpThreads) smp_sel_local(int n, int k, SmpWork w) {
  __shared__ int hist[256];
  __shared__ unsigned sel[2];
  __shared__ int wave_tot[kSmpWaves];
  if (w.st->flags & kFlagBad) return;
  const Slice sl = slice_of(n, blockIdx.x, gridDim.x);
  const int want = min(k, sl.hi - sl.lo);
  const int t = threadIdx.x;
  const float inv = w.st->inv;
  if (t == 0) {
    sel[0] = 0u;
    sel[1] = 0u;
  }
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    hist[t] = 0;
    __syncthreads();
    const unsigned prefix = sel[0];
    for (int i = sl.lo + t; i < sl.hi; i += kSmpThreads) {
      std::uint32_t key;
      if (pass == 0) {
        const float p = w.p[i] * inv;
        w.p[i] = p;
        key = key_bits(p);
      } else {
        key = key_bits(w.p[i]);
      }
      if (pass == 0 || (key >> (shift + 8)) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1);
    }
    __syncthreads();
    if (want > 0) radix_pick(hist, want, sel);
    __syncthreads();
  }
  const std::uint32_t K = sel[0];
  const int need = want - static_cast<int>(sel[1]);  // keys equal to K that are kept
  std::uint32_t* keys = w.keys + blockIdx.x * kSelectMax;
  std::int32_t* idx = w.idx + blockIdx.x * kSelectMax;
  int above_done = 0, ties_done = 0;
  for (int c0 = sl.lo; c0 < sl.hi; c0 += kSmpThreads) {
    const int i = c0 + t;
    const bool in = want > 0 && i < sl.hi;
    const std::uint32_t key = in ? key_bits(w.p[i]) : 0u;
    const bool above = in && key > K, tie = in && key == K;
    // One exchange carries both counts: above in the high half, ties low.
    int tot = 0;
    const int before = block_count_prefix<kSmpWaves>((above ? 1 << 16 : 0) + (tie ? 1 : 0), wave_tot, &tot);
    const int a_before = above_done + (before >> 16), t_before = ties_done + (before & 0xffff);
    if (above || (tie && t_before < need)) {
      const int pos = a_before + min(t_before, need);
      keys[pos] = key;
      idx[pos] = i;
    }
    above_done += tot >> 16;
    ties_done += tot & 0xffff;
  }
  if (t == 0) w.part_i[blockIdx.x] = want;
}

// One workgroup: the select over every slice's candidates, each thread
// holding a run of kRun slots in registers (vector loads, all issued at
// once: the candidates come from other XCDs' workgroups), then the k kept,
// ranked, into keys_sorted / idx_sorted.  With at most kSelectMax ranked
// values the rest of sampling_probabilities and sample() (sampling.cpp:36-77)
// is short enough for one lane to run exactly as the reference does: the
// top-p cumulative and the renormalisation sum are the same left fold over
// the ranking, and the draw's running sum over index order adds only the
// kept entries (the others are +0, which leaves a double sum unchanged).  So
// the state is written with the exact sum, and with draw set the index too.
constexpr int kMergeThreads = 1024;
__global__ void __launch_bounds__(kMergeThreads) smp_sel_merge(int k, float top_p, double target, int draw, SmpWork w,
                                                               std::int32_t* __restrict__ also,
                                                               SampleLog* __restrict__ log) {
  constexpr int kRun = kCandMax / kMergeThreads;
  constexpr int kWaves = kMergeThreads / 64;
  static_assert(kRun == 8 && kSelectMax % kRun == 0, "a thread's run is two 16-byte loads inside one slice");
  __shared__ int hist[256];
  __shared__ unsigned sel[2];
  __shared__ int wave_tot[kWaves];
  __shared__ std::uint32_t sk[kSelectMax];
  __shared__ std::int32_t si[kSelectMax];
  __shared__ int slot;
  if (w.st->flags & kFlagBad) return;
  const int t = threadIdx.x;
  const int c_lo = t * kRun;
  // Slots past a slice's count hold stale values and are never used.
  const int valid = min(kRun, max(0, w.part_i[c_lo / kSelectMax] - c_lo % kSelectMax));
  const auto* kp = reinterpret_cast<const uint4*>(w.keys + c_lo);
  const auto* ip = reinterpret_cast<const uint4*>(w.idx + c_lo);
  const uint4 k0 = kp[0], k1 = kp[1], i0 = ip[0], i1 = ip[1];
  const std::uint32_t key[kRun] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
  const std::int32_t id[kRun] = {static_cast<std::int32_t>(i0.x), static_cast<std::int32_t>(i0.y),
                                 static_cast<std::int32_t>(i0.z), static_cast<std::int32_t>(i0.w),
                                 static_cast<std::int32_t>(i1.x), static_cast<std::int32_t>(i1.y),
                                 static_cast<std::int32_t>(i1.z), static_cast<std::int32_t>(i1.w)};
  if (t == 0) {
    sel[0] = 0u;
    sel[1] = 0u;
    slot = 0;
  }
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    if (t < 256) hist[t] = 0;
    __syncthreads();
    const unsigned prefix = sel[0];
#pragma unroll
    for (int j = 0; j < kRun; ++j)
      if (j < valid && (pass == 0 || (key[j] >> (shift + 8)) == prefix)) atomicAdd(&hist[(key[j] >> shift) & 255u], 1);
    __syncthreads();
    radix_pick(hist, k, sel);
    __syncthreads();
  }
  const std::uint32_t K = sel[0];
  const int need = k - static_cast<int>(sel[1]);
  int my_ties = 0;
#pragma unroll
  for (int j = 0; j < kRun; ++j) my_ties += (j < valid && key[j] == K) ? 1 : 0;
  int tot = 0;
  int tie_rank = block_count_prefix<kWaves>(my_ties, wave_tot, &tot);  // the candidates are in index order
#pragma unroll
  for (int j = 0; j < kRun; ++j) {
    bool keep = j < valid && key[j] > K;
    if (j < valid && key[j] == K) keep = tie_rank++ < need;
    if (keep) {
      const int q = atomicAdd(&slot, 1);
      sk[q] = key[j];
      si[q] = id[j];
    }
  }
  __syncthreads();
  __shared__ float rv[kSelectMax];        // the ranking's values
  __shared__ std::int32_t ri[kSelectMax]; // and indices
  __shared__ float fo[kSelectMax];        // the kept f in index order
  __shared__ std::int32_t io[kSelectMax];
  __shared__ int keep_s;
  __shared__ double s2_s;
  if (t < k) {
    const std::uint32_t kt = sk[t];
    const std::int32_t it = si[t];
    int r = 0;
    for (int q = 0; q < k; ++q) r += (sk[q] > kt || (sk[q] == kt && si[q] < it)) ? 1 : 0;
    w.keys_sorted[r] = kt;
    w.idx_sorted[r] = it;
    rv[r] = __builtin_bit_cast(float, kt);
    ri[r] = it;
  }
  __syncthreads();
  // Wave 0 runs the sequential folds with lane i holding ranked value i,
  // read in order with v_readlane (no LDS round trip per term).
  if (t < 64) {
    const float v = t < k ? rv[t] : 0.0f;
    const std::int32_t vi = t < k ? ri[t] : 0;
    // sampling.cpp:36-45 and :50-53: the cumulative stops at keep - 1, where
    // it equals the sum of the kept.
    double cum = 0.0;
    int keep = k;
    bool cut = false;
#pragma unroll
    for (int i = 0; i < kSelectMax; ++i) {
      if (i < k && !cut) {
        cum += static_cast<double>(readlane_f32(v, i));
        if (top_p < 1.0f && cum >= static_cast<double>(top_p)) {
          keep = i + 1;
          cut = true;
        }
      }
    }
    const double s2 = cum;
    // The kept values renormalised, placed in index order.
    if (t < keep) {
      int pos = 0;
#pragma unroll
      for (int q = 0; q < kSelectMax; ++q)
        if (q < keep) pos += __builtin_amdgcn_readlane(vi, q) < vi ? 1 : 0;
      fo[pos] = renorm(v, s2);
      io[pos] = vi;
    }
    if (t == 0) {
      keep_s = keep;
      s2_s = s2;
    }
  }
  __syncthreads();
  if (t < 64) {
    const int keep = keep_s;
    const double s2 = s2_s;
    const float f = t < keep ? fo[t] : 0.0f;
    const std::int32_t fi = t < keep ? io[t] : 0;
    int id = -1;
    if (draw) {
      // sampling.cpp:66-76.  target <= 0 is reached at index 0 whatever p[0];
      // the filtered entries add +0 to the running sum.
      id = target <= 0.0 ? 0 : -1;
      double cum = 0.0;
#pragma unroll
      for (int j = 0; j < kSelectMax; ++j) {
        if (j < keep && id < 0) {
          cum += static_cast<double>(readlane_f32(f, j));
          if (cum >= target) id = __builtin_amdgcn_readlane(fi, j);
        }
      }
      // Else the last nonzero entry (never absent: the top entry's f is at
      // least 1 / keep).
      const unsigned long long nz = __builtin_amdgcn_ballot_w64(t < keep && f > 0.0f);
      if (id < 0 && nz != 0) id = __builtin_amdgcn_readlane(fi, 63 - __builtin_clzll(nz));
      if (id < 0) id = 0;
    }
    if (t == 0) {
      SmpState* st = w.st;
      st->keep = keep;
      st->s2_lo = s2;
      st->s2_hi = s2;
      st->p_thr = rv[keep - 1];
      st->idx_last = ri[keep - 1];
      st->seq_paths |= kSeqSelect;
      if (draw) {
        st->id = id;
        st->decided = 1;
        if (also != nullptr) *also = id;
        if (log != nullptr) *log = SampleLog{id, 1};
      }
    }
  }
}

// Top-k and top-p (sampling.cpp:28-51) over the first m ranked values
// (m = k; `vals` is the ranking, or the unranked p when nothing is
// filtered: then m = n and every entry is kept), and the bounds on the
// renormalisation sum of the kept ones (:53-57).
__global__ void __launch_bounds__(kSmpThreads) smp_keep(const float* __restrict__ vals,
                                                        const std::int32_t* __restrict__ idx_sorted, int m, int n,
                                                        float top_p, int scaled, SmpWork w) {
  __shared__ double red_d[kSmpWaves];
  __shared__ int red_i[kSmpWaves];
  __shared__ double sh[kSmpThreads];
  __shared__ double pre[kSmpBlocks + 1];
  __shared__ float stage[2 * kSeqChunk];
  __shared__ int stop[2];
  __shared__ double seq;
  __shared__ bool last;
  if (w.st->flags & kFlagBad) return;
  const float mult = scaled ? 1.0f : w.st->inv;  // unscaled: vals holds e, p = e * inv
  auto v = [vals, mult](int j) { return vals[j] * mult; };
  const Slice sl = slice_of(m, blockIdx.x, gridDim.x);
  const double part = slice_sum(v, sl.lo, sl.hi, red_d);
  if (threadIdx.x == 0) {
    w.part_d[blockIdx.x] = part;
    last = arrive_last(&w.st->counter);
  }
  __syncthreads();
  if (!last) return;
  const int nb = gridDim.x;
  partial_prefix(w.part_d, 1, nb, sh, pre);
  const double sigma = smp_sigma(m);
  int keep = m;
  bool exact = false;
  double s2 = 0.0;
  if (top_p < 1.0f) {
    const double t = static_cast<double>(top_p);
    const int b_e = first_block_reaching(pre, nb, 1.0 + sigma, t, red_i);
    const int b_l = first_block_reaching(pre, nb, 1.0 - sigma, t, red_i);
    bool decided = false;
    if (b_e == nb) {
      decided = true;  // the running sum certainly stays below top_p: keep = m
    } else if (b_l < nb) {
      const Slice se = slice_of(m, b_e, nb), sl2 = slice_of(m, b_l, nb);
      const int j_e = slice_first_reach(v, se.lo, se.hi, pre[b_e], 1.0 + sigma, t, sh, red_i);
      const int j_l = slice_first_reach(v, sl2.lo, sl2.hi, pre[b_l], 1.0 - sigma, t, sh, red_i);
      if (j_l < sl2.hi && j_e == j_l) {
        keep = j_e + 1;
        decided = true;
      }
    }
    if (!decided) {
      const int j = block_sequential_sum(v, m, true, t, &seq, stage, stop);
      keep = j < m ? j + 1 : m;
      s2 = seq;
      exact = true;
      if (threadIdx.x == 0) w.st->seq_paths |= kSeqTopP;
    }
  }
  if (!exact) {
    // P = running sum through keep - 1.
    const int per = (m + nb - 1) / nb;
    const int b_k = (keep - 1) / per;  // the slice holding index keep - 1
    const Slice sk = slice_of(m, b_k, nb);
    const double within = slice_sum(v, sk.lo, keep, red_d);
    s2 = pre[b_k] + within;
  }
  if (threadIdx.x == 0) {
    const double sg = smp_sigma(keep);
    w.st->keep = keep;
    w.st->s2_lo = exact ? s2 : s2 * (1.0 - sg);
    w.st->s2_hi = exact ? s2 : s2 * (1.0 + sg);
    if (idx_sorted != nullptr) {
      w.st->p_thr = v(keep - 1);
      w.st->idx_last = idx_sorted[keep - 1];
    } else {
      w.st->p_thr = -__builtin_inff();
      w.st->idx_last = n;
    }
    reset_counter(&w.st->counter);
  }
}

// The exact renormalisation sum (sampling.cpp:53-56): the kept ranked values
// in ranking order, sequentially.  One workgroup; nothing to do when the
// bound already pinned it.
__global__ void __launch_bounds__(kSmpThreads) smp_seq_sum2(const float* __restrict__ ranked, SmpWork w) {
  __shared__ float stage[2 * kSeqChunk];
  __shared__ int stop[2];
  __shared__ double seq;
  if (w.st->flags & kFlagBad) return;
  if (w.st->s2_lo == w.st->s2_hi) return;
  const int keep = w.st->keep;
  block_sequential_sum([ranked](int j) { return ranked[j]; }, keep, false, 0.0, &seq, stage, stop);
  if (threadIdx.x == 0) {
    w.st->s2_lo = seq;
    w.st->s2_hi = seq;
    w.st->seq_paths |= kSeqSum2;
  }
}

// sample() (sampling.cpp:60-77) given its draw: the filtered probabilities
// f = float(double(p) / s2) lie in [f(s2_hi), f(s2_lo)]; the first index
// whose running sum reaches target, or else the last nonzero entry.
__global__ void __launch_bounds__(kSmpThreads) smp_draw(int n, double target, int scaled, SmpWork w,
                                                        std::int32_t* __restrict__ also, SampleLog* __restrict__ log) {
  __shared__ double red_d[kSmpWaves];
  __shared__ int red_i[kSmpWaves];
  __shared__ double sh[kSmpThreads];
  __shared__ double pre_lo[kSmpBlocks + 1], pre_hi[kSmpBlocks + 1];
  __shared__ float stage[2 * kSeqChunk];
  __shared__ int stop[2];
  __shared__ double seq;
  __shared__ bool last;
  if (w.st->flags & kFlagBad) return;
  const float* p = w.p;
  const float mult = scaled ? 1.0f : w.st->inv;
  const float p_thr = w.st->p_thr;
  const int idx_last = w.st->idx_last;
  const double s2_lo = w.st->s2_lo, s2_hi = w.st->s2_hi;
  auto f_lo = [=](int i) {
    const float x = p[i] * mult;
    return kept(x, i, p_thr, idx_last) ? renorm(x, s2_hi) : 0.0f;
  };
  auto f_hi = [=](int i) {
    const float x = p[i] * mult;
    return kept(x, i, p_thr, idx_last) ? renorm(x, s2_lo) : 0.0f;
  };
  const Slice sl = slice_of(n, blockIdx.x, gridDim.x);
  double sum_lo = 0.0, sum_hi = 0.0;
  int nz_lo = -1, nz_hi = -1;
  for (int i = sl.lo + static_cast<int>(threadIdx.x); i < sl.hi; i += kSmpThreads) {
    const float a = f_lo(i), b = f_hi(i);
    sum_lo = sum_lo + static_cast<double>(a);
    sum_hi = sum_hi + static_cast<double>(b);
    if (a > 0.0f) nz_lo = i;
    if (b > 0.0f) nz_hi = i;
  }
  sum_lo = block_sum_d(sum_lo, red_d);
  sum_hi = block_sum_d(sum_hi, red_d);
  nz_lo = block_max_i(nz_lo, red_i);
  nz_hi = block_max_i(nz_hi, red_i);
  if (threadIdx.x == 0) {
    w.part_d[2 * blockIdx.x] = sum_lo;
    w.part_d[2 * blockIdx.x + 1] = sum_hi;
    w.part_i[2 * blockIdx.x] = nz_lo;
    w.part_i[2 * blockIdx.x + 1] = nz_hi;
    last = arrive_last(&w.st->counter);
  }
  __syncthreads();
  if (!last) return;
  const int nb = gridDim.x;
  partial_prefix(w.part_d, 2, nb, sh, pre_lo);
  partial_prefix(w.part_d + 1, 2, nb, sh, pre_hi);
  int last_lo = -1, last_hi = -1;
  for (int b = threadIdx.x; b < nb; b += kSmpThreads) {
    last_lo = max(last_lo, load_relaxed(w.part_i + 2 * b));
    last_hi = max(last_hi, load_relaxed(w.part_i + 2 * b + 1));
  }
  last_lo = block_max_i(last_lo, red_i);
  last_hi = block_max_i(last_hi, red_i);
  const double sigma = smp_sigma(n);
  const int b_e = first_block_reaching(pre_hi, nb, 1.0 + sigma, target, red_i);
  const int b_l = first_block_reaching(pre_lo, nb, 1.0 - sigma, target, red_i);
  int id = -1;
  if (b_e == nb) {
    // The running sum certainly stays below target: the last nonzero entry.
    if (last_lo == last_hi) id = last_lo < 0 ? 0 : last_lo;  // (never empty: the top entry is kept and > 0)
  } else if (b_l < nb) {
    const Slice se = slice_of(n, b_e, nb), sl2 = slice_of(n, b_l, nb);
    const int j_e = slice_first_reach(f_hi, se.lo, se.hi, pre_hi[b_e], 1.0 + sigma, target, sh, red_i);
    const int j_l = slice_first_reach(f_lo, sl2.lo, sl2.hi, pre_lo[b_l], 1.0 - sigma, target, sh, red_i);
    if (j_l < sl2.hi && j_e == j_l) id = j_e;
  }
  if (id < 0 && s2_lo == s2_hi) {
    // Exact probabilities, the running sum's bound leaves the index open:
    // the sequential running sum.
    const int j = block_sequential_sum(f_lo, n, true, target, &seq, stage, stop);
    id = j < n ? j : (last_lo < 0 ? 0 : last_lo);
    if (threadIdx.x == 0) w.st->seq_paths |= kSeqDraw;
  }
  if (threadIdx.x == 0) {
    w.st->id = id;
    w.st->decided = id >= 0 ? 1 : 0;
    if (id >= 0 && also != nullptr) *also = id;
    if (log != nullptr) *log = SampleLog{id, id >= 0 ? 1 : 0};
    reset_counter(&w.st->counter);
  }
}

// sampling_probabilities' result, with the exact renormalisation sum.
__global__ void __launch_bounds__(kSmpThreads) smp_write(int n, SmpWork w, float* __restrict__ out) {
  const int i = blockIdx.x * kSmpThreads + threadIdx.x;
  if (i >= n) return;
  const float x = w.p[i];
  out[i] = kept(x, i, w.st->p_thr, w.st->idx_last) ? renorm(x, w.st->s2_lo) : 0.0f;
}

// ------------------------------------------------------------ ranking sort
// The ranking of smp_scale's keys (the bits of p >= +0, so key order is p
// order): descending key, ties in ascending index, i.e. the order
// std::stable_sort gives with p[a] > p[b].  A stable LSD radix sort of
// k' = ~key ascending over four 8-bit digits; each pass takes three launches
// over tiles of per_tile consecutive elements: smp_sort_hist (the tile's
// digit counts, and how many of the tile's elements have a smaller digit),
// smp_sort_scan (each digit's start in each tile: digits in order, tiles in
// order within a digit) and smp_sort_scatter (every element to its digit's
// next slot, in index order within the tile).  The first pass reads the keys
// and takes the element's index as its value, the last writes ~k' (the key
// again).  Counts are kept [digit][tile].
constexpr int kSortThreads = 256;
constexpr int kSortWaves = kSortThreads / 64;
constexpr int kSortDigits = 256;
constexpr int kSortMaxTiles = 4096;

// Exclusive prefix sum of v over the workgroup's threads in thread order
// (kSortThreads of them); *total receives the sum of all.  Ends with every
// thread past its reads of the LDS scratch.
__device__ __forceinline__ unsigned block_excl_scan(unsigned v, unsigned* scratch, unsigned* total) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  unsigned incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const unsigned u = __shfl_up(incl, o, 64);
    if (lane >= o) incl += u;
  }
  if (lane == 63) scratch[w] = incl;
  __syncthreads();
  unsigned base = 0, all = 0;
#pragma unroll
  for (int x = 0; x < kSortWaves; ++x) {
    if (x < w) base += scratch[x];
    all += scratch[x];
  }
  *total = all;
  __syncthreads();
  return base + incl - v;
}

__global__ void __launch_bounds__(kSortThreads) smp_sort_hist(const std::uint32_t* __restrict__ keys, int n,
                                                              int per_tile, int shift, int invert,
                                                              unsigned* __restrict__ hist, unsigned* __restrict__ below,
                                                              int tiles) {
  __shared__ unsigned h[kSortDigits];
  __shared__ unsigned scratch[kSortWaves];
  const int t = blockIdx.x, tid = threadIdx.x;
  h[tid] = 0;
  __syncthreads();
  const int lo = t * per_tile, hi = min(n, lo + per_tile);
  for (int i = lo + tid; i < hi; i += kSortThreads) {
    const std::uint32_t k = invert ? ~keys[i] : keys[i];
    atomicAdd(&h[(k >> shift) & 255u], 1u);
  }
  __syncthreads();
  const unsigned c = h[tid];
  unsigned all;
  const unsigned smaller = block_excl_scan(c, scratch, &all);
  hist[static_cast<std::size_t>(tid) * tiles + t] = c;
  below[static_cast<std::size_t>(tid) * tiles + t] = smaller;
}

// One workgroup per digit d: its start = the elements of all tiles with a
// smaller digit (the sum of `below` over the tiles), then hist[d][t] becomes
// that start plus the digit's count in tiles 0 .. t-1.
__global__ void __launch_bounds__(kSortThreads) smp_sort_scan(unsigned* __restrict__ hist,
                                                              const unsigned* __restrict__ below, int tiles) {
  __shared__ unsigned scratch[kSortWaves];
  const int d = blockIdx.x, tid = threadIdx.x;
  unsigned* row = hist + static_cast<std::size_t>(d) * tiles;
  const unsigned* brow = below + static_cast<std::size_t>(d) * tiles;
  unsigned part = 0;
  for (int t = tid; t < tiles; t += kSortThreads) part += brow[t];
  unsigned carry;
  (void)block_excl_scan(part, scratch, &carry);
  for (int t0 = 0; t0 < tiles; t0 += kSortThreads) {
    const int t = t0 + tid;
    const unsigned c = t < tiles ? row[t] : 0u;
    unsigned all;
    const unsigned excl = block_excl_scan(c, scratch, &all);
    if (t < tiles) row[t] = carry + excl;
    carry += all;
  }
}

// Rounds of 256 consecutive elements: a lane's rank among the lanes of its
// wavefront with the same digit from eight ballots, the wavefronts' counts
// per digit through LDS (earlier wavefronts first), then the digit's running
// position advanced by the round's count.
__global__ void __launch_bounds__(kSortThreads) smp_sort_scatter(const std::uint32_t* __restrict__ kin,
                                                                 const std::int32_t* __restrict__ iin,
                                                                 std::uint32_t* __restrict__ kout,
                                                                 std::int32_t* __restrict__ iout, int n, int per_tile,
                                                                 int shift, int first, int last,
                                                                 const unsigned* __restrict__ offs, int tiles) {
  __shared__ unsigned base[kSortDigits];
  __shared__ unsigned wcnt[kSortWaves][kSortDigits];
  const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  base[tid] = offs[static_cast<std::size_t>(tid) * tiles + t];
  const unsigned long long below = lane == 0 ? 0ull : ~0ull >> (64 - lane);
  const int lo = t * per_tile, hi = min(n, lo + per_tile);
  for (int r0 = lo; r0 < hi; r0 += kSortThreads) {
    const int i = r0 + tid;
    const bool live = i < hi;
    std::uint32_t k = 0;
    std::int32_t v = 0;
    if (live) {
      k = first ? ~kin[i] : kin[i];
      v = first ? i : iin[i];
    }
    const unsigned d = (k >> shift) & 255u;
    unsigned long long peers = __ballot(live);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const unsigned long long set = __ballot((d >> b) & 1u);
      peers &= ((d >> b) & 1u) ? set : ~set;
    }
    const unsigned rank = static_cast<unsigned>(__popcll(peers & below));
#pragma unroll
    for (int x = 0; x < kSortWaves; ++x) wcnt[x][tid] = 0;
    __syncthreads();  // zeros (and, in the first round, base) visible
    if (live && rank == 0) wcnt[w][d] = static_cast<unsigned>(__popcll(peers));
    __syncthreads();
    if (live) {
      unsigned pos = base[d] + rank;
      for (int x = 0; x < w; ++x) pos += wcnt[x][d];
      kout[pos] = last ? ~k : k;
      iout[pos] = v;
    }
    __syncthreads();  // every position taken before base moves
    unsigned sum = 0;
#pragma unroll
    for (int x = 0; x < kSortWaves; ++x) sum += wcnt[x][tid];
    base[tid] += sum;
  }
}

// Elements per tile: 1024, or more so that there are at most kSortMaxTiles.
int sort_per_tile(std::size_t n) {
  const std::size_t per = std::max<std::size_t>(1024, ceil_div(n, static_cast<std::size_t>(kSortMaxTiles)));
  return static_cast<int>(ceil_div(per, static_cast<std::size_t>(kSortThreads)) * kSortThreads);
}

// ------------------------------------------------------------------- host
struct SmpBuffers {
  std::size_t cap = 0;
  void* base = nullptr;
  std::uint32_t* sort_keys = nullptr;  // the ranking sort's second buffer of keys,
  std::int32_t* sort_idx = nullptr;    // of indices,
  unsigned* sort_hist = nullptr;       // and its digit counts ([digit][tile])
  unsigned* sort_below = nullptr;      // and the tiles' counts of smaller digits
  float* host_io = nullptr;  // staging for the host-pointer entry points (device)
  std::int32_t* id_dev = nullptr;
  SmpWork w{};
};
SmpBuffers g_smp;
bool g_exact_only = false;

int smp_reserve(std::size_t n, hipStream_t s) {
  if (n <= g_smp.cap) return LLMI_OK;
  LLMI_TRY_HIP(hipStreamSynchronize(s));
  if (g_smp.base != nullptr) LLMI_TRY_HIP(hipFree(g_smp.base));
  g_smp = SmpBuffers{};
  const std::size_t tiles = ceil_div(n, static_cast<std::size_t>(sort_per_tile(n)));
  auto al = [](std::size_t b) { return (b + 255) & ~static_cast<std::size_t>(255); };
  // The top-k selection writes up to kCandMax candidates into keys / idx.
  const std::size_t vn = n > static_cast<std::size_t>(kCandMax) ? n : static_cast<std::size_t>(kCandMax);
  const std::size_t vec = al(vn * 4);
  const std::size_t bytes = 9 * vec + 2 * al(sizeof(unsigned) * kSortDigits * tiles) +
                            al(sizeof(double) * 2 * kSmpBlocks) + al(sizeof(int) * 2 * kSmpBlocks) +
                            al(sizeof(float) * kSmpBlocks) + al(sizeof(SmpState)) + al(sizeof(std::int32_t));
  LLMI_TRY_HIP(hipMalloc(&g_smp.base, bytes));
  char* c = static_cast<char*>(g_smp.base);
  auto take = [&c, &al](std::size_t b) {
    void* r = c;
    c += al(b);
    return r;
  };
  SmpWork& w = g_smp.w;
  w.p = static_cast<float*>(take(vn * 4));
  w.keys = static_cast<std::uint32_t*>(take(vn * 4));
  w.keys_sorted = static_cast<std::uint32_t*>(take(vn * 4));
  w.idx = static_cast<std::int32_t*>(take(vn * 4));
  w.idx_sorted = static_cast<std::int32_t*>(take(vn * 4));
  g_smp.host_io = static_cast<float*>(take(vn * 4));
  (void)take(vn * 4);  // spare
  g_smp.sort_keys = static_cast<std::uint32_t*>(take(vn * 4));
  g_smp.sort_idx = static_cast<std::int32_t*>(take(vn * 4));
  g_smp.sort_hist = static_cast<unsigned*>(take(sizeof(unsigned) * kSortDigits * tiles));
  g_smp.sort_below = static_cast<unsigned*>(take(sizeof(unsigned) * kSortDigits * tiles));
  w.part_d = static_cast<double*>(take(sizeof(double) * 2 * kSmpBlocks));
  w.part_i = static_cast<int*>(take(sizeof(int) * 2 * kSmpBlocks));
  w.part_f = static_cast<float*>(take(sizeof(float) * kSmpBlocks));
  w.st = static_cast<SmpState*>(take(sizeof(SmpState)));
  g_smp.id_dev = static_cast<std::int32_t*>(take(sizeof(std::int32_t)));
  LLMI_TRY_HIP(hipMemsetAsync(w.st, 0, sizeof(SmpState), s));
  g_smp.cap = n;
  return LLMI_OK;
}

int smp_check_cfg(const llmi_hip_sampling* cfg, std::size_t n) {
  LLMI_REQUIRE(cfg != nullptr, "sampling: null config");
  LLMI_REQUIRE(n >= 1 && n <= (std::size_t{1} << 28), "sampling: need 1 <= n <= 2^28 logits");
  return LLMI_OK;
}

// The ranking of keys[0, n) into keys_sorted / idx_sorted (the sort kernels
// above): passes 0 and 2 write the sort's own buffers, 1 and 3 the sorted
// ones; keys is only read.
int smp_sort(std::size_t n, hipStream_t s) {
  const SmpWork& w = g_smp.w;
  const int ni = static_cast<int>(n), per = sort_per_tile(n);
  const int tiles = static_cast<int>(ceil_div(n, static_cast<std::size_t>(per)));
  LLMI_REQUIRE(n <= g_smp.cap && tiles <= kSortMaxTiles, "sampling: ranking larger than its workspace");
  const std::uint32_t* kin = w.keys;
  const std::int32_t* iin = nullptr;
  for (int pass = 0; pass < 4; ++pass) {
    std::uint32_t* kout = pass % 2 == 0 ? g_smp.sort_keys : w.keys_sorted;
    std::int32_t* iout = pass % 2 == 0 ? g_smp.sort_idx : w.idx_sorted;
    smp_sort_hist<<<tiles, kSortThreads, 0, s>>>(kin, ni, per, 8 * pass, pass == 0 ? 1 : 0, g_smp.sort_hist,
                                                 g_smp.sort_below, tiles);
    smp_sort_scan<<<kSortDigits, kSortThreads, 0, s>>>(g_smp.sort_hist, g_smp.sort_below, tiles);
    smp_sort_scatter<<<tiles, kSortThreads, 0, s>>>(kin, iin, kout, iout, ni, per, 8 * pass, pass == 0 ? 1 : 0,
                                                    pass == 3 ? 1 : 0, g_smp.sort_hist, tiles);
    kin = kout;
    iin = iout;
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

// What smp_front passes to the merge kernel's draw: with the top-k select
// (top_k <= kSelectMax) the draw is exact there and smp_draw is not needed.
struct FrontDraw {
  double target;
  std::int32_t* also;
  SampleLog* log;
};

// Everything up to and including smp_keep.  *ranked: whether the ranking
// (keys_sorted / idx_sorted) was built.  *drawn: whether the select path
// already drew the index for `draw` (null: no draw wanted).
int smp_front(const float* logits, std::size_t n, const llmi_hip_sampling& cfg, bool need_ranking, hipStream_t s,
              bool* ranked, bool* drawn, const FrontDraw* draw = nullptr, SampleLog* log = nullptr) {
  const int ni = static_cast<int>(n);
  const std::size_t k = cfg.top_k == 0 || cfg.top_k > n ? n : cfg.top_k;
  const bool filtering = k < n || cfg.top_p < 1.0f;
  *ranked = filtering || need_ranking;
  *drawn = false;
  SmpWork& w = g_smp.w;
  smp_max<<<kSmpBlocks, kSmpThreads, 0, s>>>(logits, ni, cfg.temperature, w, log);
  smp_exp<<<kSmpBlocks, kSmpThreads, 0, s>>>(logits, ni, cfg.temperature, w);
  LLMI_TRY_HIP(hipGetLastError());
  if (*ranked && k < n && k <= static_cast<std::size_t>(kSelectMax)) {
    // Only the first k of the ranking are read: select them.
    const int ki = static_cast<int>(k);
    smp_sel_local<<<kSmpBlocks, kSmpThreads, 0, s>>>(ni, ki, w);
    smp_sel_merge<<<1, kMergeThreads, 0, s>>>(ki, cfg.top_p, draw != nullptr ? draw->target : 0.0,
                                              draw != nullptr ? 1 : 0, w, draw != nullptr ? draw->also : nullptr, log);
    *drawn = draw != nullptr;
  } else if (*ranked) {
    smp_scale<<<static_cast<unsigned>(ceil_div(n, kSmpThreads)), kSmpThreads, 0, s>>>(ni, w, 1);
    if (int rc = smp_sort(n, s)) return rc;
    smp_keep<<<kSmpBlocks, kSmpThreads, 0, s>>>(reinterpret_cast<const float*>(w.keys_sorted), w.idx_sorted,
                                                static_cast<int>(k), ni, cfg.top_p, 1, w);
  } else {
    smp_keep<<<kSmpBlocks, kSmpThreads, 0, s>>>(w.p, nullptr, ni, ni, 2.0f, 0, w);
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

int smp_read_state(SmpState* st, hipStream_t s) {
  LLMI_TRY_HIP(hipMemcpyAsync(st, g_smp.w.st, sizeof(SmpState), hipMemcpyDeviceToHost, s));
  LLMI_TRY_HIP(hipStreamSynchronize(s));
  return LLMI_OK;
}

int smp_bad_input(const SmpState& st) {
  if (st.flags & kFlagNaN) return fail(LLMI_ERR_ARG, "sampling: logits / temperature has a NaN entry");
  return fail(LLMI_ERR_ARG, "sampling: logits / temperature has a +inf entry");
}

}  // namespace

void release_sampling_workspace() {
  if (g_smp.base != nullptr) (void)hipFree(g_smp.base);
  g_smp = SmpBuffers{};
}

// Draws one index on the device; *id_host receives it.  `also` (device, may
// be null) receives it too, on the stream, before the host learns it.
int sample_device(const float* logits, std::size_t n, const llmi_hip_sampling& cfg, double target,
                  std::int32_t* id_host, std::int32_t* also, hipStream_t s) {
  if (int rc = smp_check_cfg(&cfg, n)) return rc;
  if (int rc = smp_reserve(n, s)) return rc;
  if (cfg.temperature <= 0.0f) {  // sampling.cpp:61: the first maximum, nothing drawn
    std::int32_t* dst = also != nullptr ? also : g_smp.id_dev;
    smp_argmax<<<kSmpBlocks, kSmpThreads, 0, s>>>(logits, static_cast<int>(n), g_smp.w, dst);
    LLMI_TRY_HIP(hipGetLastError());
    LLMI_TRY_HIP(hipMemcpyAsync(id_host, dst, sizeof(std::int32_t), hipMemcpyDeviceToHost, s));
    LLMI_TRY_HIP(hipStreamSynchronize(s));
    return LLMI_OK;
  }
  bool ranked = false, drawn = false;
  const FrontDraw fd{target, also, nullptr};
  if (int rc = smp_front(logits, n, cfg, g_exact_only, s, &ranked, &drawn, &fd)) return rc;
  SmpWork& w = g_smp.w;
  const int ni = static_cast<int>(n);
  if (!drawn) {
    if (g_exact_only) smp_seq_sum2<<<1, kSmpThreads, 0, s>>>(reinterpret_cast<const float*>(w.keys_sorted), w);
    smp_draw<<<kSmpBlocks, kSmpThreads, 0, s>>>(ni, target, ranked ? 1 : 0, w, also, nullptr);
  }
  LLMI_TRY_HIP(hipGetLastError());
  SmpState st{};
  if (int rc = smp_read_state(&st, s)) return rc;
  if (st.flags & kFlagAllNegInf) {
    // Every logit is -inf: the reference's probabilities are NaN and its
    // draw falls through to argmax(logits), the first entry.
    *id_host = 0;
    if (also != nullptr) LLMI_TRY_HIP(hipMemcpyAsync(also, id_host, sizeof(std::int32_t), hipMemcpyHostToDevice, s));
    LLMI_TRY_HIP(hipStreamSynchronize(s));
    return LLMI_OK;
  }
  if (st.flags & kFlagBad) return smp_bad_input(st);
  if (!st.decided) {
    // The exact renormalisation sum, which needs the ranking.
    if (!ranked) {
      smp_keys<<<static_cast<unsigned>(ceil_div(n, kSmpThreads)), kSmpThreads, 0, s>>>(ni, w);
      LLMI_TRY_HIP(hipGetLastError());
      if (int rc = smp_sort(n, s)) return rc;
    }
    smp_seq_sum2<<<1, kSmpThreads, 0, s>>>(reinterpret_cast<const float*>(w.keys_sorted), w);
    smp_draw<<<kSmpBlocks, kSmpThreads, 0, s>>>(ni, target, ranked ? 1 : 0, w, also, nullptr);
    LLMI_TRY_HIP(hipGetLastError());
    if (int rc = smp_read_state(&st, s)) return rc;
    if (!st.decided) return fail(LLMI_ERR_STATE, "sampling: the exact draw did not decide (internal error)");
  }
  *id_host = st.id;
  return LLMI_OK;
}

// sample_device's kernels without the read-back: the drawn index goes to
// `also` (device) and, with the state, to *log; a step whose log says
// undecided (state bit 0 clear: a bound left the index open, or the logits
// were bad) must be redrawn through sample_device.  temperature > 0 only.
int sample_device_async(const float* logits, std::size_t n, const llmi_hip_sampling& cfg, double target,
                        std::int32_t* also, SampleLog* log, hipStream_t s) {
  if (int rc = smp_check_cfg(&cfg, n)) return rc;
  LLMI_REQUIRE(cfg.temperature > 0.0f, "sampling: the asynchronous draw needs temperature > 0");
  if (int rc = smp_reserve(n, s)) return rc;
  bool ranked = false, drawn = false;
  const FrontDraw fd{target, also, log};
  if (int rc = smp_front(logits, n, cfg, g_exact_only, s, &ranked, &drawn, &fd, log)) return rc;
  SmpWork& w = g_smp.w;
  const int ni = static_cast<int>(n);
  if (!drawn) {
    if (g_exact_only) smp_seq_sum2<<<1, kSmpThreads, 0, s>>>(reinterpret_cast<const float*>(w.keys_sorted), w);
    smp_draw<<<kSmpBlocks, kSmpThreads, 0, s>>>(ni, target, ranked ? 1 : 0, w, also, log);
  }
  LLMI_TRY_HIP(hipGetLastError());
  return LLMI_OK;
}

}  // namespace llmi_hip

using namespace llmi_hip;

int llmi_hip_sample_dev(const float* logits, size_t n, const llmi_hip_sampling* cfg, double target, int32_t* id,
                        void* stream) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(logits != nullptr && id != nullptr, "sample: null pointer");
  if (int rc = smp_check_cfg(cfg, n)) return rc;
  return sample_device(logits, n, *cfg, target, id, nullptr, pick(stream));
}

int llmi_hip_sample(const float* logits, size_t n, const llmi_hip_sampling* cfg, double target, int32_t* id) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(logits != nullptr && id != nullptr, "sample: null pointer");
  if (int rc = smp_check_cfg(cfg, n)) return rc;
  hipStream_t s = library_stream();
  if (int rc = smp_reserve(n, s)) return rc;
  LLMI_TRY_HIP(hipMemcpyAsync(g_smp.host_io, logits, n * sizeof(float), hipMemcpyHostToDevice, s));
  return sample_device(g_smp.host_io, n, *cfg, target, id, nullptr, s);
}

int llmi_hip_sampling_probabilities(const float* logits, size_t n, const llmi_hip_sampling* cfg, float* probs) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(logits != nullptr && probs != nullptr, "sampling_probabilities: null pointer");
  if (int rc = smp_check_cfg(cfg, n)) return rc;
  hipStream_t s = library_stream();
  if (int rc = smp_reserve(n, s)) return rc;
  const std::size_t k = cfg->top_k == 0 || cfg->top_k > n ? n : cfg->top_k;
  float* dev_in = g_smp.host_io;
  LLMI_TRY_HIP(hipMemcpyAsync(dev_in, logits, n * sizeof(float), hipMemcpyHostToDevice, s));
  if (cfg->temperature <= 0.0f) {  // sampling.cpp:13-19: all mass on the first maximum
    std::int32_t best = 0;
    if (int rc = llmi_hip_argmax_dev(dev_in, n, g_smp.id_dev, s)) return rc;
    LLMI_TRY_HIP(hipMemcpyAsync(&best, g_smp.id_dev, sizeof(best), hipMemcpyDeviceToHost, s));
    LLMI_TRY_HIP(hipStreamSynchronize(s));
    std::fill(probs, probs + n, 0.0f);
    probs[best] = 1.0f;
    return LLMI_OK;
  }
  bool ranked = false, drawn = false;
  if (int rc = smp_front(dev_in, n, *cfg, true, s, &ranked, &drawn)) return rc;
  SmpWork& w = g_smp.w;
  smp_seq_sum2<<<1, kSmpThreads, 0, s>>>(reinterpret_cast<const float*>(w.keys_sorted), w);
  float* out = reinterpret_cast<float*>(w.keys);  // the keys are no longer needed
  smp_write<<<static_cast<unsigned>(ceil_div(n, kSmpThreads)), kSmpThreads, 0, s>>>(static_cast<int>(n), w, out);
  LLMI_TRY_HIP(hipGetLastError());
  SmpState st{};
  if (int rc = smp_read_state(&st, s)) return rc;
  if (st.flags & kFlagAllNegInf) {
    // Every logit is -inf: the reference's softmax gives NaN everywhere, its
    // ranking keeps index order and nothing is renormalised (sum > 0 fails).
    for (std::size_t i = 0; i < n; ++i) probs[i] = i < k ? __builtin_nanf("") : 0.0f;
    return LLMI_OK;
  }
  if (st.flags & kFlagBad) return smp_bad_input(st);
  LLMI_TRY_HIP(hipMemcpy(probs, out, n * sizeof(float), hipMemcpyDeviceToHost));
  return LLMI_OK;
}

int llmi_hip_sampling_set_exact_only(int on) {
  g_exact_only = on != 0;
  return LLMI_OK;
}

int llmi_hip_sampling_last_paths(int* paths) {
  LLMI_REQUIRE_INIT();
  LLMI_REQUIRE(paths != nullptr, "sampling_last_paths: null pointer");
  *paths = 0;
  if (g_smp.w.st == nullptr) return LLMI_OK;
  SmpState st{};
  if (int rc = smp_read_state(&st, library_stream())) return rc;
  *paths = st.seq_paths;
  return LLMI_OK;
}
