// Codebook calibration on the device: fit_codebook
// (src/alelyon_compute_kit/_kit/python/vq.py:182-257) as a chain of kernels
// that needs no host round trip, bit-identical to the reference's Python and
// to host_fit.cpp.
//
// One fit (a "problem") per blockIdx.y (assign) or blockIdx.x (the
// single-block kernels); the fused VQAdamW step runs its three state fits as
// three problems of the same launches. Per iteration:
//   assign  one lane per sample vector: float64 nearest entry, the used mask;
//   keep    (only when a warm start fits a sample smaller than the tensor)
//           each block first decides the warm-start keep rule's condition
//           (vq.py:216-222: some entry the sample never selected is not a
//           copy of an earlier entry); when it holds, the whole tensor's
//           float64 nearest entries;
//   update  one 1024-lane block: the members are grouped by entry and summed
//           in float64 (numpy's axis-0 mean), by all waves in any order
//           when no partial sum can round, else by the entry's own wave in
//           sample order;
//           then entries in ascending order take their mean, or, when empty
//           and not kept, the sample vector farthest from the book as it
//           stands at that moment (vq.py:232-257).
// The mean's sum order is sequential per component, as numpy sums axis 0.
// The reseed distance sums the G squared differences in numpy's pairwise
// order (eight interleaved partial sums), and its argmax takes the first
// maximum or the first NaN.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <climits>
#include <cstdint>

#include "fit_device.hpp"
#include "kernels.hpp"

namespace ackvq {
namespace {

using fitdev::linspace_at;
using fitdev::nearest64;

constexpr uint32_t kAssignThreads = 256;
constexpr uint32_t kUpdateThreads = 1024;  // 16 waves: wave e owns entry e
constexpr uint32_t kStageBytes = 131072;    // sample rows staged per round in update (all of a
                                             // 4,096-vector group-8 sample)

__device__ __forceinline__ bool finite_f32(float x) { return fabsf(x) <= FLT_MAX; }

template <int G>
__device__ __forceinline__ const float* sample_of(const FitArgs& a, uint32_t p) {
  return a.sample + uint64_t(p) * a.count * G;
}

// Rows linspace(0, complete-1, count) of a dense tensor; one lane per value.
// Block 0 also sets up the (one-problem) fit as k_fit_init does: the starting
// book (init, or sample rows linspace(0, count-1, 16), read straight from the
// tensor) and cleared flags, saving that launch.
template <int G>
__global__ __launch_bounds__(256) void k_fit_sample_dense(const float* values, FitArgs a,
                                                          const float* init) {
  float* out = const_cast<float*>(a.sample);
  const uint32_t total = a.count * G;
  bool bad = false;
  for (uint32_t e = blockIdx.x * 256 + threadIdx.x; e < total; e += gridDim.x * 256) {
    const uint32_t row = linspace_at(a.complete, a.count, e / G);
    const float v = values[uint64_t(row) * G + e % G];
    bad |= !finite_f32(v);
    out[e] = v;
  }
  if (blockIdx.x == 0) {
    for (uint32_t i = threadIdx.x; i < 16 * G; i += 256) {
      float v;
      if (init != nullptr) {
        v = init[i];
        bad |= !finite_f32(v);
      } else {
        const uint32_t row = linspace_at(a.complete, a.count, linspace_at(a.count, 16, i / G));
        v = values[uint64_t(row) * G + i % G];
      }
      a.book[i] = v;
    }
    if (threadIdx.x < 4) a.flags[threadIdx.x] = 0;
  }
  if (__any(bad) && (threadIdx.x % warpSize) == 0) atomicOr(a.status, 1u);
}

// Starting book: init, or sample rows linspace(0, count-1, 16) (vq.py:208-213);
// clears the masks. One block per problem.
template <int G>
__global__ __launch_bounds__(256) void k_fit_init(FitArgs a, const float* init) {
  const uint32_t p = blockIdx.x;
  float* book = a.book + p * 16 * G;
  const float* sample = sample_of<G>(a, p);
  bool bad = false;
  for (uint32_t i = threadIdx.x; i < 16 * G; i += 256) {
    float v;
    if (init != nullptr) {
      v = init[p * 16 * G + i];
      bad |= !finite_f32(v);
    } else {
      v = sample[uint64_t(linspace_at(a.count, 16, i / G)) * G + i % G];
    }
    book[i] = v;
  }
  if (threadIdx.x < 4) a.flags[p * 4 + threadIdx.x] = 0;
  if (__any(bad) && (threadIdx.x % warpSize) == 0) atomicOr(a.status, 1u);
}

template <int G>
__device__ __forceinline__ void load_book64(const float* book, double* sbook) {
  for (uint32_t i = threadIdx.x; i < 16 * G; i += blockDim.x) sbook[i] = double(book[i]);
}

// Nearest entry of every sample vector (vq.py:214); the used mask.
template <int G>
__global__ __launch_bounds__(kAssignThreads) void k_fit_assign(FitArgs a) {
  const uint32_t p = blockIdx.y;
  __shared__ double sbook[16 * G];
  load_book64<G>(a.book + p * 16 * G, sbook);
  __syncthreads();
  if (blockIdx.x == 0)  // the keep pass reads the book as float64 from here
    for (uint32_t i = threadIdx.x; i < 16 * G; i += kAssignThreads) a.book64[p * 16 * G + i] = sbook[i];
  const float* sample = sample_of<G>(a, p);
  uint8_t* idx = a.idx + uint64_t(p) * a.count;
  uint32_t used = 0;
  for (uint32_t i = blockIdx.x * kAssignThreads + threadIdx.x; i < a.count;
       i += gridDim.x * kAssignThreads) {
    double x[G];
    const float4* row = reinterpret_cast<const float4*>(sample + uint64_t(i) * G);
#pragma unroll
    for (int q = 0; q < G / 4; ++q) {
      const float4 v = row[q];
      x[4 * q] = v.x; x[4 * q + 1] = v.y; x[4 * q + 2] = v.z; x[4 * q + 3] = v.w;
    }
    const uint32_t e = nearest64<G>(x, sbook);
    idx[i] = uint8_t(e);
    used |= 1u << e;
  }
  for (int off = 1; off < warpSize; off <<= 1) used |= __shfl_xor(used, off);
  if (used && (threadIdx.x % warpSize) == 0) atomicOr(&a.flags[p * 4], used);
}

// The keep pass over a dense tensor (one problem): entries its complete
// vectors select under the current book.
template <int G>
__global__ __launch_bounds__(256) void k_fit_keep_dense(FitArgs a, const float* values) {
  __shared__ float sbk[16 * G];
  __shared__ uint32_t scand[1];
  fitdev::keep_candidates<G>(a.book, a.flags, 1, sbk, scand);
  if (scand[0] == 0) return;
  const double* __restrict__ book64 = a.book64;
  __shared__ uint32_t bused;
  if (threadIdx.x == 0) bused = 0;
  __syncthreads();
  uint32_t used = 0;
  for (uint64_t v = uint64_t(blockIdx.x) * 256 + threadIdx.x; v < a.complete;
       v += uint64_t(gridDim.x) * 256) {
    double x[G];
#pragma unroll
    for (int j = 0; j < G; ++j) x[j] = double(values[v * G + j]);
    used |= 1u << fitdev::nearest64_uniform<G>(x, book64);
  }
  // one global atomic per block, and none when its bits are already set
  for (int off = 1; off < warpSize; off <<= 1) used |= __shfl_xor(used, off);
  if (used && (threadIdx.x % warpSize) == 0) atomicOr(&bused, used);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t seen = __hip_atomic_load(&a.flags[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (bused & ~seen) atomicOr(&a.flags[1], bused);
  }
}

// numpy's pairwise sum of the G >= 8 squared differences (G a multiple of
// 8) between x (float64) and an entry (float64, or float32 converted
// exactly): eight interleaved partial sums r[j % 8] taken in j order,
// combined ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)).
template <int G, typename T>
__device__ __forceinline__ double pairwise_gap(const double (&x)[G], const T* entry) {
  double r[8];
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const double d = x[j] - double(entry[j]);
    const double sq = d * d;
    r[j % 8] = j < 8 ? sq : r[j % 8] + sq;
  }
  return ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
}

// The gap rule of vq.py:254-256 over several entries: a NaN distance wins,
// else the smallest. Held as the smallest gap that is not NaN and a flag for
// NaN; gaps are sums of squares, never -0, so neither depends on the order
// gaps arrive in (and fmin's choice when one operand is NaN never shows).
struct Nearest {
  double lo;
  uint32_t nan;  // nonzero once a NaN gap arrived: a lane value, kept off the scalar unit
  __device__ __forceinline__ void add(double gap) {
    lo = fmin(lo, gap);
    nan |= uint32_t(gap != gap);
  }
  __device__ __forceinline__ double value() const {
    return nan ? __longlong_as_double(0x7ff8000000000000ll) : lo;
  }
};
__device__ __forceinline__ Nearest nearest_of(double gap) {
  return Nearest{gap, uint32_t(gap != gap)};
}
__device__ __forceinline__ Nearest nearest_none() {
  return Nearest{__longlong_as_double(0x7ff0000000000000ll), 0u};
}

// The first reseed's hi for one row: the gaps of the untouched entries
// [e, 16) but the twins, storing hi over [e', 16) for each e' in `store`.
// Visits only the entries that need a gap or a store, highest first.
template <int G>
__device__ __forceinline__ double untouched_gap(const double (&x)[G], const double* cur64,
                                                uint32_t e, uint32_t twin, uint32_t store,
                                                double* suffix, uint32_t count, uint32_t i) {
  Nearest hi = nearest_none();
  uint32_t todo = (~twin | store) & (0xffffu << e) & 0xffffu;
  while (todo) {
    const uint32_t ee = 31u - uint32_t(__builtin_clz(todo));
    todo &= ~(1u << ee);
    if (!((twin >> ee) & 1u)) hi.add(pairwise_gap<G>(x, cur64 + ee * G));
    if ((store >> ee) & 1u) suffix[uint64_t(ee) * count + i] = hi.value();
  }
  return hi.value();
}

// A row's gap to the whole book, every entry measured (a reseed that no later
// reseed follows keeps nothing for later).
template <int G>
__device__ __forceinline__ double book_gap(const double (&x)[G], const double* cur64) {
  Nearest g = nearest_none();
  // two entries a step for group 8, one for wider rows: unrolled further,
  // the compiler holds every entry's float64 row in registers at once
  constexpr int kStep = G == 8 ? 2 : 1;
#pragma unroll kStep
  for (uint32_t ee = 0; ee < 16; ++ee) g.add(pairwise_gap<G>(x, cur64 + ee * G));
  return g.value();
}

template <int G>
__device__ __forceinline__ void row_as_double(const float* sample, uint32_t i, double (&x)[G]) {
  const float4* row = reinterpret_cast<const float4*>(sample + uint64_t(i) * G);
#pragma unroll
  for (int q = 0; q < G / 4; ++q) {
    const float4 v = row[q];
    x[4 * q] = v.x; x[4 * q + 1] = v.y; x[4 * q + 2] = v.z; x[4 * q + 3] = v.w;
  }
}

// The argmax rule of vq.py:257 (the first NaN if any, else the largest gap,
// ties to the lower row) on integer keys: a gap is >= +0 (a sum of squares)
// or NaN, so its bit pattern orders as the value, and NaN maps above every
// gap; equal keys go to the lower row. "None" is key 0 with row 0xffffffff,
// which any row beats.
struct FarKey {
  uint64_t key;
  uint32_t row;
};
__device__ __forceinline__ uint64_t far_key(double gap) {
  return gap != gap ? ~0ull : uint64_t(__double_as_longlong(gap));
}
__device__ __forceinline__ FarKey farther_key(FarKey a, FarKey b) {
  return (a.key > b.key || (a.key == b.key && a.row < b.row)) ? a : b;
}
__device__ __forceinline__ FarKey shfl_xor_key(FarKey v, int off) {
  FarKey o;
  o.key = uint64_t(__shfl_xor(static_cast<unsigned long long>(v.key), off));
  o.row = uint32_t(__shfl_xor(int(v.row), off));
  return o;
}
// The block's farthest row: a butterfly within each wave, then one over the
// 16 wave results; every thread returns the same row. Consecutive calls
// alternate between two scratch halves: a wave reaches the call after next
// only past the next call's barrier, which every wave reaches after reading
// this one's half, so no barrier guards the reuse.
__device__ __forceinline__ uint32_t block_farthest(FarKey best, FarKey* scratch) {
  for (int off = 1; off < warpSize; off <<= 1) best = farther_key(best, shfl_xor_key(best, off));
  const uint32_t lane = threadIdx.x % warpSize;
  if (lane == 0) scratch[threadIdx.x / warpSize] = best;
  __syncthreads();
  constexpr uint32_t kWaves = kUpdateThreads / 64;
  FarKey all = lane < kWaves ? scratch[lane] : FarKey{0, 0xffffffffu};
  for (int off = 1; off < int(kWaves); off <<= 1) all = farther_key(all, shfl_xor_key(all, off));
  return uint32_t(__shfl(int(all.row), 0));
}

// _reseed (vq.py:232-257) of entry e for the whole block: the sample row whose
// nearest entry of the book as it stands (`cur64`: entries below e already
// updated this iteration, the others as they were) is farthest. Every thread
// returns the same row.
//
// A row's gap is the nearer of near, over the updated entries [0, e), and hi,
// over the untouched entries [e, 16). The first reseed of an iteration
// (`first`) measures both. A later reseed at e measures only the entries
// updated since the previous one ([done, e); entry `done`, the previous
// reseed's row, read from the sample at `done_row`) and takes hi over [e, 16) from
// suffix[head], which the first reseed stored. An untouched entry with a
// bitwise copy at a higher index (bit set in `twin`) has that copy's gap, so
// a minimum over a range that runs to 16 need not measure it, and two
// reseeds with only such entries between them share one hi. `store` names
// the entries e' whose hi over [e', 16) the first reseed stores. A first
// reseed that no later one follows (`single`) measures the whole book in one
// unrolled pass and keeps nothing.
template <int G>
__device__ uint32_t reseed_row(const float* sample, uint32_t count, const double* cur64,
                               uint32_t e, uint32_t done, const float* done_row, bool first,
                               bool single, uint32_t twin, uint32_t store, uint32_t head,
                               double* near, double* suffix, FarKey* scratch) {
  FarKey best{0, 0xffffffffu};
  for (uint32_t i = threadIdx.x; i < count; i += kUpdateThreads) {
    double x[G];
    row_as_double<G>(sample, i, x);
    if (single) {
      best = farther_key(best, FarKey{far_key(book_gap<G>(x, cur64)), i});
      continue;
    }
    Nearest lo = first ? nearest_none() : nearest_of(near[i]);
    if (!first) lo.add(pairwise_gap<G>(x, done_row));
#pragma unroll 1
    for (uint32_t ee = first ? 0 : done + 1; ee < e; ++ee)
      lo.add(pairwise_gap<G>(x, cur64 + ee * G));
    near[i] = lo.value();
    lo.add(first ? untouched_gap<G>(x, cur64, e, twin, store, suffix, count, i)
                 : suffix[uint64_t(head) * count + i]);
    best = farther_key(best, FarKey{far_key(lo.value()), i});
  }
  return block_farthest(best, scratch);
}

// reseed_row for samples of at most kRegRows rows per thread: each thread
// keeps near and hi of its rows (t, t + kUpdateThreads, ...) in registers
// across the iteration's reseeds; a later reseed reads a stored hi only when
// `reload` (an entry between it and the previous reseed counts), and issues
// those reads before any gap arithmetic. Same rows, same values, same choice
// as reseed_row.
constexpr uint32_t kRegRows = 4;
template <int G>
__device__ uint32_t reseed_row_regs(const float* sample, uint32_t count, const double* cur64,
                                    uint32_t e, uint32_t done, const float* done_row,
                                    bool first, bool single, bool reload, uint32_t twin,
                                    uint32_t store,
                                    double (&near_r)[kRegRows], double (&hi_r)[kRegRows],
                                    double* suffix, FarKey* scratch) {
  static_assert(G == 8, "four rows of a wider group do not fit in registers");
  FarKey best{0, 0xffffffffu};
  if (reload) {
#pragma unroll
    for (uint32_t r = 0; r < kRegRows; ++r) {
      const uint32_t i = threadIdx.x + r * kUpdateThreads;
      hi_r[r] = i < count ? suffix[uint64_t(e) * count + i] : 0.0;
    }
  }
#pragma unroll
  for (uint32_t r = 0; r < kRegRows; ++r) {
    const uint32_t i = threadIdx.x + r * kUpdateThreads;
    if (i >= count) break;
    double x[G];
    row_as_double<G>(sample, i, x);
    if (single) {
      best = farther_key(best, FarKey{far_key(book_gap<G>(x, cur64)), i});
      continue;
    }
    Nearest lo = first ? nearest_none() : nearest_of(near_r[r]);
    if (!first) lo.add(pairwise_gap<G>(x, done_row));
#pragma unroll 1
    for (uint32_t ee = first ? 0 : done + 1; ee < e; ++ee)
      lo.add(pairwise_gap<G>(x, cur64 + ee * G));
    near_r[r] = lo.value();
    if (first) hi_r[r] = untouched_gap<G>(x, cur64, e, twin, store, suffix, count, i);
    lo.add(hi_r[r]);
    best = farther_key(best, FarKey{far_key(lo.value()), i});
  }
  return block_farthest(best, scratch);
}

// A reseed that no later one follows, over a staged sample (`rows` in LDS,
// `ids` each row's entry from the assign pass). A row's gap to its own
// entry, U, bounds its nearest gap g from above (the same float64 steps, over
// one of the 16 entries). Each wave's row of largest U is measured exactly
// (256 lanes: 16 rows x 16 entries), and T is the largest of those 16 g.
// Every row that can win or tie has g >= T, so U >= T: only those rows,
// listed in `list`, are measured against the whole book. A NaN U, or a NaN
// T, keeps a row on the list. Same row as measuring every row. `wrow` holds
// 16 row numbers, `sgap` 256 gaps and T.
template <int G>
__device__ __noinline__ uint32_t lone_reseed(const float* rows, const uint8_t* ids,
                                             uint32_t count, const double* cur64,
                                             uint16_t* list, uint32_t* nlist, double* sgap,
                                             uint32_t* wrow, FarKey* scratch) {
  const uint32_t lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  FarKey best{0, 0xffffffffu};
  for (uint32_t i = threadIdx.x; i < count; i += kUpdateThreads) {
    double x[G];
    row_as_double<G>(rows, i, x);
    best = farther_key(best, FarKey{far_key(pairwise_gap<G>(x, cur64 + uint32_t(ids[i]) * G)), i});
  }
  for (int off = 1; off < warpSize; off <<= 1) best = farther_key(best, shfl_xor_key(best, off));
  if (lane == 0) wrow[wave] = best.row < count ? best.row : 0u;  // a wave with no row: row 0
  if (threadIdx.x == 0) *nlist = 0;
  __syncthreads();
  if (threadIdx.x < 256) {
    double x[G];
    row_as_double<G>(rows, wrow[threadIdx.x / 16], x);
    sgap[threadIdx.x] = pairwise_gap<G>(x, cur64 + (threadIdx.x % 16) * G);
  }
  __syncthreads();
  if (threadIdx.x < 64) {  // T: the largest exact g of the 16 rows, NaN if any is NaN
    double v = 0.0;
    uint32_t vnan = 0;
    if (lane < 16) {
      Nearest g = nearest_none();
      for (uint32_t q = 0; q < 16; ++q) g.add(sgap[lane * 16 + q]);
      v = g.lo;
      vnan = g.nan;
    }
    for (int off = 1; off < 16; off <<= 1) {
      v = fmax(v, __shfl_xor(v, off));
      vnan |= uint32_t(__shfl_xor(int(vnan), off));
    }
    if (lane == 0) sgap[256] = vnan ? __longlong_as_double(0x7ff8000000000000ll) : v;
  }
  __syncthreads();
  const double T = sgap[256];
  for (uint32_t i0 = 0; i0 < count; i0 += kUpdateThreads) {  // whole waves: the list by ballot
    const uint32_t i = i0 + threadIdx.x;
    bool keep = false;
    if (i < count) {
      double x[G];
      row_as_double<G>(rows, i, x);
      keep = !(pairwise_gap<G>(x, cur64 + uint32_t(ids[i]) * G) < T);
    }
    const uint64_t bal = __ballot(keep);
    uint32_t base = 0;
    if (lane == 0 && bal != 0) base = atomicAdd(nlist, uint32_t(__popcll(bal)));
    base = uint32_t(__shfl(int(base), 0));
    const uint32_t rank =
        __builtin_amdgcn_mbcnt_hi(uint32_t(bal >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(bal), 0u));
    if (keep) list[base + rank] = uint16_t(i);
  }
  __syncthreads();
  const uint32_t n = *nlist;
  FarKey win{0, 0xffffffffu};
  for (uint32_t k = threadIdx.x; k < n; k += kUpdateThreads) {
    const uint32_t i = list[k];
    double x[G];
    row_as_double<G>(rows, i, x);
    win = farther_key(win, FarKey{far_key(book_gap<G>(x, cur64)), i});
  }
  return block_farthest(win, scratch);
}

// Entry sums per component in any order, when that order cannot matter: the
// values are float32, all multiples of 2^L (L the lowest set bit among an
// entry's members in that component), so every partial sum of any subset is
// a multiple of 2^L no larger than the sum of magnitudes A; when
// 2 A < 2^(L + 53) each is a double exactly, no addition rounds, and the
// result is the sequential sum's bits (numpy's axis-0 order) in every order.
// (A is itself a rounded sum; its relative error, below 2^-40, is covered by
// taking 2 A.)
//
// The members, grouped by entry in `order`, are cut into one equal share per
// wave whatever entries they belong to, so an entry holding the whole sample
// is summed by all 16 waves. Within a share, lane j + G s takes component j
// of the members k with k mod (64 / G) = s, with four accumulators; the
// lanes of a component combine, and the wave adds its partial sum, its
// magnitude sum and its lowest bit into the (entry, component) slots with
// LDS atomics (exact sums again). A value that is not finite sets the slot's
// lowest bit to kNotFinite, which fails the test.
constexpr int kNotFinite = INT_MIN;
constexpr int kNoBit = 1 << 20;  // lowest bit of a slot no nonzero value reached

// The lowest set bit of a finite float's value, as a power of two; kNoBit for
// a zero. Branch-free: bit 23 set in the word stands for the implicit bit of a
// normal (ctz = the mantissa field's trailing zeros, 23 when it is zero) and
// caps a denormal's count; max(e, 1) - 150 is the exponent of the field's
// bit 0 for both. Equal, for every finite bit pattern, to the field-by-field
// form (exponent e - 150 or -149, plus the trailing zeros of the mantissa
// with its implicit bit).
__device__ __forceinline__ int low_bit_exponent(float v) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t e = (b >> 23) & 255u;
  const int low = int(e > 1u ? e : 1u) - 150 + int(__builtin_ctz(b | 0x800000u));
  return (b << 1) != 0u ? low : kNoBit;
}

template <int G>
__device__ __forceinline__ void exact_share(const float* xs, const uint16_t* order,
                                            uint32_t rows, const uint32_t* etotal,
                                            double* epart, double* emag, int* elow) {
  constexpr uint32_t S = 64 / G;  // member subsets per component
  constexpr uint32_t kWaves = kUpdateThreads / 64;
  const uint32_t lane = threadIdx.x % 64, j = lane % G, sub = lane / G;
  const uint32_t wave = threadIdx.x / 64;
  const uint32_t share = (rows + kWaves - 1) / kWaves;
  const uint32_t lo = min(rows, wave * share), hi = min(rows, lo + share);
  const int totals = lane < 16 ? int(etotal[lane]) : 0;  // one LDS read; lane e holds entry e's
  uint32_t start = 0;
  for (uint32_t e = 0; e < 16; ++e) {
    const uint32_t end = start + uint32_t(__builtin_amdgcn_readlane(totals, int(e)));
    const uint32_t first = max(start, lo), last = min(end, hi);
    start = end;
    if (first >= last) continue;
    double acc[4] = {0.0, 0.0, 0.0, 0.0}, mag = 0.0;
    int low = kNoBit;
    uint32_t top = 0;  // largest magnitude's bits shifted left: 0xff000000 and up is not finite
    uint32_t k = first + sub;
    for (; k + 3 * S < last; k += 4 * S) {  // every load of a step, then the arithmetic
      uint32_t ix[4];
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) ix[u] = order[k + u * S];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = xs[ix[u] * G + j];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        acc[u] += double(v[u]);
        mag += fabs(double(v[u]));
        low = min(low, low_bit_exponent(v[u]));
        top = max(top, __float_as_uint(v[u]) << 1);
      }
    }
    for (; k < last; k += S) {
      const float v = xs[uint32_t(order[k]) * G + j];
      acc[0] += double(v);
      mag += fabs(double(v));
      low = min(low, low_bit_exponent(v));
      top = max(top, __float_as_uint(v) << 1);
    }
    double part = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    low = top < 0xff000000u ? low : kNotFinite;
#pragma unroll
    for (uint32_t off = G; off < 64; off <<= 1) {
      part += __shfl_xor(part, int(off));
      mag += __shfl_xor(mag, int(off));
      low = min(low, __shfl_xor(low, int(off)));
    }
    if (lane < G) {
      atomicAdd(&epart[e * G + j], part);
      atomicAdd(&emag[e * G + j], mag);
      atomicMin(&elow[e * G + j], low);
    }
  }
}

// The test of exact_share's slots for one (entry, component): every value
// finite and 2 A < 2^(L + 53); A = 0 (every member zero) always passes.
__device__ __forceinline__ bool exact_slot(double mag, int low) {
  return low != kNotFinite && (mag == 0.0 || ilogb(mag) + 2 <= low + 53);
}

// Means and reseeds of one iteration (vq.py:223-229). One block per problem.
template <int G>
__global__ __launch_bounds__(kUpdateThreads) void k_fit_update(FitArgs a) {
  constexpr uint32_t kRows = kStageBytes / (4 * G);  // rows per staged round
  constexpr uint32_t kBlocks = kRows / 64;            // 64-row blocks per staged round
  static_assert(kRows % 64 == 0 && kBlocks <= 64, "one lane per block in the offset scan");
  __shared__ float4 xs4[kStageBytes / 16];
  __shared__ uint8_t ids[kRows];
  __shared__ uint16_t order[kRows];                   // the round's rows, grouped by entry
  __shared__ uint16_t bcount[kBlocks * 16];           // members of entry e in block b
  __shared__ uint16_t bstart[kBlocks * 16];           // where they go in `order`
  __shared__ uint32_t etotal[16];
  __shared__ __align__(16) float cur[16 * G];
  __shared__ double cur64[16 * G];                    // cur as float64, for the reseed gaps
  __shared__ uint32_t twins;                          // entries with a bitwise copy above them
  __shared__ uint32_t nlist;                          // lone_reseed's list length
  __shared__ double sgap[257];                        // lone_reseed's 16 rows x 16 entries, T
  __shared__ uint32_t wrow[16];
  __shared__ float mean[16 * G];
  __shared__ uint32_t members[16];
  __shared__ FarKey scratch[2 * (kUpdateThreads / 64)];  // block_farthest's two halves
  __shared__ double epart[16 * G];                    // exact_share's slots
  __shared__ double emag[16 * G];
  __shared__ int elow[16 * G];

  const uint32_t p = blockIdx.x;
  const uint32_t t = threadIdx.x;
  const uint32_t wave = t / warpSize;  // the entry this wave sums
  const uint32_t lane = t % warpSize;
  const uint32_t count = a.count;
  const float* sample = sample_of<G>(a, p);
  const uint8_t* idx = a.idx + uint64_t(p) * count;
  float* book = a.book + p * 16 * G;
  uint32_t* flags = a.flags + p * 4;
  const uint32_t kept = flags[1];  // the keep pass's entries (read early: used at the end)
  if (t == 0) twins = 0;
  for (uint32_t i = t; i < 16 * G; i += kUpdateThreads) {
    cur[i] = book[i];
    cur64[i] = double(book[i]);
    epart[i] = 0.0;
    emag[i] = 0.0;
    elow[i] = kNoBit;
  }

  // Per-entry sums in sample order. Adding +0.0 for a skipped slot is exact:
  // a sum that starts at +0 is never -0, and NaN and infinities pass through.
  double sum = 0.0;
  uint32_t n = 0;
  const float* xs = reinterpret_cast<const float*>(xs4);
  for (uint32_t c0 = 0; c0 < count; c0 += kRows) {
    const uint32_t rows = count - c0 < kRows ? count - c0 : kRows;
    __syncthreads();
    const float4* src = reinterpret_cast<const float4*>(sample + uint64_t(c0) * G);
    {
      // every load of the round first, then the LDS writes: one round trip
      // to memory instead of one per loop step
      constexpr uint32_t kQ = kStageBytes / 16 / kUpdateThreads, kI = kRows / kUpdateThreads;
      static_assert(kQ * kUpdateThreads * 16 == kStageBytes && kI * kUpdateThreads == kRows,
                    "whole staging steps per thread");
      const uint32_t nq = rows * G / 4;
      float4 v[kQ];
      uint32_t iv[kI];
#pragma unroll
      for (uint32_t i = 0; i < kQ; ++i) {
        const uint32_t q = t + i * kUpdateThreads;
        v[i] = q < nq ? src[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
#pragma unroll
      for (uint32_t i = 0; i < kI; ++i) {
        const uint32_t q = t + i * kUpdateThreads;
        iv[i] = q < rows ? idx[c0 + q] : 0u;
      }
#pragma unroll
      for (uint32_t i = 0; i < kQ; ++i)
        if (t + i * kUpdateThreads < nq) xs4[t + i * kUpdateThreads] = v[i];
#pragma unroll
      for (uint32_t i = 0; i < kI; ++i)
        if (t + i * kUpdateThreads < rows) ids[t + i * kUpdateThreads] = uint8_t(iv[i]);
    }
    __syncthreads();
    // A stable counting sort of the round's rows by entry, then wave e adds
    // its members' values in sample order, 16 per round trip.
    const uint32_t nblk = (rows + 63) / 64;
    for (uint32_t b = wave; b < nblk; b += 16) {  // counts: one wave per block
      const uint32_t r = b * 64 + lane;
      const uint32_t id = r < rows ? ids[r] : 16u;
      uint32_t mine = 0;
#pragma unroll
      for (uint32_t e = 0; e < 16; ++e) {
        const uint32_t c = __popcll(__ballot(id == e));
        mine = lane == e ? c : mine;
      }
      if (lane < 16) bcount[b * 16 + lane] = uint16_t(mine);
    }
    __syncthreads();
    uint32_t before = 0;  // wave e: members of entry e in the blocks before lane's
    {
      const uint32_t c = lane < nblk ? bcount[lane * 16 + wave] : 0u;
      uint32_t incl = c;
#pragma unroll
      for (uint32_t off = 1; off < 64; off <<= 1) {
        const uint32_t o = uint32_t(__shfl_up(int(incl), off));
        incl += lane >= off ? o : 0u;
      }
      before = incl - c;
      if (lane == 63) etotal[wave] = incl;
    }
    __syncthreads();
    uint32_t estart = 0;
    for (uint32_t e = 0; e < wave; ++e) estart += etotal[e];
    const uint32_t ecount = etotal[wave];
    if (lane < nblk) bstart[lane * 16 + wave] = uint16_t(estart + before);
    __syncthreads();
    for (uint32_t b = wave; b < nblk; b += 16) {  // scatter, in row order within an entry
      const uint32_t r = b * 64 + lane;
      const uint32_t id = r < rows ? ids[r] : 16u;
      uint32_t pos = 0;
#pragma unroll
      for (uint32_t e = 0; e < 16; ++e) {
        const uint64_t bal = __ballot(id == e);
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi(uint32_t(bal >> 32),
                                                        __builtin_amdgcn_mbcnt_lo(uint32_t(bal), 0u));
        pos = id == e ? rank : pos;
      }
      if (id < 16) order[bstart[b * 16 + id] + pos] = uint16_t(r);
    }
    __syncthreads();
    n += ecount;
    const uint32_t j = lane < G ? lane : 0;
    // One staging round: every entry's sum in any order first (exact_share,
    // spread over all waves); an entry keeps it when no partial sum can
    // round, else its wave takes the sequential loop below.
    if (count <= kRows) {
      exact_share<G>(xs, order, rows, etotal, epart, emag, elow);
      __syncthreads();
      const bool ok = lane >= G || exact_slot(emag[wave * G + j], elow[wave * G + j]);
      if (!__any(!ok)) {
        sum = epart[wave * G + j];
        continue;
      }
    }
    // whole batches of 16: the next batch's rows are read before this batch's
    // additions, which then run unconditionally
    const uint32_t whole = ecount / 16 * 16;
    uint32_t rowv[16];
    if (whole > 0) {
#pragma unroll
      for (uint32_t q = 0; q < 16; ++q) rowv[q] = order[estart + q];
    }
    for (uint32_t k0 = 0; k0 < whole; k0 += 16) {
      float xv[16];
#pragma unroll
      for (uint32_t q = 0; q < 16; ++q) xv[q] = xs[rowv[q] * G + j];
      if (k0 + 16 < whole) {
#pragma unroll
        for (uint32_t q = 0; q < 16; ++q) rowv[q] = order[estart + k0 + 16 + q];
      }
#pragma unroll
      for (uint32_t q = 0; q < 16; ++q) sum = sum + double(xv[q]);
    }
    for (uint32_t k = whole; k < ecount; ++k) sum = sum + double(xs[uint32_t(order[estart + k]) * G + j]);
  }
  if (lane < G && n > 0) mean[wave * G + lane] = float(sum / double(n));
  if (lane == 0) members[wave] = n;
  __syncthreads();

  // Entries in ascending order; a reseed sees the book as updated so far.
  const uint32_t filled = uint32_t(__ballot(lane < 16 && members[lane % 16] > 0));
  const uint32_t reseeds = ~filled & ~kept & 0xffffu;  // the entries this iteration reseeds
  const bool regs = G == 8 && count <= kRegRows * kUpdateThreads;
  uint32_t twin = 0, heads = 0, store = 0;
  double* near = a.gaps + uint64_t(p) * count * 17;
  double* suffix = near + count;
  double near_r[G == 8 ? kRegRows : 1];
  double hi_r[G == 8 ? kRegRows : 1];
  bool first = true;
  uint32_t done = 0, head = 0, row = 0, parity = 0;
  for (uint32_t e = 0; e < 16; ++e) {
    if ((filled >> e) & 1u) {
      if (t < G) {
        cur[e * G + t] = mean[e * G + t];
        cur64[e * G + t] = double(mean[e * G + t]);
      }
      continue;
    }
    if ((kept >> e) & 1u) continue;
    if (first && t < 256) {  // twins among the untouched entries: a bitwise equal to some b > a
      const uint32_t ea = t / 16, eb = t % 16;
      if (ea >= e && eb > ea) {
        const uint4* ra = reinterpret_cast<const uint4*>(cur + ea * G);
        const uint4* rb = reinterpret_cast<const uint4*>(cur + eb * G);
        uint32_t diff = 0;
#pragma unroll 2
        for (int q = 0; q < G / 4; ++q) {
          const uint4 u = ra[q], v = rb[q];
          diff |= (u.x ^ v.x) | (u.y ^ v.y) | (u.z ^ v.z) | (u.w ^ v.w);
        }
        if (diff == 0) atomicOr(&twins, 1u << ea);
      }
    }
    // cur64 as this reseed reads it: the means placed since the previous
    // reseed (whose own row comes from the sample) and, for the first, the twins
    if (first || (filled & ((1u << e) - (2u << done))) != 0u) __syncthreads();
    if (first) {
      twin = twins;
      // heads: the later reseeds whose hi differs from the previous reseed's
      // (an untouched entry that is no twin lies between them)
      for (uint32_t r = e + 1, prev = e; r < 16; ++r) {
        if (!((reseeds >> r) & 1u)) continue;
        if (~twin & ((1u << r) - (1u << prev))) heads |= 1u << r;
        prev = r;
      }
      // reseed_row reads a later non-head reseed's hi from this entry's
      store = heads | (!regs && (reseeds & ~heads & ~(1u << e)) ? 1u << e : 0u);
    }
    // no later reseed this iteration (group 32 keeps the general path: its
    // float64 rows leave no registers for the whole-book pass)
    const bool single = G <= 16 && first && (reseeds >> (e + 1)) == 0u;
    const bool reload = !first && ((heads >> e) & 1u);
    head = first || reload ? e : head;
    // the staged rows when they are the whole sample (one staging round)
    const float* rows_src = count <= kRows ? xs : sample;
    const float* done_row = rows_src + uint64_t(row) * G;  // the previous reseed's row
    FarKey* half = scratch + (kUpdateThreads / 64) * parity;
    parity ^= 1u;
    if (single && count <= kRows) {  // order and ids are free after the sums
      row = lone_reseed<G>(xs, ids, count, cur64, order, &nlist, sgap, wrow, scratch);
    } else if constexpr (G == 8) {  // wider rows do not fit four per thread in registers
      row = regs ? reseed_row_regs<G>(rows_src, count, cur64, e, done, done_row, first, single,
                                      reload, twin, store, near_r, hi_r, suffix, half)
                 : reseed_row<G>(rows_src, count, cur64, e, done, done_row, first, single, twin,
                                 store, head, near, suffix, half);
    } else {
      row = reseed_row<G>(rows_src, count, cur64, e, done, done_row, first, single, twin, store,
                          head, near, suffix, half);
    }
    if (t < G) {
      const float v = rows_src[uint64_t(row) * G + t];
      cur[e * G + t] = v;
      cur64[e * G + t] = double(v);
    }
    first = false;
    done = e;
  }
  __syncthreads();
  for (uint32_t i = t; i < 16 * G; i += kUpdateThreads) book[i] = cur[i];
  if (t < 4) flags[t] = 0;
}

uint32_t blocks_for(uint64_t items, uint32_t per_block, uint32_t cap) {
  uint64_t b = (items + per_block - 1) / per_block;
  if (b == 0) b = 1;
  return b > cap ? cap : uint32_t(b);
}

template <int G>
hipError_t fit_group(hipStream_t s, const FitArgs& a, uint32_t problems, uint32_t iterations,
                     const float* init, const FitWhole& whole, bool book_ready) {
  if (!book_ready) k_fit_init<G><<<problems, 256, 0, s>>>(a, init);
  // The keep pass can only be due for a warm start on a sample smaller than
  // the tensor (vq.py:219).
  const bool keep = init != nullptr && a.count < a.complete;
  const dim3 assign_grid(blocks_for(a.count, kAssignThreads, 4096), problems);
  for (uint32_t it = 0; it < iterations; ++it) {
    k_fit_assign<G><<<assign_grid, kAssignThreads, 0, s>>>(a);
    if (keep) {
      if (whole.adamw != nullptr) {
        hipError_t e = launch_adamw_keep(s, *whole.adamw, a);
        if (e != hipSuccess) return e;
      } else {
        k_fit_keep_dense<G><<<blocks_for(a.complete, 256, 16384), 256, 0, s>>>(a, whole.values);
      }
    }
    k_fit_update<G><<<problems, kUpdateThreads, 0, s>>>(a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fit_sample_dense(hipStream_t s, const float* values, uint32_t group,
                                   const FitArgs& a, const float* init) {
  const dim3 grid(blocks_for(uint64_t(a.count) * group, 256, 4096));
  if (group == 8) k_fit_sample_dense<8><<<grid, 256, 0, s>>>(values, a, init);
  else if (group == 16) k_fit_sample_dense<16><<<grid, 256, 0, s>>>(values, a, init);
  else k_fit_sample_dense<32><<<grid, 256, 0, s>>>(values, a, init);
  return hipGetLastError();
}

hipError_t launch_fit(hipStream_t s, const FitArgs& a, uint32_t group, uint32_t problems,
                      uint32_t iterations, const float* init, const FitWhole& whole,
                      bool book_ready) {
  if (group == 8) return fit_group<8>(s, a, problems, iterations, init, whole, book_ready);
  if (group == 16) return fit_group<16>(s, a, problems, iterations, init, whole, book_ready);
  return fit_group<32>(s, a, problems, iterations, init, whole, book_ready);
}

}  // namespace ackvq
