// Small products of up to 8 rows of A on gfx950: "gemv-direct".
//
// For y = A . B with B stored (k, n) and its groups along n (op 2, flags 0 or
// 1 of src/alelyon_compute_kit/_kit/kernels/vq4.comp:165-176) and m <= 8 rows
// of A, each output is y[r][c] = sum_kk A[r][kk] * C_B[code(kk, c / G)][c % G].
// The bin GEMVs (k_gemv_pairs, k_gemv_rows) are built for throughput: every
// block zeroes and reduces 128 KiB of LDS bins whatever its share of k, and
// their split partials need a second launch. For one resident weight of a few
// MiB those fixed costs are the whole latency, so this kernel decodes instead:
// a lane owns one output column, looks up C_B[e][c % G] in LDS for each row's
// code e once, and accumulates every row of A times it in FP32 (fused
// multiply-add) into four accumulators per row by inner index mod 4, k
// ascending within a quarter of a slice. A's rows (decoded through A's book
// when packed, read as they are when dense) are staged in LDS per slice.
//
// Grid: (tiles of 256 output columns, slices of k, instances). The slices'
// partial sums are added by the block that finishes its tile last, in slice
// order, so results do not depend on timing: one launch, no memset. The
// arrival counters (Operands::arrivals) belong to the device handle, which
// zeroes them once when it opens; the last block of a tile sets its counter
// back to zero. A handle's launches are serialised on its stream, so no two
// launches use the same counters at once.
//
// The summation order differs from the shader's sequential one; results
// agree within FP32 rounding (slices of at most kDirectMaxSlice rows, each in
// four quarters summed in order).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "kernels.hpp"

namespace ackvq {
namespace {

constexpr uint32_t kDirectCols = 256;       // output columns per block: 4 waves x 64 lanes
constexpr uint32_t kDirectMaxSlice = 1024;  // rows of B per block (LDS staging)
constexpr uint32_t kDirectMinSlice = 64;    // no slice shorter than this
constexpr uint32_t kDirectBlocks = 256;     // most blocks a launch takes (unless tiles exceed it)
constexpr uint32_t kDirectQuarters = 4;       // row quarters of a slice: 1024 threads

__device__ __forceinline__ bool finite_f32(float x) { return fabsf(x) <= FLT_MAX; }

__device__ __forceinline__ uint32_t nibble(const uint32_t* codes, uint32_t vector) {
  return (codes[vector >> 3] >> ((vector & 7u) * 4u)) & 15u;
}

template <typename T>
__device__ __forceinline__ const T* item_ptr(const void* base, uint64_t stride, uint32_t item) {
  return reinterpret_cast<const T*>(static_cast<const char*>(base) + stride * item);
}

// M: rows of A the kernel holds (1, 2, 4 or 8); the product's m <= M rows are
// read through A's flat index (row-major, or transposed when flags bit 0 is
// set), rows m..M-1 are zero and never stored. AD: A is dense FP32 in in[0]
// (the dense-activation product); a nonfinite x sets status bit 1.
template <int G, bool AD, int M>
__global__ __launch_bounds__(1024) void k_gemv_direct(Operands o, uint32_t m, uint32_t n,
                                                     uint32_t k, uint32_t flags, uint32_t slice,
                                                     float* partial) {
  constexpr uint32_t kTileWords = kDirectCols / (8 * G);  // words of one B row in a tile
  constexpr uint32_t kThreads = kDirectCols * kDirectQuarters;
  constexpr uint32_t kPer = (M * kDirectMaxSlice + kThreads - 1) / kThreads;  // x per thread
  static_assert(kDirectQuarters * kDirectCols <= kDirectMaxSlice, "quarter sums fit in s_x");
  __shared__ __align__(16) float s_book[16 * G];
  __shared__ __align__(16) float s_abook[16 * G];
  __shared__ __align__(16) float s_x[M][kDirectMaxSlice];  // then the quarter sums
  __shared__ __align__(16) uint32_t s_w[kTileWords][kDirectMaxSlice];
  __shared__ uint32_t s_last;
  const uint32_t tile = blockIdx.x, split = blockIdx.y, item = blockIdx.z;
  const uint32_t tiles = gridDim.x, splits = gridDim.y;
  const uint32_t tid = threadIdx.x;
  const uint32_t k0 = split * slice;
  const uint32_t kn = (k - k0) < slice ? (k - k0) : slice;
  const uint32_t row_words = n / (8 * G);
  const uint32_t q0 = tile * kTileWords;
  const bool ta = (flags & 1u) != 0;
  const float* b_book = item_ptr<float>(o.in[3], o.stride[3], item);
  const float* a_book = item_ptr<float>(o.in[1], o.stride[1], item);
  const uint32_t* b_codes = item_ptr<uint32_t>(o.in[2], o.stride[2], item);

  // One round of independent loads: both books, this slice's B words, and x
  // (dense) or the code of each x (packed; decoded from the book in LDS next).
  bool bad = false;
  for (uint32_t i = tid; i < 16 * G; i += kThreads) {
    const float bv = b_book[i];
    s_book[i] = bv;
    if (!AD) s_abook[i] = a_book[i];
    if (tile == 0 && split == 0) bad |= (!AD && !finite_f32(a_book[i])) || !finite_f32(bv);
  }
  for (uint32_t i = tid; i < kn * kTileWords; i += kThreads) {
    const uint32_t r = i / kTileWords, wq = i % kTileWords;
    s_w[wq][r] = (q0 + wq < row_words) ? b_codes[uint64_t(k0 + r) * row_words + q0 + wq] : 0u;
  }
  // element i of the thread: row i / kn of A, inner index k0 + i % kn
  uint32_t code[kPer];
  float xv[kPer];
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint32_t i = tid + j * kThreads;
    const uint32_t r = i / kn, kk = k0 + i % kn;
    code[j] = 0u;
    xv[j] = 0.0f;
    if (i < M * kn && r < m) {
      const uint64_t flat = ta ? uint64_t(kk) * m + r : uint64_t(r) * k + kk;
      if (AD) {
        xv[j] = item_ptr<float>(o.in[0], o.stride[0], item)[flat];
        bad |= tile == 0 && !finite_f32(xv[j]);
      } else {
        const uint32_t* a_codes = item_ptr<uint32_t>(o.in[0], o.stride[0], item);
        code[j] = nibble(a_codes, uint32_t(flat / G)) * G + uint32_t(flat % G);
      }
    }
  }
  if (__any(bad) && (tid % warpSize) == 0) atomicOr(o.status, 1u);
  if (!AD) __syncthreads();  // the A book
#pragma unroll
  for (uint32_t j = 0; j < kPer; ++j) {
    const uint32_t i = tid + j * kThreads;
    if (i < M * kn) {
      const uint32_t r = i / kn;
      s_x[i / kn][i % kn] = AD ? xv[j] : (r < m ? s_abook[code[j]] : 0.0f);
    }
  }
  __syncthreads();

  // The lane's output column within the tile: group jl, offset t; its word
  // (wq) is the same for the whole wave. Four accumulators per row, by
  // inner index mod 4; four quarters of the slice per column.
  const uint32_t cl = tid % kDirectCols, quarter = tid / kDirectCols;
  const uint32_t jl = cl / G, t = cl % G;
  const uint32_t wq = jl / 8, shift = 4 * (jl % 8);
  const uint32_t* wrow = s_w[wq];
  const uint32_t qrows = (kn + 16 * kDirectQuarters - 1) / (16 * kDirectQuarters) * 16;
  const uint32_t r0 = quarter * qrows < kn ? quarter * qrows : kn;
  const uint32_t r1 = r0 + qrows < kn ? r0 + qrows : kn;
  float acc[M][4];
#pragma unroll
  for (int r = 0; r < M; ++r) acc[r][0] = acc[r][1] = acc[r][2] = acc[r][3] = 0.0f;
  uint32_t kk = r0;
  for (; kk + 16 <= r1; kk += 16) {
    float b[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {  // all lanes read one address: broadcasts
      const uint4 w4 = *reinterpret_cast<const uint4*>(wrow + kk + i);
      b[i] = s_book[((w4.x >> shift) & 15u) * G + t];
      b[i + 1] = s_book[((w4.y >> shift) & 15u) * G + t];
      b[i + 2] = s_book[((w4.z >> shift) & 15u) * G + t];
      b[i + 3] = s_book[((w4.w >> shift) & 15u) * G + t];
    }
#pragma unroll
    for (int r = 0; r < M; ++r) {
#pragma unroll
      for (int i = 0; i < 16; i += 4) {
        const float4 x4 = *reinterpret_cast<const float4*>(&s_x[r][kk + i]);
        acc[r][0] = fmaf(x4.x, b[i], acc[r][0]);
        acc[r][1] = fmaf(x4.y, b[i + 1], acc[r][1]);
        acc[r][2] = fmaf(x4.z, b[i + 2], acc[r][2]);
        acc[r][3] = fmaf(x4.w, b[i + 3], acc[r][3]);
      }
    }
  }
  // The tail: whole steps of 4 rows, then up to 3 rows, each row kk still into
  // accumulator kk mod 4 (kk is a multiple of 4 here), every index a constant:
  // a run-time accumulator index becomes a chain of selects over all M x 4
  // accumulators per row (measured at 10 us for M = 8).
  for (; kk + 4 <= r1; kk += 4) {
    const uint4 w4 = *reinterpret_cast<const uint4*>(wrow + kk);
    const float b0 = s_book[((w4.x >> shift) & 15u) * G + t];
    const float b1 = s_book[((w4.y >> shift) & 15u) * G + t];
    const float b2 = s_book[((w4.z >> shift) & 15u) * G + t];
    const float b3 = s_book[((w4.w >> shift) & 15u) * G + t];
#pragma unroll
    for (int r = 0; r < M; ++r) {
      const float4 x4 = *reinterpret_cast<const float4*>(&s_x[r][kk]);
      acc[r][0] = fmaf(x4.x, b0, acc[r][0]);
      acc[r][1] = fmaf(x4.y, b1, acc[r][1]);
      acc[r][2] = fmaf(x4.z, b2, acc[r][2]);
      acc[r][3] = fmaf(x4.w, b3, acc[r][3]);
    }
  }
#pragma unroll
  for (uint32_t j = 0; j < 3; ++j) {
    if (kk + j < r1) {
      const float bk = s_book[((wrow[kk + j] >> shift) & 15u) * G + t];
#pragma unroll
      for (int r = 0; r < M; ++r) acc[r][j] = fmaf(s_x[r][kk + j], bk, acc[r][j]);
    }
  }
  __syncthreads();  // every wave is done with s_x: it now holds the quarter sums
  float* s_red = &s_x[0][0];  // [quarter][row][column]
#pragma unroll
  for (int r = 0; r < M; ++r)
    s_red[(quarter * M + r) * kDirectCols + cl] = (acc[r][0] + acc[r][1]) + (acc[r][2] + acc[r][3]);
  __syncthreads();

  const uint32_t c = tile * kDirectCols + cl;
  const uint32_t slot = item * tiles + tile;
  float* part = partial + uint64_t(slot) * splits * M * kDirectCols;
  // Publish the partials, then count the arrival; the last block of the tile
  // adds the partials in slice order. The partials are agent-scope atomic
  // stores and loads (device-coherent: they bypass the per-XCD L2s). The
  // block's barrier orders its threads' stores before thread 0's arrival, a
  // release at agent scope; the last block's thread 0 then takes an
  // agent-scope acquire fence, and its barrier orders the block's loads after
  // it: every block's partials happen before the last block reads them. Only
  // the last block of a tile pays the acquire (an L2 invalidation); a full
  // device fence in every block measured 30 us on this kernel.
  // thread (quarter q, column) publishes rows q, q + 4, ...: the quarters in order
  for (uint32_t r = quarter; r < uint32_t(M); r += kDirectQuarters) {
    float mine = s_red[r * kDirectCols + cl];
#pragma unroll
    for (uint32_t qq = 1; qq < kDirectQuarters; ++qq) mine += s_red[(qq * M + r) * kDirectCols + cl];
    __hip_atomic_store(&part[(split * M + r) * kDirectCols + cl], mine, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (tid == 0) {
    const bool last = __hip_atomic_fetch_add(&o.arrivals[slot], 1u, __ATOMIC_RELEASE,
                                             __HIP_MEMORY_SCOPE_AGENT) == splits - 1;
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    s_last = last ? 1u : 0u;
  }
  __syncthreads();
  if (s_last == 0) return;
  // thread (quarter q, column) sums rows q, q + 4, ... over the slices, in
  // slice order, eight loads in flight per round trip
  bool out_bad = false;
  float* out = reinterpret_cast<float*>(static_cast<char*>(o.out) + o.stride[4] * item);
  for (uint32_t r = quarter; r < m; r += kDirectQuarters) {
    float y = 0.0f;
    uint32_t sp = 0;
    for (; sp + 8 <= splits; sp += 8) {
      float v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
        v[i] = __hip_atomic_load(&part[((sp + i) * M + r) * kDirectCols + cl], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int i = 0; i < 8; ++i) y += v[i];
    }
    for (; sp < splits; ++sp)
      y += __hip_atomic_load(&part[(sp * M + r) * kDirectCols + cl], __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    if (c < n) {
      out[uint64_t(r) * n + c] = y;
      out_bad |= !finite_f32(y);
    }
  }
  if (__any(out_bad) && (tid % warpSize) == 0) atomicOr(o.status, 1u);
  if (tid == 0)
    __hip_atomic_store(&o.arrivals[slot], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

uint32_t rows_held(uint32_t m) { return m <= 1 ? 1u : m <= 2 ? 2u : m <= 4 ? 4u : 8u; }

void direct_shape(uint32_t n, uint32_t k, uint32_t group, uint32_t count, uint32_t* tiles,
                  uint32_t* splits, uint32_t* slice) {
  *tiles = (n + kDirectCols - 1) / kDirectCols;
  const uint64_t blocks = uint64_t(*tiles) * count;
  // At most kDirectBlocks blocks (one per compute unit): a launch a few blocks
  // past it leaves those compute units two blocks each, and the product waits
  // for them (m = 8, 6144 x 4096: 37.6 us with 264 blocks, 24.8 with 240).
  uint32_t s = blocks >= kDirectBlocks ? 1u : uint32_t(kDirectBlocks / blocks);
  const uint32_t most = (k + kDirectMinSlice - 1) / kDirectMinSlice;
  const uint32_t least = (k + kDirectMaxSlice - 1) / kDirectMaxSlice;
  s = s < most ? s : most;
  s = s > least ? s : least;
  s = s > 0 ? s : 1;
  uint32_t sl = (k + s - 1) / s;
  sl = (sl + 3) / 4 * 4;  // whole 16-byte LDS reads
  *slice = sl;
  *splits = (k + sl - 1) / sl;
  (void)group;
}

template <int G, bool AD, int M>
hipError_t launch_gm(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                     uint32_t flags, void* workspace) {
  uint32_t tiles, splits, slice;
  direct_shape(n, k, G, o.count, &tiles, &splits, &slice);
  dim3 grid(tiles, splits, o.count);
  k_gemv_direct<G, AD, M><<<grid, kDirectCols * kDirectQuarters, 0, s>>>(
      o, m, n, k, flags, slice, static_cast<float*>(workspace));
  return hipGetLastError();
}

template <int G, bool AD>
hipError_t launch_g(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                    uint32_t flags, void* workspace) {
  switch (rows_held(m)) {
    case 1: return launch_gm<G, AD, 1>(s, o, m, n, k, flags, workspace);
    case 2: return launch_gm<G, AD, 2>(s, o, m, n, k, flags, workspace);
    case 4: return launch_gm<G, AD, 4>(s, o, m, n, k, flags, workspace);
    default: return launch_gm<G, AD, 8>(s, o, m, n, k, flags, workspace);
  }
}

}  // namespace

bool direct_applies(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                    uint32_t count) {
  if (m == 0 || m > kDirectMaxRows || (flags & 2u) != 0 || n % (8 * group) != 0 || k == 0 ||
      count == 0)
    return false;
  if (count > 65535) return false;
  const uint64_t tiles = (n + kDirectCols - 1) / kDirectCols;
  if (tiles * count > kDirectCounters) return false;
  return uint64_t(n) * k * count <= kDirectMaxWeights;
}

size_t direct_workspace_bytes(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t count) {
  uint32_t tiles, splits, slice;
  direct_shape(n, k, group, count, &tiles, &splits, &slice);
  return size_t(count) * tiles * splits * rows_held(m) * kDirectCols * sizeof(float);
}

hipError_t launch_direct(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                         uint32_t group, uint32_t flags, bool dense, void* workspace) {
  if (group == 8) return dense ? launch_g<8, true>(s, o, m, n, k, flags, workspace)
                               : launch_g<8, false>(s, o, m, n, k, flags, workspace);
  if (group == 16) return dense ? launch_g<16, true>(s, o, m, n, k, flags, workspace)
                                : launch_g<16, false>(s, o, m, n, k, flags, workspace);
  return dense ? launch_g<32, true>(s, o, m, n, k, flags, workspace)
               : launch_g<32, false>(s, o, m, n, k, flags, workspace);
}

}  // namespace ackvq
