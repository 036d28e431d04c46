// Single small m = 1 products on gfx950: "gemv-direct".
//
// For y = x . B with B stored (k, n) and its groups along n (op 2, flags 0 of
// src/alelyon_compute_kit/_kit/kernels/vq4.comp:165-176) and one row of A, each
// output is y[c] = sum_kk x[kk] * C_B[code(kk, c / G)][c % G]. The pair-bin
// GEMV (k_gemv_pairs) is built for throughput: every block zeroes and reduces
// 128 KiB of LDS bins whatever its share of k, and its split partials need a
// second launch. For one resident weight of a few MiB those fixed costs are
// the whole latency, so this kernel decodes instead: a lane owns one output
// column, looks up C_B[e][c % G] in LDS for each row's code e and accumulates
// x[kk] times it in FP32 (fused multiply-add) into four accumulators by row
// mod 4, k ascending within a slice.
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
// agree within FP32 rounding (slices of at most kDirectMaxSlice rows).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "kernels.hpp"

namespace ackvq {
namespace {

constexpr uint32_t kDirectCols = 256;       // output columns per block: 4 waves x 64 lanes
constexpr uint32_t kDirectMaxSlice = 1024;  // rows of B per block (LDS staging)
constexpr uint32_t kDirectMinSlice = 64;    // no slice shorter than this
constexpr uint32_t kDirectBlocks = 256;     // blocks a launch aims for
constexpr uint32_t kDirectQuarters = 4;       // row quarters of a slice: 1024 threads

__device__ __forceinline__ bool finite_f32(float x) { return fabsf(x) <= FLT_MAX; }

__device__ __forceinline__ uint32_t nibble(const uint32_t* codes, uint32_t vector) {
  return (codes[vector >> 3] >> ((vector & 7u) * 4u)) & 15u;
}

template <typename T>
__device__ __forceinline__ const T* item_ptr(const void* base, uint64_t stride, uint32_t item) {
  return reinterpret_cast<const T*>(static_cast<const char*>(base) + stride * item);
}

// AD: x is a dense FP32 row in in[0] (the dense-activation product); a
// nonfinite x sets status bit 1.
template <int G, bool AD>
__global__ __launch_bounds__(1024) void k_gemv_direct(Operands o, uint32_t n, uint32_t k,
                                                     uint32_t slice, float* partial) {
  constexpr uint32_t kTileWords = kDirectCols / (8 * G);  // words of one B row in a tile
  __shared__ __align__(16) float s_book[16 * G];
  __shared__ __align__(16) float s_abook[16 * G];
  __shared__ __align__(16) float s_x[kDirectMaxSlice];
  __shared__ __align__(16) uint32_t s_w[kTileWords][kDirectMaxSlice];
  __shared__ uint32_t s_last;
  __shared__ float s_red[kDirectQuarters][kDirectCols];
  const uint32_t tile = blockIdx.x, split = blockIdx.y, item = blockIdx.z;
  const uint32_t tiles = gridDim.x, splits = gridDim.y;
  const uint32_t tid = threadIdx.x;
  const uint32_t k0 = split * slice;
  const uint32_t kn = (k - k0) < slice ? (k - k0) : slice;
  const uint32_t row_words = n / (8 * G);
  const uint32_t q0 = tile * kTileWords;
  const float* b_book = item_ptr<float>(o.in[3], o.stride[3], item);
  const float* a_book = item_ptr<float>(o.in[1], o.stride[1], item);
  const uint32_t* b_codes = item_ptr<uint32_t>(o.in[2], o.stride[2], item);

  // One round of independent loads: both books, this slice's B words and x
  // (dense) or A's code words (packed; decoded from the book in LDS next).
  bool bad = false;
  for (uint32_t i = tid; i < 16 * G; i += blockDim.x) {
    const float bv = b_book[i];
    s_book[i] = bv;
    if (!AD) s_abook[i] = a_book[i];
    if (tile == 0 && split == 0) bad |= (!AD && !finite_f32(a_book[i])) || !finite_f32(bv);
  }
  for (uint32_t i = tid; i < kn * kTileWords; i += blockDim.x) {
    const uint32_t r = i / kTileWords, wq = i % kTileWords;
    s_w[wq][r] = (q0 + wq < row_words) ? b_codes[uint64_t(k0 + r) * row_words + q0 + wq] : 0u;
  }
  if (AD) {
    const float* xd = item_ptr<float>(o.in[0], o.stride[0], item);
    for (uint32_t i = tid; i < kn; i += blockDim.x) {
      const float v = xd[k0 + i];
      s_x[i] = v;
      bad |= tile == 0 && !finite_f32(v);
    }
  }
  if (__any(bad) && (tid % warpSize) == 0) atomicOr(o.status, 1u);
  if (!AD) {
    // one thread per A group of the slice: its code from one word, its G
    // values from the book
    const uint32_t* a_codes = item_ptr<uint32_t>(o.in[0], o.stride[0], item);
    const uint32_t u0 = k0 / G, un = (k0 + kn - 1) / G - u0 + 1;
    const uint32_t code = tid < un ? nibble(a_codes, u0 + tid) : 0u;  // un <= 129
    __syncthreads();  // the A book
    if (tid < un) {
      for (uint32_t s = 0; s < uint32_t(G); ++s) {
        const uint32_t kk = (u0 + tid) * G + s;
        if (kk >= k0 && kk < k0 + kn) s_x[kk - k0] = s_abook[code * G + s];
      }
    }
  }
  __syncthreads();

  // the lane's output column within the tile: group jl, offset t; its word
  // (wq) is the same for the whole wave. Four accumulators, by row mod 4.
  const uint32_t cl = tid % kDirectCols, quarter = tid / kDirectCols;
  const uint32_t jl = cl / G, t = cl % G;
  const uint32_t wq = jl / 8, shift = 4 * (jl % 8);
  const uint32_t* wrow = s_w[wq];
  // this thread's quarter of the slice: rows [r0, r1), r0 a multiple of 16
  const uint32_t qrows = (kn + 16 * kDirectQuarters - 1) / (16 * kDirectQuarters) * 16;
  const uint32_t r0 = quarter * qrows < kn ? quarter * qrows : kn;
  const uint32_t r1 = r0 + qrows < kn ? r0 + qrows : kn;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  uint32_t r = r0;
  for (; r + 16 <= r1; r += 16) {
    uint32_t w[16];
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {  // all lanes read one address: broadcasts
      const uint4 w4 = *reinterpret_cast<const uint4*>(wrow + r + i);
      const float4 x4 = *reinterpret_cast<const float4*>(s_x + r + i);
      w[i] = w4.x; w[i + 1] = w4.y; w[i + 2] = w4.z; w[i + 3] = w4.w;
      x[i] = x4.x; x[i + 1] = x4.y; x[i + 2] = x4.z; x[i + 3] = x4.w;
    }
    float b[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) b[i] = s_book[((w[i] >> shift) & 15u) * G + t];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i % 4] = fmaf(x[i], b[i], acc[i % 4]);
  }
  for (; r < r1; ++r)
    acc[r % 4] = fmaf(s_x[r], s_book[((wrow[r] >> shift) & 15u) * G + t], acc[r % 4]);
  s_red[quarter][cl] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  __syncthreads();

  const uint32_t c = tile * kDirectCols + cl;
  const uint32_t slot = item * tiles + tile;
  float* part = partial + uint64_t(slot) * splits * kDirectCols;
  // Publish the partial, then count the arrival; the last block of the tile
  // adds the partials in slice order. The partials are device-coherent atomic
  // stores and loads (they bypass the per-XCD L2s), and every store has
  // completed (vmcnt 0) before the block's arrival is counted, so the last
  // block reads them all without a device-wide fence (which writes back and
  // invalidates the whole L2: measured at 30 us on this kernel).
  if (quarter == 0) {  // the quarters in order
    float mine = s_red[0][cl];
#pragma unroll
    for (uint32_t qq = 1; qq < kDirectQuarters; ++qq) mine += s_red[qq][cl];
    __hip_atomic_store(&part[split * kDirectCols + cl], mine, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(&o.arrivals[slot], 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == splits - 1 ? 1u : 0u;
  __syncthreads();
  if (s_last == 0 || quarter != 0) return;
  float y = 0.0f;
  uint32_t sp = 0;
  for (; sp + 4 <= splits; sp += 4) {  // four loads in flight, added in slice order
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      v[i] = __hip_atomic_load(&part[(sp + i) * kDirectCols + cl], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    y += v[0]; y += v[1]; y += v[2]; y += v[3];
  }
  for (; sp < splits; ++sp)
    y += __hip_atomic_load(&part[sp * kDirectCols + cl], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  bool out_bad = false;
  if (c < n) {
    float* out = reinterpret_cast<float*>(static_cast<char*>(o.out) + o.stride[4] * item);
    out[c] = y;
    out_bad = !finite_f32(y);
  }
  if (__any(out_bad) && (tid % warpSize) == 0) atomicOr(o.status, 1u);
  if (tid == 0)
    __hip_atomic_store(&o.arrivals[slot], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

void direct_shape(uint32_t n, uint32_t k, uint32_t group, uint32_t count, uint32_t* tiles,
                  uint32_t* splits, uint32_t* slice) {
  *tiles = (n + kDirectCols - 1) / kDirectCols;
  const uint64_t blocks = uint64_t(*tiles) * count;
  uint32_t s = blocks >= kDirectBlocks ? 1u : uint32_t((kDirectBlocks + blocks - 1) / blocks);
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

template <int G, bool AD>
hipError_t launch_g(hipStream_t s, const Operands& o, uint32_t n, uint32_t k, void* workspace) {
  uint32_t tiles, splits, slice;
  direct_shape(n, k, G, o.count, &tiles, &splits, &slice);
  dim3 grid(tiles, splits, o.count);
  k_gemv_direct<G, AD><<<grid, kDirectCols * kDirectQuarters, 0, s>>>(o, n, k, slice,
                                                    static_cast<float*>(workspace));
  return hipGetLastError();
}

}  // namespace

bool direct_applies(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                    uint32_t count) {
  if (m != 1 || (flags & 2u) != 0 || n % (8 * group) != 0 || k == 0 || count == 0) return false;
  if (count > 65535) return false;
  const uint64_t tiles = (n + kDirectCols - 1) / kDirectCols;
  if (tiles * count > kDirectCounters) return false;
  return uint64_t(n) * k * count <= kDirectMaxWeights;
}

size_t direct_workspace_bytes(uint32_t n, uint32_t k, uint32_t group, uint32_t count) {
  uint32_t tiles, splits, slice;
  direct_shape(n, k, group, count, &tiles, &splits, &slice);
  return size_t(count) * tiles * splits * kDirectCols * sizeof(float);
}

hipError_t launch_direct(hipStream_t s, const Operands& o, uint32_t n, uint32_t k, uint32_t group,
                         bool dense, void* workspace) {
  if (group == 8) return dense ? launch_g<8, true>(s, o, n, k, workspace)
                               : launch_g<8, false>(s, o, n, k, workspace);
  if (group == 16) return dense ? launch_g<16, true>(s, o, n, k, workspace)
                                : launch_g<16, false>(s, o, n, k, workspace);
  return dense ? launch_g<32, true>(s, o, n, k, workspace)
               : launch_g<32, false>(s, o, n, k, workspace);
}

}  // namespace ackvq
