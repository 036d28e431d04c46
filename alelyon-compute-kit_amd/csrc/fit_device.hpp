// Device helpers of the codebook calibration (fit_codebook,
// src/alelyon_compute_kit/_kit/python/vq.py:182-257), shared by the fit
// kernels and the AdamW keep pass. Every float64 step is ordered as numpy
// orders the reference's expressions, and the library is compiled with
// -ffp-contract=off, so results are bit-identical to the host restatement
// (host_fit.cpp) and to the reference's Python.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace ackvq {
namespace fitdev {

// Row i of floor(numpy.linspace(0, n - 1, num)) (vq.py:206-207): i * ((n -
// 1) / (num - 1)) in float64, the last element exactly n - 1.
__device__ __forceinline__ uint32_t linspace_at(uint64_t n, uint32_t num, uint32_t i) {
  if (num <= 1) return 0;
  const double delta = double(n - 1);
  const double div = double(num - 1);
  const double step = delta / div;
  double y = step == 0.0 ? (double(i) / div) * delta : double(i) * step;
  y = y + 0.0;
  if (i == num - 1) y = delta;
  return uint32_t(floor(y));
}

// The float64 CPU encode's argmin for one complete vector (vq.py:166-174):
// d = d + (x_j - c_j)^2 over j ascending, every operation rounded; the first
// minimum wins, and a NaN distance wins at once (np.argmin). `book` holds the
// 16 x G entries as float64.
template <int G>
__device__ __forceinline__ uint32_t nearest64(const double (&x)[G], const double* book) {
  double best = 0.0;
  uint32_t sel = 0;
#pragma unroll 1
  for (uint32_t e = 0; e < 16; ++e) {
    double d = 0.0;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const double delta = x[j] - book[e * G + j];
      const double sq = delta * delta;
      d = d + sq;
    }
    const bool nan = d != d;
    if (e == 0 || nan || d < best) {
      best = d;
      sel = e;
      if (nan) break;
    }
  }
  return sel;
}

// One entry's float64 distance, in nearest64's order of operations.
template <int G>
__device__ __forceinline__ double dist64(const double (&x)[G], const double* c) {
  double d = 0.0;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const double delta = x[j] - c[j];
    const double sq = delta * delta;
    d = d + sq;
  }
  return d;
}

// nearest64 with the book in global memory, read at wave-uniform addresses
// (scalar loads, no LDS traffic), and a loop over the entries that no lane
// leaves early: the first NaN distance still wins, through a flag.
template <int G>
__device__ __forceinline__ uint32_t nearest64_uniform(const double (&x)[G],
                                                      const double* __restrict__ book) {
  double best = 0.0;
  uint32_t sel = 0;
  bool done = false;
#pragma unroll 2
  for (uint32_t e = 0; e < 16; ++e) {
    const double d = dist64<G>(x, book + e * G);
    const bool nan = d != d;
    if (!done && (e == 0 || nan || d < best)) {
      best = d;
      sel = e;
    }
    done = done || nan;
  }
  return sel;
}

// vq.py:216-222's condition for the keep pass, for `problems` (at most 4)
// fits at once: the entries each problem's sample left unused (bit clear in
// flags[4 p], the assign pass's mask) that are not copies of an earlier entry
// of its book (float compare: -0 equals 0, NaN equals nothing). Called by
// every thread of the block; scand[p] receives problem p's entries. `sbook`
// is block scratch of problems x 16 x G floats.
template <int G>
__device__ __forceinline__ void keep_candidates(const float* book, const uint32_t* flags,
                                                uint32_t problems, float* sbook,
                                                uint32_t* scand) {
  for (uint32_t i = threadIdx.x; i < problems * 16 * G; i += blockDim.x) sbook[i] = book[i];
  __syncthreads();
  if (threadIdx.x < 64) {
    const uint32_t p = threadIdx.x / 16, e = threadIdx.x % 16;
    bool candidate = false;
    if (p < problems && !((flags[4 * p] >> e) & 1u)) {
      const float* row = sbook + (p * 16 + e) * G;
      bool duplicate = false;
      for (uint32_t j = 0; j < e && !duplicate; ++j) {
        const float* other = sbook + (p * 16 + j) * G;
        bool equal = true;
        for (int q = 0; q < G; ++q) equal &= row[q] == other[q];
        duplicate = equal;
      }
      candidate = !duplicate;
    }
    const uint64_t bits = __ballot(candidate);
    if (threadIdx.x < problems) scand[threadIdx.x] = uint32_t(bits >> (16 * threadIdx.x)) & 0xffffu;
  }
  __syncthreads();
}

}  // namespace fitdev
}  // namespace ackvq
