// vq4/v1 packed-pair products C = op(A) . op(B) for gfx950 (op 2 of
// src/alelyon_compute_kit/_kit/kernels/vq4.comp:165-176).
//
// Two implementations live here:
//
// * General: 64x64 output tiles, both operands decoded per element into LDS
//   through the flat storage index (groups may straddle rows), each output
//   accumulated as total = total + a*b with k ascending and every operation
//   rounded -- the shader's order, so its results are bit-identical to
//   vq4.comp. Serves every shape and layout.
//
// * GemvBins (small m, B stored (k,n) with each row a whole number of
//   words): per output group j and code e the kernel accumulates
//   S[r][j][e] = sum over rows k with code(k,j) = e of x[r][k] with one LDS
//   atomic add per nibble, then y[r][j*G+t] = sum_e C_B[e][t] * S[r][j][e].
//   That is G times fewer additions than decoding the weight, which is what
//   lets a product that reads only half a byte per G weights run at the
//   packed-weight bandwidth instead of the FP32 FMA rate. The summation
//   order differs from the shader's; results agree within FP32 rounding.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "kernels.hpp"

namespace ackvq {
namespace {

__device__ __forceinline__ bool finite_f32(float x) { return fabsf(x) <= FLT_MAX; }

__device__ __forceinline__ uint32_t nibble(const uint32_t* codes, uint32_t vector) {
  return (codes[vector >> 3] >> ((vector & 7u) * 4u)) & 15u;
}

template <typename T>
__device__ __forceinline__ const T* item_ptr(const void* base, uint64_t stride, uint32_t item) {
  return reinterpret_cast<const T*>(static_cast<const char*>(base) + stride * item);
}
template <typename T>
__device__ __forceinline__ T* item_ptr_mut(void* base, uint64_t stride, uint32_t item) {
  return reinterpret_cast<T*>(static_cast<char*>(base) + stride * item);
}

__device__ void sweep_books(const float* a, const float* b, uint32_t values, uint32_t* status) {
  bool bad = false;
  for (uint32_t i = threadIdx.x; i < values; i += blockDim.x)
    bad |= !finite_f32(a[i]) || !finite_f32(b[i]);
  if (__any(bad) && (threadIdx.x % warpSize) == 0) atomicOr(status, 1u);
}

// ---- General -------------------------------------------------------------
constexpr int kGT = 64;   // output tile edge
constexpr int kGK = 16;   // inner step
constexpr int kGThreads = 256;

template <int G>
__global__ __launch_bounds__(kGThreads) void k_matmul_general(Operands o, uint32_t m, uint32_t n,
                                                              uint32_t k, uint32_t flags) {
  __shared__ float sa_book[16 * G];
  __shared__ float sb_book[16 * G];
  __shared__ float as[kGK][kGT + 4];
  __shared__ float bs[kGK][kGT + 4];
  const uint32_t tid = threadIdx.x;
  const uint32_t tx = tid % 16, ty = tid / 16;
  const uint32_t n0 = blockIdx.x * kGT, m0 = blockIdx.y * kGT;
  for (uint32_t item = blockIdx.z; item < o.count; item += gridDim.z) {
    const uint32_t* a_codes = item_ptr<uint32_t>(o.in[0], o.stride[0], item);
    const float* a_book = item_ptr<float>(o.in[1], o.stride[1], item);
    const uint32_t* b_codes = item_ptr<uint32_t>(o.in[2], o.stride[2], item);
    const float* b_book = item_ptr<float>(o.in[3], o.stride[3], item);
    float* out = item_ptr_mut<float>(o.out, o.stride[4], item);
    __syncthreads();
    for (uint32_t i = tid; i < 16 * G; i += kGThreads) {
      sa_book[i] = a_book[i];
      sb_book[i] = b_book[i];
    }
    if (blockIdx.x == 0 && blockIdx.y == 0) sweep_books(a_book, b_book, 16 * G, o.status);
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    for (uint32_t k0 = 0; k0 < k; k0 += kGK) {
      __syncthreads();
#pragma unroll
      for (int t = 0; t < (kGK * kGT) / kGThreads; ++t) {
        const uint32_t e = tid + t * kGThreads;
        const uint32_t r = e % kGT, kk = e / kGT;
        const uint32_t inner = k0 + kk;
        float av = 0.0f, bv = 0.0f;
        if (inner < k) {
          const uint32_t row = m0 + r;
          if (row < m) {
            const uint32_t flat = (flags & 1u) ? inner * m + row : row * k + inner;
            av = sa_book[nibble(a_codes, flat / G) * G + flat % G];
          }
          const uint32_t col = n0 + r;
          if (col < n) {
            const uint32_t flat = (flags & 2u) ? col * k + inner : inner * n + col;
            bv = sb_book[nibble(b_codes, flat / G) * G + flat % G];
          }
        }
        as[kk][r] = av;
        bs[kk][r] = bv;
      }
      __syncthreads();
      const uint32_t steps = (k - k0) < kGK ? (k - k0) : kGK;
      for (uint32_t kk = 0; kk < steps; ++kk) {
        float a[4], b[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = as[kk][ty + 16 * i];
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = bs[kk][tx + 16 * j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float product = a[i] * b[j];
            acc[i][j] = acc[i][j] + product;
          }
      }
    }
    bool bad = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t row = m0 + ty + 16 * i;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t col = n0 + tx + 16 * j;
        if (row < m && col < n) {
          out[uint64_t(row) * n + col] = acc[i][j];
          bad |= !finite_f32(acc[i][j]);
        }
      }
    }
    if (__any(bad) && (tid % warpSize) == 0) atomicOr(o.status, 1u);
  }
}

// ---- GemvBins ------------------------------------------------------------
// Tile: kTileWords words of each B row (8 * kTileWords output groups), all m
// rows of A, a slice of k. In one batch each wave covers 32 rows: lane
// (q = lane % 32, half = lane / 32) reads word q of rows base + half*16 + u,
// u < 16, so every load instruction of a wave reads two whole 128-byte tile
// rows and a lane's 16 activations are contiguous in LDS. The next batch's
// words are loaded while the current batch is binned.
//
// The bins are 32-bit fixed point: x is scaled by 2^s (s from the A
// codebook's largest magnitude) and rounded to an integer once, when it is
// staged in LDS, and the bins are summed with integer LDS atomics -- exact,
// and on gfx950 some thirty times the rate of FP32 LDS atomics. Every
// kWindow rows the integer bins are flushed into FP32 accumulators held in
// registers, which bounds |bin| < 2^30 (no overflow) while keeping the
// rounding of x to 2^-s at most 2^-23 of the largest |x|.
// Bins are laid out [r][nibble][e][q]: the 32 lanes of a half-wave hit 32
// distinct banks for any codes.
constexpr int kTileWords = 32;
constexpr int kTileGroups = kTileWords * 8;
constexpr int kBinThreads = 256;
constexpr int kBinWaves = kBinThreads / 64;
constexpr int kRowsPerLane = 16;
constexpr uint32_t kBatchRows = kBinWaves * 2 * kRowsPerLane;   // 128 rows per batch
constexpr uint32_t kGemvMaxM = 8;
constexpr uint32_t kWindow = 1024;                              // rows per integer window
constexpr uint32_t kXBytes = 16384;                             // LDS for staged x
constexpr int kBinsPerThread = 16 * kTileGroups / kBinThreads;  // 16 bins per M row

// Rows of x staged at once: whole batches (so a lane's 16 activations never
// straddle a restage), restaged whenever the chunk is used up.
template <int M>
__host__ __device__ constexpr uint32_t x_chunk_rows() {
  return (kXBytes / (4 * M)) / kBatchRows * kBatchRows;
}
static_assert(x_chunk_rows<kGemvMaxM>() >= kBatchRows, "staged x must hold one batch per row");

// Byte offset of bin (e, q) for nibble NIB of w inside one M row's bins.
template <int NIB>
__device__ __forceinline__ uint32_t bin_byte(uint32_t w, uint32_t q4) {
  return (__builtin_amdgcn_ubfe(w, 4 * NIB, 4) << 7) | q4;
}

typedef __attribute__((address_space(3))) int32_t lds_i32;

// Integer add into LDS at an absolute byte address. The bins sit at LDS
// address 0 (the kernel has no static LDS), so a bin's address is known to
// the compiler bit for bit and needs no base addition.
__device__ __forceinline__ void lds_add(uint32_t byte_addr, int32_t v) {
  __hip_atomic_fetch_add(reinterpret_cast<lds_i32*>(static_cast<size_t>(byte_addr)), v,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ uint32_t bin_index(uint32_t r, uint32_t nib, uint32_t e, uint32_t q) {
  return ((r * 8 + nib) * 16 + e) * kTileWords + q;
}

// x[r][kk] for rows r < m and inner rows [k0, kend), decoded from A by flat
// index, scaled by 2^shift and rounded to int32 into sxq[r * rows + kk].
template <int G, int M>
__device__ void stage_x(const uint32_t* a_codes, const float* sa_book, uint32_t k, uint32_t flags,
                        uint32_t k0, uint32_t kend, uint32_t rows, int shift, int32_t* sxq) {
  for (uint32_t e = threadIdx.x; e < M * rows; e += blockDim.x) {
    const uint32_t r = e / rows, kk = e % rows;
    const uint32_t inner = k0 + kk;
    int32_t v = 0;
    if (inner < kend) {
      const uint32_t flat = (flags & 1u) ? inner * M + r : r * k + inner;
      v = int32_t(rintf(ldexpf(sa_book[nibble(a_codes, flat / G) * G + flat % G], shift)));
    }
    sxq[e] = v;
  }
}

// Largest |value| of a 16 x G book, reduced over the block.
template <int G>
__device__ float book_absmax(const float* sbook, float* sred) {
  float v = 0.0f;
  for (uint32_t i = threadIdx.x; i < 16 * G; i += blockDim.x) v = fmaxf(v, fabsf(sbook[i]));
  for (int off = 1; off < warpSize; off <<= 1) v = fmaxf(v, __shfl_xor(v, off));
  if (threadIdx.x % warpSize == 0) sred[threadIdx.x / warpSize] = v;
  __syncthreads();
  float m = 0.0f;
  for (uint32_t i = 0; i < blockDim.x / warpSize; ++i) m = fmaxf(m, sred[i]);
  __syncthreads();
  return m;
}

// Load this lane's 16 words of a batch (zero past kend or off the tile).
__device__ __forceinline__ void load_batch(const uint32_t* col_codes, uint32_t row_words,
                                           uint32_t first, uint32_t kend, bool live,
                                           uint32_t (&w)[kRowsPerLane]) {
#pragma unroll
  for (int u = 0; u < kRowsPerLane; ++u) {
    const uint32_t row = first + u;
    w[u] = (live && row < kend) ? col_codes[uint64_t(row) * row_words] : 0u;
  }
}

// grid: (n tiles, k splits, instances). Dynamic shared memory: the integer
// bins (M * 16 * kTileGroups) then the staged x (M * x_chunk_rows int32).
template <int G, int M>
__global__ __launch_bounds__(kBinThreads) void k_gemv_bins(Operands o, uint32_t n, uint32_t k,
                                                           uint32_t flags, uint32_t ks,
                                                           float* partial) {
  constexpr uint32_t kXRows = x_chunk_rows<M>();
  // All LDS is dynamic so the bins start at address 0: a bin address is then
  // (e << 7) | q4 with disjoint bits, one AND-OR per nibble.
  extern __shared__ int32_t smem[];
  int32_t* bins = smem;
  int32_t* sxq = smem + M * 16 * kTileGroups;
  float* fbins = reinterpret_cast<float*>(smem);
  float* sa_book = reinterpret_cast<float*>(sxq + kXBytes / 4);
  float* sb_book = sa_book + 16 * G;
  float* sred = sb_book + 16 * G;
  const uint32_t tid = threadIdx.x;
  const uint32_t tile = blockIdx.x, split = blockIdx.y;
  const uint32_t row_words = n / (8 * G);
  const uint32_t k0 = split * ks;
  const uint32_t kend = (k0 + ks) < k ? (k0 + ks) : k;
  const uint32_t lane = tid % 64, wave = tid / 64;
  const uint32_t q = lane % 32, half = lane / 32;
  const uint32_t q4 = q * 4;
  const uint32_t lane_row = wave * 32 + half * kRowsPerLane;  // first row of this lane in a batch
  const uint32_t word_col = tile * kTileWords + q;
  const bool live = word_col < row_words;
  // Defensive: absolute bin addresses assume the bins start at LDS 0.
  if (static_cast<uint32_t>(reinterpret_cast<size_t>((lds_i32*)bins)) != 0) {
    if (tid == 0) atomicOr(o.status, 2u);
    return;
  }
  for (uint32_t item = blockIdx.z; item < o.count; item += gridDim.z) {
    const uint32_t* a_codes = item_ptr<uint32_t>(o.in[0], o.stride[0], item);
    const float* a_book = item_ptr<float>(o.in[1], o.stride[1], item);
    const uint32_t* b_codes = item_ptr<uint32_t>(o.in[2], o.stride[2], item);
    const float* b_book = item_ptr<float>(o.in[3], o.stride[3], item);
    const uint32_t* col_codes = b_codes + word_col;
    // the first batch's words are in flight while the block sets up
    uint32_t wn[kRowsPerLane];
    load_batch(col_codes, row_words, k0 + lane_row, kend, live, wn);
    __syncthreads();
    for (uint32_t i = tid; i < 16 * G; i += kBinThreads) {
      sa_book[i] = a_book[i];
      sb_book[i] = b_book[i];
    }
    for (uint32_t i = tid; i < M * 16 * kTileGroups; i += kBinThreads) bins[i] = 0;
    if (tile == 0 && split == 0) sweep_books(a_book, b_book, 16 * G, o.status);
    __syncthreads();
    // 2^shift * max|x| * kWindow < 2^30: no window sum can overflow int32.
    const float xmax = book_absmax<G>(sa_book, sred);
    int shift = 0;
    if (xmax > 0.0f) {
      int ex;
      frexpf(xmax, &ex);  // xmax < 2^ex, so xmax * kWindow < 2^(ex + 10)
      shift = 30 - (ex + 10);
      shift = shift < -126 ? -126 : (shift > 126 ? 126 : shift);
    }
    const float unscale = ldexpf(1.0f, -shift);
    float acc[M][kBinsPerThread];
#pragma unroll
    for (int r = 0; r < M; ++r)
#pragma unroll
      for (int i = 0; i < kBinsPerThread; ++i) acc[r][i] = 0.0f;

    uint32_t xbase = k0;  // first row of the staged x chunk
    stage_x<G, M>(a_codes, sa_book, k, flags, xbase, kend, kXRows, shift, sxq);
    __syncthreads();
    for (uint32_t kb = k0; kb < kend; kb += kBatchRows) {
      uint32_t w[kRowsPerLane];
#pragma unroll
      for (int u = 0; u < kRowsPerLane; ++u) w[u] = wn[u];
      if (kb + kBatchRows < kend)
        load_batch(col_codes, row_words, kb + kBatchRows + lane_row, kend, live, wn);
      if (live) {
        const uint32_t first = kb + lane_row;
#pragma unroll
        for (int r = 0; r < M; ++r) {
          const uint32_t base = r * (16 * kTileGroups * 4);
          // the lane's 16 activations, 16-byte aligned; rows past kend are
          // staged as zero (and carry w = 0), so their adds are no-ops
          const int4* xr = reinterpret_cast<const int4*>(sxq + r * kXRows + (first - xbase));
          int32_t xs[kRowsPerLane];
#pragma unroll
          for (int i = 0; i < kRowsPerLane / 4; ++i) {
            const int4 v = xr[i];
            xs[4 * i] = v.x; xs[4 * i + 1] = v.y; xs[4 * i + 2] = v.z; xs[4 * i + 3] = v.w;
          }
#pragma unroll
          for (int u = 0; u < kRowsPerLane; ++u) {
            const int32_t xv = xs[u];
            const uint32_t ww = w[u];
            lds_add(base + 0 * 2048 + bin_byte<0>(ww, q4), xv);
            lds_add(base + 1 * 2048 + bin_byte<1>(ww, q4), xv);
            lds_add(base + 2 * 2048 + bin_byte<2>(ww, q4), xv);
            lds_add(base + 3 * 2048 + bin_byte<3>(ww, q4), xv);
            lds_add(base + 4 * 2048 + bin_byte<4>(ww, q4), xv);
            lds_add(base + 5 * 2048 + bin_byte<5>(ww, q4), xv);
            lds_add(base + 6 * 2048 + bin_byte<6>(ww, q4), xv);
            lds_add(base + 7 * 2048 + bin_byte<7>(ww, q4), xv);
          }
        }
      }
      const uint32_t done = kb + kBatchRows;
      const bool flush = done >= kend || (done - k0) % kWindow == 0;
      const bool restage = done < kend && done - xbase >= kXRows;
      if (flush || restage) {
        __syncthreads();
        if (flush) {
          // the window ends: integer bins -> FP32 accumulators, bins reset
#pragma unroll
          for (int r = 0; r < M; ++r)
#pragma unroll
            for (int i = 0; i < kBinsPerThread; ++i) {
              const uint32_t b = r * 16 * kTileGroups + tid + i * kBinThreads;
              acc[r][i] += float(bins[b]);
              bins[b] = 0;
            }
        }
        if (restage) {
          xbase = done;
          stage_x<G, M>(a_codes, sa_book, k, flags, xbase, kend, kXRows, shift, sxq);
        }
        __syncthreads();
      }
    }
#pragma unroll
    for (int r = 0; r < M; ++r)
#pragma unroll
      for (int i = 0; i < kBinsPerThread; ++i)
        fbins[r * 16 * kTileGroups + tid + i * kBinThreads] = acc[r][i] * unscale;
    __syncthreads();

    // Finalise this tile: y[r][j*G+t] = sum_e C_B[e][t] * S[r][j][e].
    const uint32_t groups = (row_words - tile * kTileWords) < kTileWords
                                ? (row_words - tile * kTileWords) * 8
                                : kTileGroups;
    if (gridDim.y == 1) {
      float* out = item_ptr_mut<float>(o.out, o.stride[4], item);
      bool bad = false;
      for (uint32_t e = tid; e < M * groups * G; e += kBinThreads) {
        const uint32_t r = e / (groups * G);
        const uint32_t jt = e % (groups * G);
        const uint32_t j = jt / G, t = jt % G;
        float y = 0.0f;
#pragma unroll
        for (uint32_t c = 0; c < 16; ++c)
          y = fmaf(sb_book[c * G + t], fbins[bin_index(r, j % 8, c, j / 8)], y);
        out[uint64_t(r) * n + tile * kTileGroups * G + jt] = y;
        bad |= !finite_f32(y);
      }
      if (__any(bad) && (tid % warpSize) == 0) atomicOr(o.status, 1u);
    } else {
      // partial[item][tile][split][r][j][e]
      float* p = partial + ((uint64_t(item) * gridDim.x + tile) * gridDim.y + split) *
                               (M * 16 * kTileGroups);
      for (uint32_t e = tid; e < M * 16 * kTileGroups; e += kBinThreads) {
        const uint32_t r = e / (16 * kTileGroups);
        const uint32_t je = e % (16 * kTileGroups);
        const uint32_t j = je / 16, c = je % 16;
        p[e] = fbins[bin_index(r, j % 8, c, j / 8)];
      }
    }
  }
}

// Sum the split-k bins in split order (one thread per bin), then apply the B
// codebook. grid: (n tiles * kFinishParts, 1, instances); each block owns
// kTileGroups / kFinishParts groups of one tile.
constexpr uint32_t kFinishParts = 16;
constexpr uint32_t kFinishGroups = kTileGroups / kFinishParts;  // 16 groups, 256 bins

template <int G, int M>
__global__ __launch_bounds__(256) void k_gemv_bins_finish(Operands o, uint32_t n, uint32_t splits,
                                                          uint32_t tiles, const float* partial) {
  __shared__ float sb_book[16 * G];
  __shared__ float ssum[M][kFinishGroups * 16];
  const uint32_t tile = blockIdx.x / kFinishParts, part = blockIdx.x % kFinishParts;
  const uint32_t row_words = n / (8 * G);
  const uint32_t groups = (row_words - tile * kTileWords) < kTileWords
                              ? (row_words - tile * kTileWords) * 8
                              : kTileGroups;
  const uint32_t j0 = part * kFinishGroups;
  if (j0 >= groups) return;
  const uint32_t jn = (groups - j0) < kFinishGroups ? (groups - j0) : kFinishGroups;
  for (uint32_t item = blockIdx.z; item < o.count; item += gridDim.z) {
    const float* b_book = item_ptr<float>(o.in[3], o.stride[3], item);
    float* out = item_ptr_mut<float>(o.out, o.stride[4], item);
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < 16 * G; i += blockDim.x) sb_book[i] = b_book[i];
    const float* base = partial + (uint64_t(item) * tiles + tile) * splits * (M * 16 * kTileGroups);
    for (uint32_t e = threadIdx.x; e < M * jn * 16; e += blockDim.x) {
      const uint32_t r = e / (jn * 16), je = e % (jn * 16);
      const float* p = base + r * 16 * kTileGroups + j0 * 16 + je;
      float s = 0.0f;
      for (uint32_t sp = 0; sp < splits; ++sp) s += p[uint64_t(sp) * (M * 16 * kTileGroups)];
      ssum[r][je] = s;
    }
    __syncthreads();
    bool bad = false;
    for (uint32_t e = threadIdx.x; e < M * jn * G; e += blockDim.x) {
      const uint32_t r = e / (jn * G), jt = e % (jn * G);
      const uint32_t j = jt / G, t = jt % G;
      float y = 0.0f;
#pragma unroll
      for (int c = 0; c < 16; ++c) y = fmaf(sb_book[c * G + t], ssum[r][j * 16 + c], y);
      out[uint64_t(r) * n + (tile * kTileGroups + j0) * G + jt] = y;
      bad |= !finite_f32(y);
    }
    if (__any(bad) && (threadIdx.x % warpSize) == 0) atomicOr(o.status, 1u);
  }
}

// ---- GemvPairs (m = 1) -----------------------------------------------------
// The two nibbles of a byte of a B row are the codes of two output groups of
// the same inner row, so they receive the same x. One integer atomic into a
// 256-way "pair bin" indexed by the whole byte replaces GemvBins' two:
//   S[2p][e]   = sum over hi of P[p][16 hi + e]   (low nibble = group 8q+2p)
//   S[2p+1][e] = sum over lo of P[p][16 e + lo]   (high nibble = group 8q+2p+1)
// Pair bins are laid out [byte value][pair p][word q] (128 KiB for a 32-word
// tile), so a bin address is (byte << 9) | (p << 7) | 4q: p is an immediate
// offset and the 32 lanes of a half-wave hit 32 distinct banks.
//
// Integer windows are kPairWindow rows: x is scaled so that
// max|x| * 2^shift * kPairWindow < 2^30 (a quantisation step of 2^-20 of
// max|x|), and the bins are flushed into FP32 registers once per window.
// Every load of the main loop is unconditional: rows past the slice read as
// zero words through the buffer descriptor's range and meet x = 0; dead words
// are clamped to the last word and never binned.
constexpr int kPairThreads = 512;
constexpr int kPairWaves = kPairThreads / 64;
constexpr uint32_t kPairBatchRows = kPairWaves * 2 * kRowsPerLane;  // 256 rows per batch
constexpr uint32_t kPairBins = 256 * 4 * kTileWords;                // 32768
constexpr uint32_t kPairXRows = 8 * kPairThreads;                   // staged x rows (16 KiB)
constexpr uint32_t kPairWindow = 2048;
constexpr int kPairVec = kPairBins / (4 * kPairThreads);            // int4 bins per thread
static_assert(kPairWindow % kPairBatchRows == 0 && kPairXRows % kPairBatchRows == 0, "batches");
static_assert(kPairXRows >= 16 * kTileGroups, "S reuses the x staging area");

template <int BYTE>
__device__ __forceinline__ uint32_t pair_addr(uint32_t w, uint32_t q4) {
  return ((__builtin_amdgcn_ubfe(w, 8 * BYTE, 8) << 9) | q4) + BYTE * 128;
}

// Buffer descriptor over the first `rows` rows of a code matrix: raw buffer
// loads past it return zero, which is how rows past a slice read.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t code_rows(const uint32_t* codes, uint32_t rows,
                                                            uint32_t row_words) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(codes), 0,
                                           int(rows * row_words * 4u), 0x00020000);
}

// This lane's 16 words of a batch from word column `col`, rows first ..
// first+15: one 32-bit byte offset per load (a matrix holds fewer than 2^30
// words), no 64-bit address arithmetic.
__device__ __forceinline__ void load_rows(__amdgpu_buffer_rsrc_t rs, uint32_t col,
                                          uint32_t row_words, uint32_t first,
                                          uint32_t (&w)[kRowsPerLane]) {
  const uint32_t base = (first * row_words + col) * 4u;
#pragma unroll
  for (int u = 0; u < kRowsPerLane; ++u)
    w[u] = uint32_t(__builtin_amdgcn_raw_buffer_load_b32(rs, base + u * row_words * 4u, 0, 0));
}

// Largest |value| of a 16 x G book in LDS, per wave.
template <int G>
__device__ float wave_book_absmax(const float* sbook) {
  float v = 0.0f;
  for (uint32_t i = threadIdx.x % 64; i < 16 * G; i += 64) v = fmaxf(v, fabsf(sbook[i]));
  for (int off = 1; off < 64; off <<= 1) v = fmaxf(v, __shfl_xor(v, off));
  return v;
}

// x rows [xbase, xbase + kPairXRows) of the single row of A, scaled by
// 2^shift and rounded, into sxq; rows at or past kend are zero. Thread t
// stages rows 8t .. 8t+7, which lie in one group of A (8 divides G and
// xbase); `a_word` is the code word holding that group's nibble.
template <int G>
__device__ void stage_x1(uint32_t a_word, const float* sa_book, uint32_t xbase, uint32_t kend,
                         int shift, int32_t* sxq) {
  const uint32_t r0 = xbase + 8 * threadIdx.x;
  int32_t v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (r0 < kend) {
    const uint32_t code = (a_word >> (((r0 / G) & 7u) * 4u)) & 15u;
    const float4* c = reinterpret_cast<const float4*>(sa_book + code * G + r0 % G);
    const float4 c0 = c[0], c1 = c[1];
    const float x[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
    for (int i = 0; i < 8; ++i)
      v[i] = (r0 + i < kend) ? int32_t(rintf(ldexpf(x[i], shift))) : 0;
  }
  int4* dst = reinterpret_cast<int4*>(sxq + 8 * threadIdx.x);
  dst[0] = make_int4(v[0], v[1], v[2], v[3]);
  dst[1] = make_int4(v[4], v[5], v[6], v[7]);
}

__device__ __forceinline__ uint32_t stage_word(const uint32_t* a_codes, uint32_t xbase,
                                               uint32_t kend, uint32_t group) {
  const uint32_t r0 = xbase + 8 * threadIdx.x;
  return r0 < kend ? a_codes[(r0 / group) >> 3] : 0u;
}

// What an instance's set-up reads from global memory besides its first batch
// of B words, loaded during the previous instance: this thread's staging code
// word and one entry of each book (16 * G <= kPairThreads).
struct PairAhead {
  uint32_t a_word;
  float a_entry, b_entry;
};

template <int G>
__device__ __forceinline__ void pair_setup_loads(const Operands& o, uint32_t item, uint32_t k0,
                                                 uint32_t kend, PairAhead& ah) {
  const uint32_t* a_codes = item_ptr<uint32_t>(o.in[0], o.stride[0], item);
  const float* a_book = item_ptr<float>(o.in[1], o.stride[1], item);
  const float* b_book = item_ptr<float>(o.in[3], o.stride[3], item);
  ah.a_word = stage_word(a_codes, k0, kend, G);
  const uint32_t i = threadIdx.x < 16 * G ? threadIdx.x : 0;
  ah.a_entry = a_book[i];
  ah.b_entry = b_book[i];
}

// grid: (n tiles, k splits, z); block z serves instances z, z + gridDim.z, ...
// ks is a multiple of kPairBatchRows. Dynamic shared memory: pair bins,
// staged x (later S), the A and B books.
template <int G>
__global__ __launch_bounds__(kPairThreads) void k_gemv_pairs(Operands o, uint32_t n, uint32_t k,
                                                             uint32_t ks, float* partial) {
  static_assert(16 * G <= kPairThreads, "one book entry per thread");
  extern __shared__ int32_t smem[];
  int32_t* bins = smem;
  int32_t* sxq = smem + kPairBins;
  float* ss = reinterpret_cast<float*>(sxq);  // S after the main loop: [e][n8][q]
  float* sa_book = reinterpret_cast<float*>(sxq + kPairXRows);
  float* sb_book = sa_book + 16 * G;
  const uint32_t tid = threadIdx.x;
  const uint32_t tile = blockIdx.x, split = blockIdx.y;
  const uint32_t row_words = n / (8 * G);
  const uint32_t k0 = split * ks;
  const uint32_t kend = (k0 + ks) < k ? (k0 + ks) : k;
  const uint32_t lane = tid % 64, wave = tid / 64;
  const uint32_t q = lane % 32, half = lane / 32;
  const uint32_t q4 = q * 4;
  const uint32_t lane_row = wave * 32 + half * kRowsPerLane;
  const bool live = tile * kTileWords + q < row_words;
  const uint32_t word_col = live ? tile * kTileWords + q : row_words - 1;
  if (static_cast<uint32_t>(reinterpret_cast<size_t>((lds_i32*)bins)) != 0) {
    if (tid == 0) atomicOr(o.status, 2u);
    return;
  }
  int4* bins4 = reinterpret_cast<int4*>(bins);
  PairAhead ah;
  uint32_t wn[kRowsPerLane];  // the next batch's words
  if (blockIdx.z < o.count) {
    pair_setup_loads<G>(o, blockIdx.z, k0, kend, ah);
    load_rows(code_rows(item_ptr<uint32_t>(o.in[2], o.stride[2], blockIdx.z), kend, row_words),
              word_col, row_words, k0 + lane_row, wn);
  }
  for (uint32_t item = blockIdx.z; item < o.count; item += gridDim.z) {
    const uint32_t* a_codes = item_ptr<uint32_t>(o.in[0], o.stride[0], item);
    const __amdgpu_buffer_rsrc_t b_rows =
        code_rows(item_ptr<uint32_t>(o.in[2], o.stride[2], item), kend, row_words);
    // The last batch loads the next instance's first batch (this one's when
    // there is none, unused): the batch loads never sit behind a branch, so
    // the wait before binning a batch leaves the following batch in flight.
    const uint32_t next = item + gridDim.z;
    const bool has_next = next < o.count;
    const __amdgpu_buffer_rsrc_t next_rows =
        code_rows(item_ptr<uint32_t>(o.in[2], o.stride[2], has_next ? next : item), kend,
                  row_words);
    const uint32_t a_word = ah.a_word;
    __syncthreads();  // the previous instance's S and books are no longer read
    if (tid < 16 * G) {
      sa_book[tid] = ah.a_entry;
      sb_book[tid] = ah.b_entry;
    }
#pragma unroll
    for (int i = 0; i < kPairVec; ++i) bins4[tid + i * kPairThreads] = make_int4(0, 0, 0, 0);
    __syncthreads();
    if (tile == 0 && split == 0) sweep_books(sa_book, sb_book, 16 * G, o.status);
    const float xmax = wave_book_absmax<G>(sa_book);
    int shift = 0;
    if (xmax > 0.0f) {
      int ex;
      frexpf(xmax, &ex);  // xmax < 2^ex, so xmax * kPairWindow < 2^(ex + 11)
      shift = 30 - (ex + 11);
      shift = shift < -126 ? -126 : (shift > 126 ? 126 : shift);
    }
    const float unscale = ldexpf(1.0f, -shift);
    float acc[kPairVec][4];
#pragma unroll
    for (int i = 0; i < kPairVec; ++i) acc[i][0] = acc[i][1] = acc[i][2] = acc[i][3] = 0.0f;

    uint32_t xbase = k0;
    stage_x1<G>(a_word, sa_book, xbase, kend, shift, sxq);
    __syncthreads();
    for (uint32_t kb = k0; kb < kend; kb += kPairBatchRows) {
      uint32_t w[kRowsPerLane];
#pragma unroll
      for (int u = 0; u < kRowsPerLane; ++u) w[u] = wn[u];
      const bool last = kb + kPairBatchRows >= kend;
      load_rows(last ? next_rows : b_rows, word_col, row_words,
                (last ? k0 : kb + kPairBatchRows) + lane_row, wn);
      if (live) {
        const int4* xr = reinterpret_cast<const int4*>(sxq + (kb + lane_row - xbase));
        int32_t xs[kRowsPerLane];
#pragma unroll
        for (int i = 0; i < kRowsPerLane / 4; ++i) {
          const int4 v = xr[i];
          xs[4 * i] = v.x; xs[4 * i + 1] = v.y; xs[4 * i + 2] = v.z; xs[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int u = 0; u < kRowsPerLane; ++u) {
          const int32_t xv = xs[u];
          const uint32_t ww = w[u];
          lds_add(pair_addr<0>(ww, q4), xv);
          lds_add(pair_addr<1>(ww, q4), xv);
          lds_add(pair_addr<2>(ww, q4), xv);
          lds_add(pair_addr<3>(ww, q4), xv);
        }
      }
      if (last && has_next) pair_setup_loads<G>(o, next, k0, kend, ah);
      const uint32_t done = kb + kPairBatchRows;
      const bool flush = done >= kend || (done - k0) % kPairWindow == 0;
      const bool restage = done < kend && done - xbase >= kPairXRows;
      if (flush || restage) {
        // a restage reads its code word before the barrier
        const uint32_t rword = restage ? stage_word(a_codes, done, kend, G) : 0u;
        __syncthreads();
        if (flush) {
#pragma unroll
          for (int i = 0; i < kPairVec; ++i) {
            const int4 v = bins4[tid + i * kPairThreads];
            acc[i][0] += float(v.x);
            acc[i][1] += float(v.y);
            acc[i][2] += float(v.z);
            acc[i][3] += float(v.w);
            if (done < kend) bins4[tid + i * kPairThreads] = make_int4(0, 0, 0, 0);
          }
        }
        if (restage) {
          xbase = done;
          stage_x1<G>(rword, sa_book, xbase, kend, shift, sxq);
        }
        __syncthreads();
      }
    }
    // pair bins in FP32, in place; then S for the tile's groups
    float4* fb4 = reinterpret_cast<float4*>(smem);
#pragma unroll
    for (int i = 0; i < kPairVec; ++i)
      fb4[tid + i * kPairThreads] = make_float4(acc[i][0] * unscale, acc[i][1] * unscale,
                                                acc[i][2] * unscale, acc[i][3] * unscale);
    __syncthreads();
    // Thread idx takes word qq = idx % 32 (consecutive lanes read consecutive
    // banks) and nibble n8 = 2p + s, code e of the rest: group j = 8 qq + n8.
    const float* fb = reinterpret_cast<const float*>(smem);
    float* pp = partial + ((uint64_t(item) * gridDim.x + tile) * gridDim.y + split) *
                              (16 * kTileGroups);
    for (uint32_t idx = tid; idx < 16 * kTileGroups; idx += kPairThreads) {
      const uint32_t qq = idx % kTileWords, rest = idx / kTileWords;
      const uint32_t n8 = rest % 8, e = rest / 8;
      const uint32_t p = n8 / 2;
      const uint32_t stride = (n8 & 1u) ? 1u : 16u;   // the other nibble's step in the byte
      const uint32_t v0 = (n8 & 1u) ? 16u * e : e;
      float sum = 0.0f;
#pragma unroll
      for (uint32_t other = 0; other < 16; ++other)
        sum += fb[((v0 + stride * other) * 4 + p) * kTileWords + qq];
      if (gridDim.y == 1) ss[idx] = sum;
      else pp[(qq * 8 + n8) * 16 + e] = sum;  // the finish kernel's [j][e]
    }
    __syncthreads();

    const uint32_t groups = (row_words - tile * kTileWords) < kTileWords
                                ? (row_words - tile * kTileWords) * 8
                                : kTileGroups;
    if (gridDim.y == 1) {
      // thread tid always takes column t = tid % G: its 16 book entries stay in registers
      const uint32_t t = tid % G;
      float cb[16];
#pragma unroll
      for (uint32_t c = 0; c < 16; ++c) cb[c] = sb_book[c * G + t];
      float* out = item_ptr_mut<float>(o.out, o.stride[4], item);
      bool bad = false;
      for (uint32_t e = tid; e < groups * G; e += kPairThreads) {
        const uint32_t j = e / G;
        const float* sj = ss + (j % 8) * kTileWords + j / 8;
        float y = 0.0f;
#pragma unroll
        for (uint32_t c = 0; c < 16; ++c) y = fmaf(cb[c], sj[c * kTileGroups], y);
        out[tile * kTileGroups * G + e] = y;
        bad |= !finite_f32(y);
      }
      if (__any(bad) && (tid % warpSize) == 0) atomicOr(o.status, 1u);
    }
  }
}

size_t pairs_shmem(uint32_t g) {
  return size_t(kPairBins) * 4 + kPairXRows * 4 + 2 * 16 * g * 4;
}

uint32_t gemv_splits(uint32_t n, uint32_t k, uint32_t group, uint32_t count) {
  const uint32_t tiles = (n / (8 * group) + kTileWords - 1) / kTileWords;
  const uint64_t blocks = uint64_t(tiles) * count;
  // Enough blocks for 256 compute units; never slices shorter than 256 rows.
  uint32_t splits = 1;
  while (blocks * splits < 256 && k / (splits * 2) >= 256) splits *= 2;
  return splits;
}

// Slices of k for GemvPairs: gemv_splits' count, each slice rounded up to
// whole batches, and only the slices that hold rows.
void pairs_slices(uint32_t n, uint32_t k, uint32_t group, uint32_t count, uint32_t* ks,
                  uint32_t* splits) {
  const uint32_t want = gemv_splits(n, k, group, count);
  const uint32_t per = (k + want - 1) / want;
  *ks = (per + kPairBatchRows - 1) / kPairBatchRows * kPairBatchRows;
  *splits = (k + *ks - 1) / *ks;
}

size_t bins_shmem(uint32_t m, uint32_t g) {
  return size_t(m) * 16 * kTileGroups * 4 + kXBytes + 2 * 16 * g * 4 + kBinWaves * 4;
}

template <int G, int M>
hipError_t launch_bins_m(hipStream_t s, const Operands& o, uint32_t n, uint32_t k, uint32_t flags,
                         void* workspace) {
  const uint32_t tiles = (n / (8 * G) + kTileWords - 1) / kTileWords;
  const uint32_t splits = gemv_splits(n, k, G, o.count);
  const uint32_t ks = (k + splits - 1) / splits;
  const uint32_t zc = o.count < 65535 ? o.count : 65535;
  const size_t shmem = bins_shmem(M, G);
  if (shmem > 65536) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv_bins<G, M>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, int(shmem));
    if (e != hipSuccess) return e;
  }
  dim3 grid(tiles, splits, zc);
  k_gemv_bins<G, M><<<grid, kBinThreads, shmem, s>>>(o, n, k, flags, ks,
                                                     static_cast<float*>(workspace));
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || splits == 1) return err;
  dim3 fgrid(tiles * kFinishParts, 1, zc);
  k_gemv_bins_finish<G, M><<<fgrid, 256, 0, s>>>(o, n, splits, tiles,
                                                 static_cast<const float*>(workspace));
  return hipGetLastError();
}

template <int G>
hipError_t launch_pairs(hipStream_t s, const Operands& o, uint32_t n, uint32_t k, uint32_t flags,
                        void* workspace) {
  (void)flags;  // m = 1: A's flat index is the inner index either way
  const uint32_t tiles = (n / (8 * G) + kTileWords - 1) / kTileWords;
  uint32_t ks, splits;
  pairs_slices(n, k, G, o.count, &ks, &splits);
  // about one block per compute unit; each block walks its instances and
  // loads the next one's set-up while it finishes the current one
  const uint32_t per_z = tiles * splits;
  uint32_t zc = per_z >= 256 ? 1u : 256u / per_z;
  zc = zc < o.count ? zc : o.count;
  const size_t shmem = pairs_shmem(G);
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv_pairs<G>),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, int(shmem));
  if (e != hipSuccess) return e;
  dim3 grid(tiles, splits, zc);
  k_gemv_pairs<G><<<grid, kPairThreads, shmem, s>>>(o, n, k, ks, static_cast<float*>(workspace));
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || splits == 1) return err;
  dim3 fgrid(tiles * kFinishParts, 1, zc);
  k_gemv_bins_finish<G, 1><<<fgrid, 256, 0, s>>>(o, n, splits, tiles,
                                                 static_cast<const float*>(workspace));
  return hipGetLastError();
}

template <int G>
hipError_t launch_bins(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                       uint32_t flags, void* workspace) {
  switch (m) {
    case 1: return launch_bins_m<G, 1>(s, o, n, k, flags, workspace);
    case 2: return launch_bins_m<G, 2>(s, o, n, k, flags, workspace);
    case 3: return launch_bins_m<G, 3>(s, o, n, k, flags, workspace);
    case 4: return launch_bins_m<G, 4>(s, o, n, k, flags, workspace);
    case 5: return launch_bins_m<G, 5>(s, o, n, k, flags, workspace);
    case 6: return launch_bins_m<G, 6>(s, o, n, k, flags, workspace);
    case 7: return launch_bins_m<G, 7>(s, o, n, k, flags, workspace);
    default: return launch_bins_m<G, 8>(s, o, n, k, flags, workspace);
  }
}

}  // namespace

const char* matmul_path_name(MatmulPath p) {
  switch (p) {
    case MatmulPath::General: return "general";
    case MatmulPath::GemvBins: return "gemv-bins";
    case MatmulPath::GemvPairs: return "gemv-pairs";
    case MatmulPath::GemvTable: return "gemv-table";
    case MatmulPath::GramMfma: return "gram-mfma";
    case MatmulPath::RowBins: return "row-bins";
  }
  return "unknown";
}

MatmulPath choose_matmul_path(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                              uint32_t count, uint32_t policy) {
  if (policy == 1) return MatmulPath::General;
  if (count == 1 && rowbins_applies(m, n, k, group, flags)) return MatmulPath::RowBins;
  if (gram_applies(m, n, k, group, flags)) return MatmulPath::GramMfma;
  if (m <= kGemvMaxM && (flags & 2u) == 0 && n % (8 * group) == 0)
    return m == 1 ? MatmulPath::GemvPairs : MatmulPath::GemvBins;
  return MatmulPath::General;
}

size_t matmul_workspace_bytes(MatmulPath p, uint32_t m, uint32_t n, uint32_t k, uint32_t group,
                              uint32_t flags, uint32_t count) {
  (void)flags;
  if (p == MatmulPath::RowBins) return rowbins_workspace_bytes(n, k, group);
  if (p != MatmulPath::GemvBins && p != MatmulPath::GemvPairs) return 0;
  uint32_t splits = gemv_splits(n, k, group, count);
  if (p == MatmulPath::GemvPairs) {
    uint32_t ks;
    pairs_slices(n, k, group, count, &ks, &splits);
  }
  if (splits == 1) return 0;
  const uint32_t tiles = (n / (8 * group) + kTileWords - 1) / kTileWords;
  return size_t(count) * splits * tiles * m * 16 * kTileGroups * sizeof(float);
}

hipError_t launch_matmul(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                         uint32_t group, uint32_t flags, MatmulPath path, void* workspace,
                         size_t workspace_bytes) {
  (void)workspace_bytes;
  if (path == MatmulPath::RowBins) return launch_rowbins(s, o, m, n, k, group, workspace);
  if (path == MatmulPath::GramMfma) return launch_gram(s, o, m, n, k, group);
  if (path == MatmulPath::GemvPairs) {
    if (group == 8) return launch_pairs<8>(s, o, n, k, flags, workspace);
    if (group == 16) return launch_pairs<16>(s, o, n, k, flags, workspace);
    return launch_pairs<32>(s, o, n, k, flags, workspace);
  }
  if (path == MatmulPath::GemvBins) {
    if (group == 8) return launch_bins<8>(s, o, m, n, k, flags, workspace);
    if (group == 16) return launch_bins<16>(s, o, m, n, k, flags, workspace);
    return launch_bins<32>(s, o, m, n, k, flags, workspace);
  }
  const uint32_t zc = o.count < 65535 ? o.count : 65535;
  dim3 grid((n + kGT - 1) / kGT, (m + kGT - 1) / kGT, zc);
  if (group == 8) k_matmul_general<8><<<grid, kGThreads, 0, s>>>(o, m, n, k, flags);
  else if (group == 16) k_matmul_general<16><<<grid, kGThreads, 0, s>>>(o, m, n, k, flags);
  else k_matmul_general<32><<<grid, kGThreads, 0, s>>>(o, m, n, k, flags);
  return hipGetLastError();
}

}  // namespace ackvq
