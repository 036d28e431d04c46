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
// * The GEMV paths (m <= 8, B stored (k,n) with each row a whole number of
//   words): per output group j and code e they accumulate
//   S[r][j][e] = sum over rows k with code(k,j) = e of x[r][k] with integer
//   LDS atomics, then y[r][j*G+t] = sum_e C_B[e][t] * S[r][j][e]. That is G
//   times fewer additions than decoding the weight, which is what lets a
//   product that reads only half a byte per G weights run at the packed-weight
//   bandwidth instead of the FP32 FMA rate. GemvPairs (m = 1) bins whole bytes,
//   GemvRows (2..8) bins nibbles two rows at a time. The summation order
//   differs from the shader's; results agree within FP32 rounding.
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

// AD: A is a dense FP32 array in in[0] (the dense-activation product), read
// at the same flat index the packed A would be decoded at.
template <int G, bool AD>
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
    const float* a_dense = item_ptr<float>(o.in[0], o.stride[0], item);
    __syncthreads();
    for (uint32_t i = tid; i < 16 * G; i += kGThreads) {
      if (!AD) sa_book[i] = a_book[i];
      sb_book[i] = b_book[i];
    }
    if (blockIdx.x == 0 && blockIdx.y == 0)
      sweep_books(AD ? b_book : a_book, b_book, 16 * G, o.status);
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
            av = AD ? a_dense[flat] : sa_book[nibble(a_codes, flat / G) * G + flat % G];
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

// ---- shared by the GEMV paths ------------------------------------------------
// A tile is kTileWords words of each B row (8 * kTileWords output groups);
// the bins are 32-bit (or paired 64-bit) fixed point in LDS: each activation
// x is scaled by 2^s and rounded once, and integer LDS atomics -- exact, and
// on gfx950 about fifty times the rate of FP32 LDS atomics -- accumulate it.
// Rows of k are binned in windows; at a window's end its bins are flushed into
// FP32 registers, scaled back by 2^-s.
//
// The scale of a window comes from its positive and negative masses (per row
// of A), P = sum of its x > 0 and N = sum of |x| over its x < 0: a bin holds
// the sum over a subset of those rows, so every bin, and every sum of bins
// taken later, lies in [-(2^s N + rows/2), 2^s P + rows/2]. With M = max(P, N),
// choosing 2^s M (1 + 2^-8) < 2^31 keeps all of them inside int32 whatever the
// codes (the margin covers the FP32 rounding of the two sums, ~20 ulps, and
// the half-units), and makes the rounding step 2^-s at most 2^-30 (1 + 2^-8) M.
// So each x is rounded by at most 2^-31 (1 + 2^-8) M absolutely: an outlier
// raises M by its own magnitude only, and for activations of either sign M is
// about half the L1 norm P + N, one bit finer than a scale from L1.
constexpr int kTileWords = 32;
constexpr int kTileGroups = kTileWords * 8;
constexpr uint32_t kGemvMaxM = 8;    // rows of A one GEMV launch bins
constexpr uint32_t kRowsMaxM = 64;   // taller A runs GemvRows in chunks of kGemvMaxM rows
// ... when B is large enough (n * k elements) that the general kernel's few
// output tiles would leave the chip idle; smaller products keep the general
// kernel, which reproduces the shader's sums bit for bit.
constexpr uint64_t kRowsChunkMinWeight = 1ull << 20;

bool rows_apply(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags) {
  if ((flags & 2u) != 0 || n % (8 * group) != 0) return false;
  return m <= kGemvMaxM || (m <= kRowsMaxM && uint64_t(n) * k >= kRowsChunkMinWeight);
}

// "gemv-row-pairs": 2 <= m <= 8 rows of a row-major A, each its own instance of
// the m = 1 pair-bin kernel, when the row instances alone fill the chip (256
// blocks or more without splitting k). Packed A rows must start on whole code
// words (k a multiple of 8 g); dense rows may start anywhere.
bool row_pairs_apply(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                     uint32_t count, bool dense) {
  if (m < 2 || m > kGemvMaxM || flags != 0 || n % (8 * group) != 0) return false;
  if (!dense && k % (8 * group) != 0) return false;
  const uint64_t tiles = (n / (8 * group) + kTileWords - 1) / kTileWords;
  return tiles * count * m >= 256;
}

// A window's fixed-point scale: x -> rint(x 2^shift), from the window's L1.
__device__ __forceinline__ int window_shift(float l1) {
  // zero, NaN or Inf: callers raise status bit 1 for the last two (a NaN or
  // Inf value, or finite values whose L1 overflows FP32, which no int32
  // scale can hold), so whatever the bins then hold is never trusted
  if (!(l1 > 0.0f && l1 <= FLT_MAX)) return 0;
  float t = l1 * (1.0f + 0x1p-8f);
  t = t <= FLT_MAX ? t : FLT_MAX;
  int ex;
  frexpf(t, &ex);  // t < 2^ex, so 2^shift * l1 * (1 + 2^-8) < 2^31
  return 31 - ex;
}

// S 2^-shift in two power-of-two steps, so that a shift above 126
// (activations summing below 2^-96) needs no clamp: the first product is
// exact, the second rounds once, as S 2^-shift itself would.
__device__ __forceinline__ float unscale(float v, int shift) {
  const int s1 = shift < 126 ? shift : 126;
  return ldexpf(ldexpf(v, -s1), s1 - shift);
}

// 2^31 - 128, the largest float below 2^31: finite activations never reach it
// (|x| 2^shift < 2^31 (1 - 2^-9)); NaN and Inf, which status bit 1 reports,
// are clamped so that the integer conversion stays defined.
constexpr float kQuantMax = 2147483520.0f;

__device__ __forceinline__ int32_t quantize(float x, int shift) {
  const float v = rintf(ldexpf(x, shift));
  return int32_t(fminf(fmaxf(v, -kQuantMax), kQuantMax));
}

// four values quantised, as int32 bit patterns in float lanes
__device__ __forceinline__ float4 quantize4(float4 a, int shift) {
  return make_float4(__int_as_float(quantize(a.x, shift)), __int_as_float(quantize(a.y, shift)),
                     __int_as_float(quantize(a.z, shift)), __int_as_float(quantize(a.w, shift)));
}

// Sum over the 64 lanes of a wave by xor butterfly: every lane ends with the
// same value (each step adds the same two operands on both sides).
__device__ __forceinline__ float wave_sum(float v) {
  for (int off = 1; off < 64; off <<= 1) v += __shfl_xor(v, off);
  return v;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF,
                                                    0xF, false));
}
constexpr int kDppXor1 = 0xB1;  // quad_perm 1,0,3,2
constexpr int kDppXor2 = 0x4E;  // quad_perm 2,3,0,1

// Sum of the wave's values by DPP within each row of 16 lanes, then the four
// row sums read out (wave-uniform). Any wave given the same values returns the
// same sum: the order of additions is fixed.
__device__ __forceinline__ float wave_sum_rows(float v) {
  v += dpp_f32<kDppXor1>(v);
  v += dpp_f32<kDppXor2>(v);
  v += dpp_f32<0x141>(v);  // row_half_mirror: lanes 0-3 meet lanes 4-7
  v += dpp_f32<0x140>(v);  // row_mirror: lanes 0-7 meet lanes 8-15
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

typedef __attribute__((address_space(3))) int32_t lds_i32;

// Integer add into LDS at an absolute byte address. The bins sit at LDS
// address 0 (the kernels have no static LDS), so a bin's address is known
// to the compiler bit for bit and needs no base addition.
__device__ __forceinline__ void lds_add(uint32_t byte_addr, int32_t v) {
  __hip_atomic_fetch_add(reinterpret_cast<lds_i32*>(static_cast<size_t>(byte_addr)), v,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Sum the split-k bins in split order (one thread per bin), then apply the B
// codebook. grid: (n tiles * kFinishParts, M, instances); each block owns
// kTileGroups / kFinishParts groups of one tile in one row (blockIdx.y). A
// thread sums one bin over the splits in split order, with the loads of four
// splits issued before their adds: more blocks and loads in flight than one
// block per group range walking every row, and the same sums bit for bit.
constexpr uint32_t kFinishParts = 16;
constexpr uint32_t kFinishGroups = kTileGroups / kFinishParts;  // 16 groups, 256 bins
static_assert(kFinishGroups * 16 == 256, "one bin per thread of a 256-thread block");

template <int G, int M>
__global__ __launch_bounds__(256) void k_gemv_finish(Operands o, uint32_t n, uint32_t splits,
                                                          uint32_t tiles, const float* partial) {
  __shared__ float sb_book[16 * G];
  __shared__ float ssum[kFinishGroups * 16];
  const uint32_t tile = blockIdx.x / kFinishParts, part = blockIdx.x % kFinishParts;
  const uint32_t r = blockIdx.y;
  const uint32_t row_words = n / (8 * G);
  const uint32_t groups = (row_words - tile * kTileWords) < kTileWords
                              ? (row_words - tile * kTileWords) * 8
                              : kTileGroups;
  const uint32_t j0 = part * kFinishGroups;
  if (j0 >= groups || r >= uint32_t(M)) return;
  const uint32_t jn = (groups - j0) < kFinishGroups ? (groups - j0) : kFinishGroups;
  constexpr uint64_t kSplitStride = uint64_t(M) * 16 * kTileGroups;
  for (uint32_t item = blockIdx.z; item < o.count; item += gridDim.z) {
    const float* b_book = item_ptr<float>(o.in[3], o.stride[3], item);
    float* out = item_ptr_mut<float>(o.out, o.stride[4], item);
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < 16 * G; i += blockDim.x) sb_book[i] = b_book[i];
    const float* base = partial + (uint64_t(item) * tiles + tile) * splits * kSplitStride;
    const uint32_t je = threadIdx.x;
    if (je < jn * 16) {
      const float* p = base + r * 16 * kTileGroups + j0 * 16 + je;
      float s = 0.0f;
      uint32_t sp = 0;
      for (; sp + 4 <= splits; sp += 4) {
        const float v0 = p[uint64_t(sp) * kSplitStride];
        const float v1 = p[uint64_t(sp + 1) * kSplitStride];
        const float v2 = p[uint64_t(sp + 2) * kSplitStride];
        const float v3 = p[uint64_t(sp + 3) * kSplitStride];
        s += v0;
        s += v1;
        s += v2;
        s += v3;
      }
      for (; sp < splits; ++sp) s += p[uint64_t(sp) * kSplitStride];
      ssum[je] = s;
    }
    __syncthreads();
    bool bad = false;
    for (uint32_t jt = threadIdx.x; jt < jn * G; jt += blockDim.x) {
      const uint32_t j = jt / G, t = jt % G;
      float y = 0.0f;
#pragma unroll
      for (int c = 0; c < 16; ++c) y = fmaf(sb_book[c * G + t], ssum[j * 16 + c], y);
      out[uint64_t(r) * n + (tile * kTileGroups + j0) * G + jt] = y;
      bad |= !finite_f32(y);
    }
    if (__any(bad) && (threadIdx.x % warpSize) == 0) atomicOr(o.status, 1u);
  }
}

// ---- GemvPairs (m = 1) -----------------------------------------------------
// The two nibbles of a byte of a B row are the codes of two output groups of
// the same inner row, so they receive the same x. One integer atomic into a
// 256-way "pair bin" indexed by the whole byte replaces the two nibble bins:
//   S[2p][e]   = sum over hi of P[p][16 hi + e]   (low nibble = group 8q+2p)
//   S[2p+1][e] = sum over lo of P[p][16 e + lo]   (high nibble = group 8q+2p+1)
//
// Bin of byte value v at byte position p of word column q (32-word tile):
//   dword (p >> 1) * 16384 + v * 64 + (p & 1) * 32 + (q ^ p)
// and the byte address is a single v_perm of the code word with a per-lane
// constant (byte 0 = 4 (q ^ p), +128 for odd p; byte 2 = the region p >> 1)
// that takes the code byte as byte 1. A half-wave hits 32 distinct banks: one
// row of 32 word columns at one byte position, or (16-byte loads) 8 word
// columns of 4 rows whose lanes take the 4 byte positions at each step, the
// column swizzle q ^ p keeping them apart.
//
// Pipeline: each lane owns R rows of its word column per batch; D register
// buffers form a ring (the loop is unrolled by D, so no in-flight register is
// ever copied and the compiler never waits for more than the batch it bins).
// The last D batches of an instance refill with the next instance's first D,
// and an instance's set-up data (A words of the slice, one entry of each
// book) is requested one instance ahead, so loads stay in flight across set-up
// and finalisation. x is staged per row as int32 in LDS; the next batch's x is
// read before the current batch's atomics (LDS ops complete in order, so a
// read issued after them would wait for them).
//
// Windows are kPairWindow rows, the same rows one staging of x covers: the
// staging takes the window's L1 norm and every read of x quantises it with
// the window's scale (window_scale), so no sum of the window can leave int32.
//
// Finalisation: each thread flushes one 8 x 8 (or SH x SL) sub-block of the
// 16 x 16 pair-bin matrix of one (p, q), conflict-free (lanes are word
// columns); row and column sums are taken in registers and only those
// partials go through LDS.
constexpr int kPairThreads = 512;
constexpr int kPairWaves = kPairThreads / 64;
constexpr int kPairR = 16;                                          // rows per lane per batch
constexpr int kPairD = 4;                                           // batches in the ring
constexpr uint32_t kPairBatchRows = kPairWaves * 2 * kPairR;        // 256 rows per batch
constexpr uint32_t kPairBins = 256 * 4 * kTileWords;                // 32768
constexpr uint32_t kPairXRows = 4096;                               // staged x rows (16 KiB)
constexpr uint32_t kPairWindow = 4096;
constexpr uint32_t kPairMaxAWords = 2 * kPairThreads;               // A words of one slice
constexpr int kPairHB = 2, kPairLB = 2;                             // sub-blocks per (p, q)
constexpr int kPairSH = 16 / kPairHB, kPairSL = 16 / kPairLB;
static_assert(kPairWindow % kPairBatchRows == 0 && kPairXRows % kPairBatchRows == 0, "batches");
static_assert(kPairSH * kPairSL * kPairThreads == int(kPairBins), "every bin flushed once");
static_assert(kPairThreads / kTileWords == 4 * kPairHB * kPairLB, "thread roles");
static_assert(kPairXRows >= 16 * kTileGroups, "S reuses the x staging area");

// Cumulative finalise (one window per instance, g <= 16): the bins are never
// cleared between instances. Each thread keeps the int32 row and column sums
// its sub-block had at the previous instance's end, and this instance's sums
// are the differences, exact modulo 2^32 (every window sum is below 2^31 in
// magnitude). The partials then live past the bins, in the x staging area and
// the words after it: two halves of the even-nibble sums, then the complete
// odd-nibble sums (the two row halves meet inside the wave), all int32.
constexpr uint32_t kCumHalfWords = 4 * 16 * kTileWords;            // [p][e][q ^ swizzle]
constexpr uint32_t kCumHiBase = 2 * kCumHalfWords + 4;             // bank bit 2 off the halves
constexpr uint32_t kCumWords = kCumHiBase + kCumHalfWords + 12;    // 6,160 (16-byte multiple)
static_assert(kCumWords >= kPairXRows && kCumWords % 4 == 0, "the x staging area grows");
__device__ __forceinline__ uint32_t cum_part(uint32_t p, uint32_t e, uint32_t q) {
  return (p * 16 + e) * kTileWords + (q ^ (2 * (e & 3u) + 8 * p));
}

// LDS layout (bytes): bins | staged x (later S) | A book | B book x 2 | A words | wave L1 sums.
// The B book alternates between two copies by instance, so an instance's
// set-up need not wait for the previous output phase, the book's only reader.
template <int G>
struct PairLds {
  static constexpr bool cum = G <= 16;  // room for the cumulative partials
  static constexpr uint32_t xs = kPairBins * 4;
  static constexpr uint32_t af = xs + (cum ? kCumWords : kPairXRows) * 4;
  static constexpr uint32_t bb = af + 17 * G * 4;  // PK: a 17th (zero) row of A's table
  static constexpr uint32_t aw = bb + 2 * 16 * G * 4;
  static constexpr uint32_t wl1 = aw + kPairMaxAWords * 4;
  static constexpr uint32_t total = wl1 + 16 * 4;
};

__device__ __forceinline__ uint32_t pair_dword(uint32_t v, uint32_t p, uint32_t q) {
  return (p >> 1) * 16384 + v * 64 + (p & 1) * 32 + (q ^ p);
}

// v_perm constant and selector that turn byte p of a code word into the byte
// address of its bin in word column q (pair_dword times 4)
__device__ __forceinline__ uint32_t pair_const(uint32_t p, uint32_t q) {
  return (4 * (q ^ p) + 128 * (p & 1)) | ((p >> 1) << 16);
}
__device__ __forceinline__ uint32_t pair_sel(uint32_t p) { return 0x0c020400u + (p << 8); }

// Finalise partials pl/ph: [half][p][e][q ^ (2 (e & 3) + 8 p)]. The writes
// (lanes = word columns q) and the product's reads (a wave's 16 groups x 4
// codes: q's low bit, p and e & 3 vary) each spread over all 32 banks.
constexpr uint32_t kPairPartWords = (kPairHB + kPairLB) * 4 * 16 * kTileWords;  // pl, ph: 8192
constexpr uint32_t kPairTiles16 = kTileGroups / 16;               // 16-group product tiles
static_assert(kPairHB == 2 && kPairLB == 2, "the product sums two partials per S entry");
static_assert(kPairPartWords % (4 * kPairThreads) == 0 && kPairPartWords <= kPairBins, "pl/ph clears");
__device__ __forceinline__ uint32_t pair_part(uint32_t half, uint32_t p, uint32_t e, uint32_t q) {
  return ((half * 4 + p) * 16 + e) * kTileWords + (q ^ (2 * (e & 3u) + 8 * p));
}

// Largest of the wave's values, for values that are >= 0 and not NaN (their
// bit patterns then order as the floats do): DPP within each row of 16, then
// the four row results.
__device__ __forceinline__ float wave_max_nonneg(float m) {
  int v = __float_as_int(m);
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false));  // row_half_mirror
  v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false));  // row_mirror
  const int r = max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
                    max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
  return __int_as_float(r);
}

// Cache policy of the loads that stream B's codes: non-temporal (the `nt`
// bit), since every code word is read once. It measured ~7 % faster on the
// config-3 GEMV than the default policy.
constexpr int kStreamLoad = 2;

// Buffer descriptor over the first `bytes` of an array: raw buffer loads past
// it return zero, which is how rows past a slice (or a missing instance) read.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t words_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}

struct PairAhead {
  uint32_t w0, w1;  // A words tid and tid + kPairThreads of the slice (PK: w0 = word `lane`)
  float a, b;       // entry tid of the A and B books
  float4 a4;        // PK: A book values 4 lane .. 4 lane + 3
};

// grid: (n tiles, k splits, z); block z serves instances z, z + gridDim.z, ...
// ks is a multiple of kPairBatchRows. AD: x is dense FP32 in in[0] (in[1] is
// not read); a nonfinite x sets status bit 1.
// SW: the slice is one window (ks <= kPairWindow), so the bins are read out
// once, at the end, and no FP32 accumulator lives through the main loop.
// X4 (rows of whole 32-word tiles): each lane loads 4 adjacent words of 4 rows
// with 16-byte loads, a quarter of the load instructions. Eight lanes cover a
// row, so the 32 lanes of a half-wave hold 4 rows; a lane rotates its 4 words
// by its row slot so that at every atomic the half-wave still covers the 32
// word columns once (32 distinct banks).
//
// PK (packed x, one window, cumulative bins: the batched decode shape): x is
// never staged. A wave's 32 rows of a batch lie in one A word, so each lane
// keeps one A word of the slice in a register (lane l: word l) and read_x
// decodes its rows from that word (v_readlane) and the A book in LDS. The A
// book alternates between two LDS copies by instance and the next instance's
// copy is written one instance ahead, so an instance's set-up writes LDS only
// where no wave can still be reading. The window's L1 norm is a code
// histogram against the book's row norms, which every wave forms alike from
// registers (so all waves hold the same scale without exchanging it). An
// instance then has two barriers: before the flush and before the product.
//
// Row instances (mrows > 1: "gemv-row-pairs", 2 <= m <= 8 with A row-major):
// each row of A is an instance of its own, instance i = (item i / mrows, row
// i % mrows), binning that row against the item's B. A block's instance
// sequence starts at an XCD-aware position, so the mrows instances of one item
// run at the same time on blocks of one XCD and read B's codes through its L2
// once from HBM. The caller guarantees one k slice (no split).
template <int G, bool AD, bool SW, bool X4>
__global__ __launch_bounds__(kPairThreads, 2) void k_gemv_pairs(Operands o, uint32_t n,
                                                                uint32_t k, uint32_t ks,
                                                                float* partial, uint32_t mrows) {
  constexpr uint32_t R = kPairR, D = kPairD, BR = kPairBatchRows;
  constexpr int kSPer = 16 * kTileGroups / kPairThreads;
  static_assert(16 * G <= kPairThreads, "one book entry per thread");
  static_assert(D % 2 == 0, "x buffers alternate by batch parity");
  using L = PairLds<G>;
  constexpr bool PK = SW && !AD && L::cum;
  // PK: one A word per lane covers a window (kPairWindow rows), one float4 per
  // lane covers the A book, and the A book's second copy fits the words' area
  static_assert(!PK || (kPairWindow / (8 * G) <= 64 && 16 * G <= 4 * 64 &&
                        17 * G <= kPairMaxAWords), "PK registers and LDS");
  extern __shared__ int32_t smem[];
  char* lds = reinterpret_cast<char*>(smem);
  int32_t* bins = smem;
  int4* bins4 = reinterpret_cast<int4*>(smem);
  float* sx = reinterpret_cast<float*>(lds + L::xs);    // the window's x, FP32
  float* af = reinterpret_cast<float*>(lds + L::af);
  float* const bb0 = reinterpret_cast<float*>(lds + L::bb);
  uint32_t* aw = reinterpret_cast<uint32_t*>(lds + L::aw);
  float* wl1 = reinterpret_cast<float*>(lds + L::wl1);  // per-wave L1 of the staged x
  float* const afx = reinterpret_cast<float*>(lds + L::aw);  // PK: the A book's second copy
  // Defensive: the perm-built bin addresses assume the bins start at LDS 0.
  if (static_cast<uint32_t>(reinterpret_cast<size_t>((lds_i32*)smem)) != 0) {
    if (threadIdx.x == 0) atomicOr(o.status, 2u);
    return;
  }
  const uint32_t tid = threadIdx.x;
  const uint32_t tile = blockIdx.x, split = blockIdx.y, zn = gridDim.z;
  const uint32_t rw = n / (8 * G);
  const uint32_t k0 = split * ks;
  const uint32_t kend = (k0 + ks) < k ? (k0 + ks) : k;
  const uint32_t nb = (kend - k0 + BR - 1) / BR;
  const uint32_t nbp = (nb + D - 1) / D * D;  // padded batches read zero words and x
  const uint32_t lane = tid % 64, wave = tid / 64;
  const uint32_t q = lane % 32, half = lane / 32;
  // X4: lane = 8 row slots x 8 four-word chunks; rx rows per lane per batch
  constexpr uint32_t RX = X4 ? R / 4 : R;
  const uint32_t chunk = lane % 8, slot = lane / 8;
  const uint32_t lane_row = X4 ? wave * (2 * R) + slot * RX : (wave * 2 + half) * R;
  // dead word columns (rw not a multiple of the tile) bin the last column into
  // bins no output reads
  const uint32_t col = X4 ? tile * kTileWords + 4 * chunk
                          : ((tile * kTileWords + q < rw) ? tile * kTileWords + q : rw - 1);
  // bin address constants (pair_const): X4, step s of word t bins byte
  // (s + slot) % 4 of word column 4 chunk + t, so the four row slots of a
  // half-wave take the four byte positions; otherwise step p bins byte p of
  // column q
  uint32_t bc[X4 ? 4 : 1][4], bsel[4];
#pragma unroll
  for (uint32_t st = 0; st < 4; ++st) {
    const uint32_t ps = X4 ? (st + slot) & 3u : st;
    bsel[st] = pair_sel(ps);
#pragma unroll
    for (uint32_t t = 0; t < (X4 ? 4u : 1u); ++t) bc[t][st] = pair_const(ps, X4 ? 4 * chunk + t : q);
  }
  const uint32_t a_w0 = k0 / G / 8;
  const uint32_t a_words = (kend - 1) / G / 8 - a_w0 + 1;

  // Opaque copies of the thread index keep per-phase addresses from being
  // hoisted out of the instance loop and held live through the main loop.
  auto opaque = [](uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
  };
  // instance i: item i / mrows, row i % mrows of A (one instance per item when mrows = 1)
  const uint32_t ninst = o.count * mrows;
  auto src_item = [&](uint32_t i) { return mrows == 1 ? i : i / mrows; };
  auto src_row = [&](uint32_t i) { return mrows == 1 ? 0u : i % mrows; };
  // A's row of instance i: packed rows start on whole words (k a multiple of 8 G)
  auto a_row_words = [&](uint32_t i) {
    return item_ptr<uint32_t>(o.in[0], o.stride[0], src_item(i)) + src_row(i) * (k / (8 * G));
  };
  auto x_row = [&](uint32_t i) {
    return item_ptr<float>(o.in[0], o.stride[0], src_item(i)) + uint64_t(src_row(i)) * k;
  };
  auto out_row = [&](uint32_t i) {
    return item_ptr_mut<float>(o.out, o.stride[4], src_item(i)) + uint64_t(src_row(i)) * n +
           tile * kTileGroups * G;
  };
  auto setup_loads = [&](uint32_t item) {
    const uint32_t lt = opaque(tid);
    const __amdgpu_buffer_rsrc_t ars = words_rsrc(a_row_words(item) + a_w0, a_words * 4u);
    const __amdgpu_buffer_rsrc_t abk = words_rsrc(
        AD ? nullptr : item_ptr<float>(o.in[1], o.stride[1], src_item(item)), AD ? 0u : 64u * G);
    const __amdgpu_buffer_rsrc_t bbk =
        words_rsrc(item_ptr<float>(o.in[3], o.stride[3], src_item(item)), 64u * G);
    PairAhead h;
    h.b = __uint_as_float(uint32_t(__builtin_amdgcn_raw_buffer_load_b32(bbk, lt * 4u, 0, 0)));
    h.w0 = h.w1 = 0;
    h.a = 0.0f;
    h.a4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (PK) {  // words and book values past the slice and the book read as zero
      const uint32_t ll = lt % 64;
      const auto v = __builtin_amdgcn_raw_buffer_load_b128(abk, ll * 16u, 0, 0);
      h.a4 = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                         __uint_as_float(v[3]));
      h.w0 = uint32_t(__builtin_amdgcn_raw_buffer_load_b32(ars, ll * 4u, 0, 0));
    } else if (!AD) {
      h.a = __uint_as_float(uint32_t(__builtin_amdgcn_raw_buffer_load_b32(abk, lt * 4u, 0, 0)));
      h.w0 = uint32_t(__builtin_amdgcn_raw_buffer_load_b32(ars, lt * 4u, 0, 0));
      h.w1 = uint32_t(__builtin_amdgcn_raw_buffer_load_b32(ars, (lt + kPairThreads) * 4u, 0, 0));
    }
    return h;
  };
  auto batch_rsrc = [&](uint32_t item) {
    const bool real = item < ninst;
    return words_rsrc(item_ptr<uint32_t>(o.in[2], o.stride[2], real ? src_item(item) : 0),
                      real ? kend * rw * 4u : 0u);
  };
  const uint32_t voff_lane = (lane_row * rw + col) * 4u;
  auto load_batch = [&](__amdgpu_buffer_rsrc_t rs, uint32_t b, uint32_t (&w)[R]) {
    uint32_t off = voff_lane + (k0 + b * BR) * rw * 4u;
    asm volatile("" : "+v"(off));  // per-row offsets formed next to each load
    if (X4) {
#pragma unroll
      for (uint32_t u = 0; u < RX; ++u) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, off + u * rw * 4u, 0, kStreamLoad);
        w[4 * u] = v[0]; w[4 * u + 1] = v[1]; w[4 * u + 2] = v[2]; w[4 * u + 3] = v[3];
      }
    } else {
#pragma unroll
      for (uint32_t u = 0; u < R; ++u)
        w[u] = uint32_t(__builtin_amdgcn_raw_buffer_load_b32(rs, off + u * rw * 4u, 0, kStreamLoad));
    }
  };

  uint32_t buf[D][R];
  float xa[RX], xb[RX];  // x of the lane's next rows as staged; quantised where binned
  // multi-window: the sub-block's FP32 accumulators; one window: its row and
  // column sums, formed as the bins are read (the same sums in the same order)
  float acc[SW ? 1 : kPairSH][SW ? 1 : kPairSL];
  float rsum[kPairSH], csum[kPairSL];
  // cumulative bins: this flush's int32 row and column sums, and the
  // previous instance's (rows 0..7, columns 8..15)
  constexpr bool CUM = SW && L::cum;
  uint32_t rsi[CUM ? kPairSH : 1], csi[CUM ? kPairSL : 1], prv[CUM ? 16 : 1];
#pragma unroll
  for (int i = 0; i < (CUM ? 16 : 1); ++i) prv[i] = 0;
  int shift = 0;  // the current window's fixed-point scale
  uint32_t xbase = k0;
  // PK: this instance's copy of the A book, and the lane's A word of the slice
  const float* af_cur = af;
  uint32_t wreg = 0;
  PairAhead cur{}, nxt{};  // set-up data of this instance and the next
  static_assert(!PK || (8 * G) % (2 * R) == 0, "a wave's rows of a batch lie in one A word");
  __amdgpu_buffer_rsrc_t x_rs = words_rsrc(nullptr, 0u);  // AD: this instance's x[0, kend)

  // Rows [xb0, xb0 + kPairXRows) of A's single row as FP32, zero past kend,
  // and each wave's share of their L1 norm in wl1. The caller's barrier
  // publishes both; take_scale() then sets the window's scale.
  auto stage_x = [&](uint32_t xb0) __attribute__((always_inline)) {
    float lp = 0.0f, ln = 0.0f;  // the window's positive and negative masses
    bool bad = false;
    for (uint32_t r4 = opaque(tid) * 4; r4 < kPairXRows; r4 += 4 * kPairThreads) {
      const uint32_t row = xb0 + r4;
      float4 f = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (AD) {
        auto ld = [&](uint32_t rr) {  // reads past kend return zero
          return __uint_as_float(uint32_t(__builtin_amdgcn_raw_buffer_load_b32(x_rs, rr * 4u, 0, 0)));
        };
        f = make_float4(ld(row), ld(row + 1), ld(row + 2), ld(row + 3));
        bad |= !finite_f32(f.x) || !finite_f32(f.y) || !finite_f32(f.z) || !finite_f32(f.w);
      } else if (row < kend) {
        const uint32_t u = row / G;
        const uint32_t code = (aw[(u >> 3) - a_w0] >> ((u & 7u) * 4u)) & 15u;
        f = *reinterpret_cast<const float4*>(af + code * G + row % G);
        if (row + 1 >= kend) f.y = 0.0f;
        if (row + 2 >= kend) f.z = 0.0f;
        if (row + 3 >= kend) f.w = 0.0f;
      }
      lp += fmaxf(f.x, 0.0f);
      ln += fmaxf(-f.x, 0.0f);
      lp += fmaxf(f.y, 0.0f);
      ln += fmaxf(-f.y, 0.0f);
      lp += fmaxf(f.z, 0.0f);
      ln += fmaxf(-f.z, 0.0f);
      lp += fmaxf(f.w, 0.0f);
      ln += fmaxf(-f.w, 0.0f);
      *reinterpret_cast<float4*>(sx + r4) = f;
    }
    lp = wave_sum(lp);
    ln = wave_sum(ln);
    if (lane == 0) {
      wl1[wave] = lp;
      wl1[kPairWaves + wave] = ln;
    }
    if (AD && tile == 0 && __any(bad) && lane == 0) atomicOr(o.status, 1u);
  };
  auto take_scale = [&]() __attribute__((always_inline)) {
    float lp = 0.0f, ln = 0.0f;
#pragma unroll
    for (int w = 0; w < kPairWaves; ++w) {
      lp += wl1[w];
      ln += wl1[kPairWaves + w];
    }
    // NaN when either mass is NaN or infinite (status bit 1 follows)
    const float l1 = fmaxf(lp, ln) + (lp - lp) + (ln - ln);
    shift = window_shift(l1);
    // finite values whose L1 overflows FP32: no scale holds the window
    if (!(l1 <= FLT_MAX) && tid == 0) atomicOr(o.status, 1u);
  };
  auto read_x = [&](uint32_t b, float (&xs)[RX]) __attribute__((always_inline)) {
    asm volatile("" : "+s"(b));
    // a padding batch: nothing staged for it (PK reads the table's zero row,
    // so that no branch separates the read from its use)
    if (!PK && k0 + b * BR >= kend) {
#pragma unroll
      for (uint32_t u = 0; u < RX; ++u) xs[u] = 0.0f;
      return;
    }
    if (PK) {
      // the wave's 2 R rows of the batch (slice rows b BR + 2 R wave ..) lie in
      // word (b BR + 2 R wave) / (8 G) of the slice, held by that lane; the
      // table holds x quantised (int32 bits), rows past the slice read row 16
      // (zeros: the slice length is a multiple of 4). Nothing uses the read
      // until the next batch, after this batch's atomics: a use right after
      // it would wait for the wave's previous atomics, which LDS completes
      // first.
      const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
      const uint32_t word =
          uint32_t(__builtin_amdgcn_readlane(int(wreg), int((b * BR + 2 * R * wv) / (8 * G))));
#pragma unroll
      for (uint32_t c4 = 0; c4 < RX / 4; ++c4) {
        const uint32_t row = b * BR + lane_row + 4 * c4;  // of the slice
        const uint32_t code = row < kend - k0 ? (word >> (((row / G) % 8u) * 4u)) & 15u : 16u;
        const float4 v = *reinterpret_cast<const float4*>(af_cur + code * G + row % G);
        xs[4 * c4] = v.x;
        xs[4 * c4 + 1] = v.y;
        xs[4 * c4 + 2] = v.z;
        xs[4 * c4 + 3] = v.w;
      }
      return;
    }
    const float4* xr = reinterpret_cast<const float4*>(sx + (k0 + b * BR + lane_row - xbase));
#pragma unroll
    for (uint32_t c4 = 0; c4 < RX / 4; ++c4) {
      const float4 v = xr[c4];
      xs[4 * c4] = v.x; xs[4 * c4 + 1] = v.y; xs[4 * c4 + 2] = v.z; xs[4 * c4 + 3] = v.w;
    }
  };
  // PK: the window's scale from an instance's set-up registers. The book's row
  // norms (entry e = its G / 4 lanes' sums) meet the slice's codes (lane l:
  // word l); every lane of every wave forms the same sums in the same order.
  auto pk_shift = [&](const PairAhead& h) __attribute__((always_inline)) {
    // entry e's positive and negative masses over its G / 4 lanes (aligned, 2 or 4)
    float pp = fmaxf(h.a4.x, 0.0f), pn = fmaxf(-h.a4.x, 0.0f);
    pp += fmaxf(h.a4.y, 0.0f);
    pn += fmaxf(-h.a4.y, 0.0f);
    pp += fmaxf(h.a4.z, 0.0f);
    pn += fmaxf(-h.a4.z, 0.0f);
    pp += fmaxf(h.a4.w, 0.0f);
    pn += fmaxf(-h.a4.w, 0.0f);
    pp += dpp_f32<kDppXor1>(pp);
    pn += dpp_f32<kDppXor1>(pn);
    if (G / 4 == 4) {
      pp += dpp_f32<kDppXor2>(pp);
      pn += dpp_f32<kDppXor2>(pn);
    }
    const uint32_t groups = (kend - k0 + G - 1) / G;
    float lp = 0.0f, ln = 0.0f;
#pragma unroll
    for (uint32_t c = 0; c < 8; ++c) {
      const uint32_t code = (h.w0 >> (4 * c)) & 15u;
      const float rp = __shfl(pp, int(code * (G / 4)));
      const float rn = __shfl(pn, int(code * (G / 4)));
      if (lane * 8 + c < groups) {
        lp += rp;
        ln += rn;
      }
    }
    const float l1 = fmaxf(wave_sum_rows(lp), wave_sum_rows(ln));
    if (!(l1 <= FLT_MAX) && tid == 0) atomicOr(o.status, 1u);  // book rows whose L1 overflows
    return __builtin_amdgcn_readfirstlane(window_shift(l1));
  };
  static_assert(!PK || G == 8 || G == 16, "book row norms over 2 or 4 lanes");
  // CUM at G = 16 with one k slice: y^T = C_B^T . S^T on v_mfma_f32_16x16x4f32,
  // S read from an instance's cumulative partials, 16 groups per product tile
  // and 4 codes per step. Lane l: A = C_B[4 ks + l/16][l % 16], B = S of group
  // 16 tile + l % 16 at code 4 ks + l/16; it ends with y[16 tile + l % 16]
  // [4 (l/16) .. 4 (l/16) + 3]. A wave reads both its tiles' partials before
  // its first product.
  //
  // Kept outputs: a global store counts in the same in-order counter as the
  // code loads, so a wait for any load issued after it also waits for the
  // store's acknowledgement, which queues behind every read in flight (tens
  // of MiB, microseconds). A deferred product therefore keeps its outputs in
  // registers until the next instance's last batch has refilled, and stores
  // them there: the first load issued after them is waited for four batches
  // and a finalisation later, when they have long been acknowledged.
  constexpr uint32_t TT = kPairTiles16 / kPairWaves;
  static_assert(kPairTiles16 % kPairWaves == 0, "whole tiles per wave");
  float4 kept[TT];
  uint32_t kept_item = 0;
  bool has_kept = false;
  const uint32_t groups_tile = (rw - tile * kTileWords) < kTileWords ? (rw - tile * kTileWords) * 8
                                                                     : kTileGroups;
  auto store_out = [&](uint32_t pitem, const float4 (&y)[TT]) __attribute__((always_inline)) {
    const uint32_t ft = opaque(tid);
    const uint32_t lane16 = ft % 16, k4 = (ft % 64) / 16;
    float* out = out_row(pitem);
    const bool vec = (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
#pragma unroll
    for (uint32_t tt = 0; tt < TT; ++tt) {
      const uint32_t j = (ft / 64 + tt * kPairWaves) * 16 + lane16;
      if (j < groups_tile) {
        float* oy = out + j * 16 + 4 * k4;
        if (vec) {
          *reinterpret_cast<float4*>(oy) = y[tt];
        } else {
          oy[0] = y[tt].x; oy[1] = y[tt].y; oy[2] = y[tt].z; oy[3] = y[tt].w;
        }
      }
    }
  };
  auto mfma_product = [&](uint32_t pitem, int pshift, const float* pbb, bool keep)
                          __attribute__((always_inline)) {
    const uint32_t ft = opaque(tid);
    const uint32_t* cpt = reinterpret_cast<const uint32_t*>(sx);
    const uint32_t lane16 = ft % 16, k4 = (ft % 64) / 16;
    const uint32_t groups = groups_tile;
    float bk[4];
#pragma unroll
    for (uint32_t ks = 0; ks < 4; ++ks) bk[ks] = pbb[(4 * ks + k4) * 16 + lane16];
    float sb[TT][4];
#pragma unroll
    for (uint32_t tt = 0; tt < TT; ++tt) {
      const uint32_t j = (ft / 64 + tt * kPairWaves) * 16 + lane16;
      const uint32_t qq = j / 8, n8 = j % 8;
      const bool odd = (n8 & 1u) != 0;
#pragma unroll
      for (uint32_t ks = 0; ks < 4; ++ks) {
        const uint32_t at = cum_part(n8 / 2, 4 * ks + k4, qq);
        const uint32_t v0 = cpt[(odd ? kCumHiBase : 0u) + at];
        const uint32_t v1 = cpt[kCumHalfWords + at];  // odd nibbles: read, unused
        sb[tt][ks] = unscale(float(int32_t(odd ? v0 : v0 + v1)), pshift);
      }
    }
    bool bad = false;
    float4 y[TT];
#pragma unroll
    for (uint32_t tt = 0; tt < TT; ++tt) {
      const uint32_t j = (ft / 64 + tt * kPairWaves) * 16 + lane16;
      typedef float float4v __attribute__((ext_vector_type(4)));
      float4v d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (uint32_t ks = 0; ks < 4; ++ks) d = __builtin_amdgcn_mfma_f32_16x16x4f32(bk[ks], sb[tt][ks], d, 0, 0, 0);
      y[tt] = make_float4(d[0], d[1], d[2], d[3]);
      if (j < groups)
        bad |= !finite_f32(d[0]) || !finite_f32(d[1]) || !finite_f32(d[2]) || !finite_f32(d[3]);
    }
    if (__any(bad) && (ft % warpSize) == 0) atomicOr(o.status, 1u);
    if (!keep || has_kept) {  // (a kept instance is stored before the next product)
      store_out(pitem, y);
      return;
    }
    kept_item = pitem;
#pragma unroll
    for (uint32_t tt = 0; tt < TT; ++tt) kept[tt] = y[tt];
    has_kept = true;
  };
  // PK at G = 16 with one k slice: an instance's product waits until the next
  // instance's first refill is in flight (its partials and B book copy stay
  // untouched until the next flush barrier)
  const bool defer = PK && G == 16 && gridDim.y == 1;
  bool pending = false;
  uint32_t p_item = 0;
  int p_shift = 0;
  const float* p_bb = bb0;
  // this thread's sub-block: word column fq, byte position fp, sub-block (fh, fl)
  auto flush = [&](bool clear) __attribute__((always_inline)) {
    const uint32_t ft = opaque(tid);
    if (CUM) {
      // half-wave = column half fl, wave = (fp, fh): the two column halves of
      // a row half are lanes l and l + 32 of one wave
      const uint32_t cq = ft % kTileWords, cl = (ft / kTileWords) % 2, cw = ft / 64;
      const uint32_t cp = cw % 4, ch = cw / 4;
#pragma unroll
      for (int a = 0; a < kPairSH; ++a)
#pragma unroll
        for (int c = 0; c < kPairSL; ++c) {
          const uint32_t v = uint32_t(bins[pair_dword(16 * (ch * kPairSH + a) + cl * kPairSL + c, cp, cq)]);
          csi[c] = a == 0 ? v : csi[c] + v;
          rsi[a] = c == 0 ? v : rsi[a] + v;
        }
      return;
    }
    const uint32_t fq = ft % kTileWords, fc = ft / kTileWords;
    const uint32_t fp = fc % 4, fs = fc / 4;
    const uint32_t fh = fs % kPairHB, fl = fs / kPairHB;
#pragma unroll
    for (int a = 0; a < kPairSH; ++a)
#pragma unroll
      for (int c = 0; c < kPairSL; ++c) {
        const uint32_t d = pair_dword(16 * (fh * kPairSH + a) + fl * kPairSL + c, fp, fq);
        if (SW) {
          const float v = float(bins[d]);
          csum[c] = a == 0 ? v : csum[c] + v;
          rsum[a] = c == 0 ? v : rsum[a] + v;
        } else {
          acc[a][c] += unscale(float(bins[d]), shift);
          if (clear) bins[d] = 0;
        }
      }
  };
  // `tail`: a batch of the peeled last D, the only ones that can be the last
  // `first`: may be the instance's batch 0, where a deferred product runs
  auto stage = [&](uint32_t (&w)[R], uint32_t b, float (&xs)[RX], float (&xn)[RX],
                   __amdgpu_buffer_rsrc_t rs_refill, uint32_t b_refill, bool tail, bool first)
                   __attribute__((always_inline)) {
    asm volatile("" : "+s"(b));  // row arithmetic is redone per batch, not strength-reduced
    const uint32_t done = (b + 1) * BR;
    const bool last = tail && b + 1 == nbp;
    const bool restage = !SW && k0 + done < kend && k0 + done - xbase >= kPairXRows;
    const bool wend = SW ? last : (done % kPairWindow == 0 || last);
    if (!restage && !last) read_x(b + 1, xn);
    // the lane's row u of batch b as binned: PK reads it quantised (rows past
    // the slice read the table's zero row), else x is quantised here
    auto x_q = [&](uint32_t u) __attribute__((always_inline)) {
      return PK ? __float_as_int(xs[u]) : quantize(xs[u], shift);
    };
    if (PK || b < nb) {  // padding batches (past the slice) bin nothing (PK: zeros)
      if (X4) {
#pragma unroll
        for (uint32_t u = 0; u < RX; ++u) {
          const int32_t xv = x_q(u);
#pragma unroll
          for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int st = 0; st < 4; ++st)
              lds_add(__builtin_amdgcn_perm(w[4 * u + t], bc[t][st], bsel[st]), xv);
        }
      } else {
#pragma unroll
        for (uint32_t u = 0; u < R; ++u) {
          const int32_t xv = x_q(u);
#pragma unroll
          for (int st = 0; st < 4; ++st) lds_add(__builtin_amdgcn_perm(w[u], bc[0][st], bsel[st]), xv);
        }
      }
    }
    load_batch(rs_refill, b_refill, w);
    __builtin_amdgcn_sched_barrier(0);
    if (first && pending) {  // every thread has written the previous instance's partials
      __syncthreads();
      mfma_product(p_item, p_shift, p_bb, true);
      pending = false;
    }
    if (last && has_kept) {
      store_out(kept_item, kept);
      has_kept = false;
    }
    if (wend) {
      __syncthreads();
      flush(!last);
      if (!last && !restage) __syncthreads();
    }
    if (restage) {
      if (!wend) __syncthreads();
      xbase = k0 + done;
      stage_x(xbase);
      __syncthreads();
      take_scale();  // the flush above used the previous window's
      read_x(b + 1, xn);
      // settle here, so at the join the common path's x (read a batch
      // earlier) needs no wait behind this batch's atomics
      __builtin_amdgcn_s_waitcnt(0xc07f);
    }
  };

  // the block's first instance; with row instances, blocks z, z + 8, z + 16, ...
  // (one XCD) take consecutive instances, the rows of one item
  const uint32_t first_inst =
      (mrows > 1 && zn % 8 == 0) ? (blockIdx.z % 8) * (zn / 8) + blockIdx.z / 8 : blockIdx.z;
  uint32_t item = first_inst;
  if (item < ninst) {
    cur = setup_loads(item);
    nxt = setup_loads(item + zn < ninst ? item + zn : item);
    const __amdgpu_buffer_rsrc_t r0 = batch_rsrc(item);
#pragma unroll
    for (uint32_t d = 0; d < D; ++d) load_batch(r0, d, buf[d]);
  }
  // the bins start at zero; each instance clears them again once its finalise
  // has read them (the set-up barriers order that before the next atomics)
#pragma unroll
  for (uint32_t i = 0; i < kPairBins / (4 * kPairThreads); ++i)
    bins4[tid + i * kPairThreads] = make_int4(0, 0, 0, 0);
  // PK: A's book quantised with an instance's scale is that instance's table
  // of x; the tables alternate between two copies by instance, and the next
  // instance's is written one instance ahead, with its scale (nshift)
  int nshift = 0;
  if (PK) {
    if (tid < G) {  // row 16, which rows past the slice read: zeros, never rewritten
      af[16 * G + tid] = 0.0f;
      afx[16 * G + tid] = 0.0f;
    }
    nshift = pk_shift(cur);
    if (4 * tid < 16 * G) *reinterpret_cast<float4*>(af + 4 * tid) = quantize4(cur.a4, nshift);
    __syncthreads();
  }
  for (; item < ninst; item += zn) {
    const uint32_t next = item + zn;
    const __amdgpu_buffer_rsrc_t cur_rs = batch_rsrc(item);
    const __amdgpu_buffer_rsrc_t next_rs = batch_rsrc(next);
    // ---- set-up ----
    // No barrier first: the previous output phase reads only S (staging area)
    // and the other copy of the B book, and its bin clears precede this
    // instance's atomics by the barriers below.
    const uint32_t st = opaque(tid);
    const uint32_t par = ((item - first_inst) / zn) & 1u;
    float* bb = bb0 + par * (16 * G);
    if (PK) {
      // No barrier: the B book copy written here was last read by the product
      // two instances back, and the A book copy written here (the next
      // instance's) by the previous instance's loop; every wave has passed
      // the previous instance's flush barrier, which follows both.
      if (st < 16 * G) bb[st] = cur.b;
      shift = nshift;
      nshift = pk_shift(nxt);
      if (4 * st < 16 * G)
        *reinterpret_cast<float4*>((par ? af : afx) + 4 * st) = quantize4(nxt.a4, nshift);
      if (tile == 0 && split == 0) {  // nonfinite book values, from the set-up registers
        const bool bad = (4 * st < 16 * G && (!finite_f32(cur.a4.x) || !finite_f32(cur.a4.y) ||
                                              !finite_f32(cur.a4.z) || !finite_f32(cur.a4.w))) ||
                         (st < 16 * G && !finite_f32(cur.b));
        if (__any(bad) && lane == 0) atomicOr(o.status, 1u);
      }
      af_cur = par ? afx : af;
      wreg = cur.w0;
      read_x(0, xa);
    } else {
      if (st < 16 * G) {
        if (!AD) af[st] = cur.a;
        bb[st] = cur.b;
      }
      if (!AD && st < a_words) aw[st] = cur.w0;
      if (!AD && st + kPairThreads < a_words) aw[st + kPairThreads] = cur.w1;
      if (AD) x_rs = words_rsrc(x_row(item), kend * 4u);
      __syncthreads();
      // the previous instance's pl/ph (the first kPairPartWords bins) are read
      if (!CUM) {
#pragma unroll
        for (uint32_t i = 0; i < kPairPartWords / (4 * kPairThreads); ++i)
          bins4[st + i * kPairThreads] = make_int4(0, 0, 0, 0);
      }
      if (tile == 0 && split == 0) sweep_books(AD ? bb : af, bb, 16 * G, o.status);
      xbase = k0;
      stage_x(xbase);
      __syncthreads();
      take_scale();
      read_x(0, xa);
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // settle the first x before the loop
    // the next instance's set-up data moves up; the one after is requested now
    cur = nxt;
    nxt = setup_loads(next + zn < ninst ? next + zn : item);
    if (!SW) {
#pragma unroll
      for (int a = 0; a < (SW ? 1 : kPairSH); ++a)
#pragma unroll
        for (int c = 0; c < (SW ? 1 : kPairSL); ++c) acc[a][c] = 0.0f;
    }

    // ---- main loop: all but the last D batches refill from this instance ----
    for (uint32_t b0 = 0; b0 + D < nbp; b0 += D) {
#pragma unroll
      for (uint32_t d = 0; d < D; d += 2) {
        stage(buf[d], b0 + d, xa, xb, cur_rs, b0 + d + D, false, d == 0 && b0 == 0);
        stage(buf[d + 1], b0 + d + 1, xb, xa, cur_rs, b0 + d + 1 + D, false, false);
      }
    }
#pragma unroll
    for (uint32_t d = 0; d < D; d += 2) {
      stage(buf[d], nbp - D + d, xa, xb, next_rs, d, true, d == 0 && nbp == D);
      stage(buf[d + 1], nbp - D + d + 1, xb, xa, next_rs, d + 1, true, false);
    }

    // ---- finalise: sub-block row/column sums, one exchange, S, outputs ----
    const uint32_t ft = opaque(tid);
    const uint32_t fq = ft % kTileWords, fc = ft / kTileWords;
    const uint32_t fp = fc % 4, fs = fc / 4;
    const uint32_t fh = fs % kPairHB, fl = fs / kPairHB;
    float* pl = reinterpret_cast<float*>(smem);           // [HB][4][16 lo][32 q], swizzled
    float* ph = pl + kPairHB * 4 * 16 * kTileWords;       // [LB][4][16 hi][32 q], swizzled
    uint32_t* cpt = reinterpret_cast<uint32_t*>(sx);      // cumulative partials
    if (CUM) {
      // the flush's mapping: column half cl = half-wave, wave = (cp, ch)
      const uint32_t cq = ft % kTileWords, cl = (ft / kTileWords) % 2, cw = ft / 64;
      const uint32_t cp = cw % 4, ch = cw / 4;
#pragma unroll
      for (int i = 0; i < kPairSH; ++i) {
        uint32_t t = rsi[i];
        rsi[i] = t - prv[i];
        prv[i] = t;
        t = csi[i];
        csi[i] = t - prv[8 + i];
        prv[8 + i] = t;
      }
      // even nibbles: this row half's partial of 8 codes
#pragma unroll
      for (int c = 0; c < kPairSL; ++c) cpt[ch * kCumHalfWords + cum_part(cp, cl * 8 + c, cq)] = csi[c];
      // odd nibbles: v_permlane32_swap trades lanes 32..63 of its first operand
      // for lanes 0..31 of its second, so lane l (cl = 0) ends with both halves
      // of row a = i and lane l + 32 (cl = 1) with both of row a = 4 + i
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const auto r = __builtin_amdgcn_permlane32_swap(rsi[i], rsi[4 + i], false, false);
        cpt[kCumHiBase + cum_part(cp, ch * 8 + cl * 4 + i, cq)] = r[0] + r[1];
      }
      if (defer) {
        pending = true;
        p_item = item;
        p_shift = shift;
        p_bb = bb;
        continue;
      }
    } else {
      __syncthreads();  // every thread has flushed its bins
    }
    if (!SW) {
#pragma unroll
      for (int c = 0; c < kPairSL; ++c) {
        float s = 0.0f;
#pragma unroll
        for (int a = 0; a < (SW ? 1 : kPairSH); ++a) s += acc[a][c];
        csum[c] = s;
      }
#pragma unroll
      for (int a = 0; a < kPairSH; ++a) {
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < (SW ? 1 : kPairSL); ++c) s += acc[a][c];
        rsum[a] = s;
      }
    }
    if (!CUM) {
#pragma unroll
      for (int c = 0; c < kPairSL; ++c)
        pl[pair_part(fh, fp, fl * kPairSL + c, fq)] = SW ? unscale(csum[c], shift) : csum[c];
#pragma unroll
      for (int a = 0; a < kPairSH; ++a)
        ph[pair_part(fl, fp, fh * kPairSH + a, fq)] = SW ? unscale(rsum[a], shift) : rsum[a];
    }
    __syncthreads();
    // S entry (p, e, q) of nibble 2 p + odd, from the cumulative partials
    auto cum_s = [&](uint32_t p, uint32_t e, uint32_t qq, bool odd) __attribute__((always_inline)) {
      const uint32_t at = cum_part(p, e, qq);
      const uint32_t v0 = cpt[(odd ? kCumHiBase : 0u) + at];
      const uint32_t v1 = cpt[kCumHalfWords + at];  // odd nibbles: read, unused
      return unscale(float(int32_t(odd ? v0 : v0 + v1)), shift);
    };
    const uint32_t groups = (rw - tile * kTileWords) < kTileWords ? (rw - tile * kTileWords) * 8
                                                                 : kTileGroups;
    float* out = out_row(item);
    if (CUM && G == 16 && gridDim.y == 1) {
      mfma_product(item, shift, bb, false);
    } else if (G == 16 && gridDim.y == 1) {
      // y^T = C_B^T . S^T on v_mfma_f32_16x16x4f32, 16 groups per tile and
      // 4 codes per step; S = the two partials of pl (even nibbles) or ph (odd
      // nibbles), each its own product. Lane l: A = C_B[4 ks + l/16][l % 16],
      // B = partial of group 16 tile + l % 16 at code 4 ks + l/16; it ends with
      // y[16 tile + l % 16][4 (l/16) .. 4 (l/16) + 3].
      const uint32_t lane16 = ft % 16, k4 = (ft % 64) / 16;
      float bk[4];
#pragma unroll
      for (uint32_t ks = 0; ks < 4; ++ks) bk[ks] = bb[(4 * ks + k4) * 16 + lane16];
      bool bad = false;
#pragma unroll
      for (uint32_t tt = 0; tt < kPairTiles16 / kPairWaves; ++tt) {
        const uint32_t tile16 = ft / 64 + tt * kPairWaves;
        if (tile16 * 16 >= groups) break;  // wave-uniform
        const uint32_t j = tile16 * 16 + lane16;
        const uint32_t qq = j / 8, n8 = j % 8;
        const float* part = (n8 & 1u) ? ph : pl;
        typedef float float4v __attribute__((ext_vector_type(4)));
        float4v d = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (uint32_t ks = 0; ks < 4; ++ks)
#pragma unroll
          for (uint32_t h = 0; h < 2; ++h)
            d = __builtin_amdgcn_mfma_f32_16x16x4f32(bk[ks], part[pair_part(h, n8 / 2, 4 * ks + k4, qq)],
                                                     d, 0, 0, 0);
        if (j < groups) {
          float* oy = out + j * 16 + 4 * k4;
          if ((reinterpret_cast<uintptr_t>(out) & 15u) == 0) {
            *reinterpret_cast<float4*>(oy) = make_float4(d[0], d[1], d[2], d[3]);
          } else {
            oy[0] = d[0]; oy[1] = d[1]; oy[2] = d[2]; oy[3] = d[3];
          }
          bad |= !finite_f32(d[0]) || !finite_f32(d[1]) || !finite_f32(d[2]) || !finite_f32(d[3]);
        }
      }
      if (__any(bad) && (ft % warpSize) == 0) atomicOr(o.status, 1u);
    } else {
      float sv[kSPer];
#pragma unroll
      for (int j = 0; j < kSPer; ++j) {
        // S entry (e, nibble n8 = 2 p + kind, word column qq)
        const uint32_t s_ = ft + j * kPairThreads;
        const uint32_t qq = s_ % kTileWords, rest = s_ / kTileWords;
        const uint32_t e = rest % 16, n8 = rest / 16;
        const uint32_t pp_ = n8 / 2;
        float v = 0.0f;
        if (CUM) {
          v = cum_s(pp_, e, qq, (n8 & 1u) != 0);
        } else if ((n8 & 1u) == 0) {
#pragma unroll
          for (int h = 0; h < kPairHB; ++h) v += pl[pair_part(h, pp_, e, qq)];
        } else {
#pragma unroll
          for (int l = 0; l < kPairLB; ++l) v += ph[pair_part(l, pp_, e, qq)];
        }
        sv[j] = v;
      }
      // S as [e][n8][q ^ 4 n8]: the writes (lanes = word columns) and the output
      // reads (a wave's 16 adjacent groups: 8 nibbles x 2 columns) each hit
      // distinct banks
      float* ss = reinterpret_cast<float*>(sx);
      if (gridDim.y == 1) {
        if (CUM) __syncthreads();  // S overwrites the cumulative partials
#pragma unroll
        for (int j = 0; j < kSPer; ++j) {
          const uint32_t s_ = ft + j * kPairThreads;
          const uint32_t qq = s_ % kTileWords, rest = s_ / kTileWords;
          ss[((rest % 16) * 8 + rest / 16) * kTileWords + (qq ^ (4 * (rest / 16)))] = sv[j];
        }
      } else {
        // the finish kernel's [j][e] with j = 8 qq + n8
        float* pp = partial + ((uint64_t(item) * gridDim.x + tile) * gridDim.y + split) *
                                  (16 * kTileGroups);
#pragma unroll
        for (int j = 0; j < kSPer; ++j) {
          const uint32_t s_ = ft + j * kPairThreads;
          const uint32_t qq = s_ % kTileWords, rest = s_ / kTileWords;
          pp[(qq * 8 + rest / 16) * 16 + rest % 16] = sv[j];
        }
      }
      __syncthreads();
      if (gridDim.y == 1) {
        // thread ft always takes columns 4 tc .. 4 tc + 3 (tc = ft % (G / 4)) of
        // its groups: their 16 x 4 book entries stay in registers, and each S
        // value read serves four outputs
        const uint32_t tc = ft % (G / 4);
        float4 cb[16];
#pragma unroll
        for (uint32_t c = 0; c < 16; ++c) cb[c] = *reinterpret_cast<const float4*>(bb + c * G + 4 * tc);
        const bool vec = (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
        bool bad = false;
        for (uint32_t e = ft; e < groups * (G / 4); e += kPairThreads) {
          const uint32_t j = e / (G / 4);
          const float* sj = ss + (j % 8) * kTileWords + ((j / 8) ^ (4 * (j % 8)));
          float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
          for (uint32_t c = 0; c < 16; ++c) {
            const float sv_ = sj[c * kTileGroups];
            y.x = fmaf(cb[c].x, sv_, y.x);
            y.y = fmaf(cb[c].y, sv_, y.y);
            y.z = fmaf(cb[c].z, sv_, y.z);
            y.w = fmaf(cb[c].w, sv_, y.w);
          }
          float* oy = out + j * G + 4 * tc;
          if (vec) {
            *reinterpret_cast<float4*>(oy) = y;
          } else {
            oy[0] = y.x; oy[1] = y.y; oy[2] = y.z; oy[3] = y.w;
          }
          bad |= !finite_f32(y.x) || !finite_f32(y.y) || !finite_f32(y.z) || !finite_f32(y.w);
        }
        if (__any(bad) && (ft % warpSize) == 0) atomicOr(o.status, 1u);
      }
    }
    // the bins past pl/ph are free now; pl/ph themselves are cleared after the
    // next instance's first barrier, when every wave has read them
    if (!CUM) {
#pragma unroll
      for (uint32_t i = kPairPartWords / (4 * kPairThreads); i < kPairBins / (4 * kPairThreads); ++i)
        bins4[ft + i * kPairThreads] = make_int4(0, 0, 0, 0);
    }
  }
  if (pending) {  // the block's last instance
    __syncthreads();
    mfma_product(p_item, p_shift, p_bb, true);
  }
  if (has_kept) store_out(kept_item, kept);
}

size_t pairs_shmem(uint32_t g) {
  return g == 8 ? PairLds<8>::total : (g == 16 ? PairLds<16>::total : PairLds<32>::total);
}

// ---- GemvRows (2 <= m <= 8) -------------------------------------------------
// Nibble bins, two rows of A per atomic: for word column q, nibble n8 (output
// group 8q + n8) and code e, the bin pair (S[2rp][j][e], S[2rp+1][j][e]) is
// one 64-bit LDS word that a single ds_add_u64 updates with the 64-bit value
// x_hi * 2^32 + x_lo (x_lo sign-extended). Integer addition then carries the
// two int32 sums exactly side by side: the low word is S_lo, the high word is
// S_hi - [S_lo < 0], recovered at the flush. Odd m pads a zero row.
//
// Bin (e, n8, rp, q) is the 8-byte word ((e * 8 + n8) * MP + rp) * 32 + q, so
// one nibble's MP row pairs sit at immediate offsets from one address (one
// bfe and one shift-add per nibble), and the 32 lanes of a half-wave (one word
// column each) touch 32 consecutive 8-byte words.
//
// The pipeline is GemvPairs': a register ring of D batches of R rows per lane,
// the next instance's first batches and set-up data requested during the
// current one, x staged per row in LDS (as the 64-bit pair values) and read
// one row ahead of that row's atomics. The staged chunk holds kRowXBytes; a
// slice longer than that is restaged, from A's words and codebook in LDS.
constexpr int kRowThreads = 512;
constexpr int kRowR = 8;                                           // rows per lane per batch
constexpr int kRowD = 4;
constexpr uint32_t kRowBatchRows = (kRowThreads / 64) * 2 * kRowR;  // 128
constexpr uint32_t kRowWindow = 4096;
constexpr uint32_t kRowXBytes = 16384;
constexpr uint32_t kRowAWords = 2048;                              // A words of a slice

// Rows of x per staged chunk for MP row pairs: a power of two, so that the
// chunks tile every window (a window's rows share one scale per row of A).
__host__ __device__ constexpr uint32_t row_x_rows(uint32_t mp) {
  uint32_t rows = kRowWindow;
  while (rows * 8 * mp > kRowXBytes) rows /= 2;
  return rows;
}

template <int G, int MP>
struct RowLds {
  static constexpr uint32_t bins = 8 * 16 * MP * kTileWords * 8;  // bytes of 64-bit bins
  static constexpr uint32_t xr = row_x_rows(MP);
  static constexpr uint32_t xs = bins;
  static constexpr uint32_t af = xs + xr * MP * 8;
  static constexpr uint32_t bb = af + 16 * G * 4;
  static constexpr uint32_t aw = bb + 16 * G * 4;
  // [sign][wave][row] positive and negative mass partials
  static constexpr uint32_t wl1 = aw + kRowAWords * 4;
  static constexpr uint32_t wsh = wl1 + 2 * (kRowThreads / 64) * 8 * 4;  // [row] window shifts
  static constexpr uint32_t total = wsh + 8 * 4;
};

typedef __attribute__((address_space(3))) int64_t lds_i64;

__device__ __forceinline__ void lds_add64(uint32_t byte_addr, int64_t v) {
  __hip_atomic_fetch_add(reinterpret_cast<lds_i64*>(static_cast<size_t>(byte_addr)), v,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Words of A one slice needs: per row of A (flags 0) or one run over all
// `mall` rows of A (flags 1, where the rows interleave along k).
struct RowAWords {
  uint32_t per_row;   // words reserved per row (flags 0)
  uint32_t total;     // words staged
};

__host__ __device__ inline RowAWords row_a_words(uint32_t m, uint32_t mall, uint32_t ks,
                                                 uint32_t group, uint32_t flags) {
  RowAWords w;
  w.per_row = ks / (8 * group) + 2;
  w.total = (flags & 1u) ? ks * mall / (8 * group) + 2 : m * w.per_row;
  return w;
}

struct RowAhead {
  uint32_t w[4];   // A words tid + j * kRowThreads
  float a, b;      // entry tid of the A and B books
};

// AD: A is dense FP32 in in[0] (in[1] is not read); a nonfinite x sets status
// bit 1. Each row of A has its own scale per window (window_scale of the
// row's L1 over the window's rows), so rows of very different magnitudes
// each keep their full precision.
// The launch bins rows r0 .. r0 + m - 1 of A's `mall` rows (outputs are
// written from o.out, which the caller offsets to row r0).
// X4 (rows of whole 32-word tiles): each lane loads 4 adjacent words of R/4
// rows with 16-byte loads and reads each row's x once for its 4 words. Within
// a half-wave, lane = 16 chunk_hi + 4 slot + chunk_lo (chunk = 4 chunk_hi +
// chunk_lo of 8 four-word chunks, slot = row of 4), and a lane rotates its 4
// words by its slot, so at every atomic each 16-lane group covers 16 word
// columns of distinct residue mod 16: distinct 8-byte bank pairs, as the
// one-word-per-lane layout has.
template <int G, int MP, bool AD, bool X4 = false>
__global__ __launch_bounds__(kRowThreads, 2) void k_gemv_rows(Operands o, uint32_t m, uint32_t n,
                                                              uint32_t k, uint32_t flags,
                                                              uint32_t ks, float* partial,
                                                              uint32_t r0, uint32_t mall) {
  constexpr uint32_t R = kRowR, D = kRowD, BR = kRowBatchRows;
  constexpr uint32_t kBins64 = 8 * 16 * MP * kTileWords;
  constexpr int kPer = kBins64 / kRowThreads;     // 64-bit bins per thread
  static_assert(kBins64 % kRowThreads == 0, "bins per thread");
  static_assert(16 * G <= kRowThreads, "one book entry per thread");
  static_assert(kRowAWords <= 4 * kRowThreads, "A words per thread");
  using L = RowLds<G, MP>;
  constexpr uint32_t XR = L::xr;
  static_assert(XR >= BR && kRowWindow % XR == 0 && XR % BR == 0, "staging chunks tile windows");
  extern __shared__ int32_t smem[];
  char* lds = reinterpret_cast<char*>(smem);
  int64_t* bins = reinterpret_cast<int64_t*>(smem);
  int2* sx = reinterpret_cast<int2*>(lds + L::xs);
  float* af = reinterpret_cast<float*>(lds + L::af);
  float* bb = reinterpret_cast<float*>(lds + L::bb);
  uint32_t* aw = reinterpret_cast<uint32_t*>(lds + L::aw);
  float* wl1 = reinterpret_cast<float*>(lds + L::wl1);
  int32_t* wsh = reinterpret_cast<int32_t*>(lds + L::wsh);
  if (static_cast<uint32_t>(reinterpret_cast<size_t>((lds_i32*)smem)) != 0) {
    if (threadIdx.x == 0) atomicOr(o.status, 2u);
    return;
  }
  const uint32_t tid = threadIdx.x;
  const uint32_t tile = blockIdx.x, split = blockIdx.y, zn = gridDim.z;
  const uint32_t rw = n / (8 * G);
  const uint32_t k0 = split * ks;
  const uint32_t kend = (k0 + ks) < k ? (k0 + ks) : k;
  const uint32_t nb = (kend - k0 + BR - 1) / BR;
  const uint32_t nbp = (nb + D - 1) / D * D;
  const uint32_t lane = tid % 64, wave = tid / 64;
  const uint32_t q = lane % 32, half = lane / 32;
  constexpr uint32_t RX = X4 ? R / 4 : R;  // rows per lane per batch
  static_assert(RX % 2 == 0, "x pairs alternate by row parity");
  const uint32_t chunk = (q / 16) * 4 + q % 4, slot = half * 4 + (q / 4) % 4;
  const uint32_t lane_row = X4 ? wave * (2 * R) + slot * RX : (wave * 2 + half) * R;
  const uint32_t col = X4 ? tile * kTileWords + 4 * chunk
                          : ((tile * kTileWords + q < rw) ? tile * kTileWords + q : rw - 1);
  const uint32_t q8 = q * 8;
  // X4: word t of the rotated row is word (t + slot) % 4 of the chunk
  uint32_t lq8[X4 ? 4 : 1];
#pragma unroll
  for (uint32_t t = 0; t < (X4 ? 4u : 1u); ++t) lq8[t] = X4 ? (4 * chunk + ((t + slot) & 3u)) * 8 : q8;
  const bool rot1 = (slot & 1u) != 0, rot2 = (slot & 2u) != 0;
  const RowAWords awn = row_a_words(m, mall, ks, G, flags);
  const uint32_t a_vec_elems = mall * k;  // A's flat extent

  auto opaque = [](uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
  };
  // first A word staged for row r (flags 0) or for the slice (flags 1)
  auto a_base = [&](uint32_t r) {
    return (flags & 1u) ? (k0 * mall / G) >> 3 : (((r0 + r) * k + k0) / G) >> 3;
  };
  auto setup_loads = [&](uint32_t item) {
    const uint32_t lt = opaque(tid);
    const uint32_t a_words_all = ((a_vec_elems + G - 1) / G + 7) / 8;
    const __amdgpu_buffer_rsrc_t ars =
        words_rsrc(item_ptr<uint32_t>(o.in[0], o.stride[0], item), a_words_all * 4u);
    const __amdgpu_buffer_rsrc_t abk =
        words_rsrc(AD ? nullptr : item_ptr<float>(o.in[1], o.stride[1], item), AD ? 0u : 64u * G);
    const __amdgpu_buffer_rsrc_t bbk = words_rsrc(item_ptr<float>(o.in[3], o.stride[3], item), 64u * G);
    RowAhead h;
    h.a = __uint_as_float(uint32_t(__builtin_amdgcn_raw_buffer_load_b32(abk, lt * 4u, 0, 0)));
    h.b = __uint_as_float(uint32_t(__builtin_amdgcn_raw_buffer_load_b32(bbk, lt * 4u, 0, 0)));
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      h.w[j] = 0;
      if (AD) continue;
      const uint32_t idx = lt + j * kRowThreads;
      // staged word idx: row idx / per_row, word idx % per_row of that row (flags 0)
      const uint32_t r = (flags & 1u) ? 0u : idx / awn.per_row;
      const uint32_t i = (flags & 1u) ? idx : idx % awn.per_row;
      const bool want = idx < awn.total && r < m;
      h.w[j] = uint32_t(__builtin_amdgcn_raw_buffer_load_b32(
          ars, want ? (a_base(r) + i) * 4u : 0xfffffff0u, 0, 0));
    }
    return h;
  };
  auto batch_rsrc = [&](uint32_t item) {
    const bool real = item < o.count;
    return words_rsrc(item_ptr<uint32_t>(o.in[2], o.stride[2], real ? item : 0),
                      real ? kend * rw * 4u : 0u);
  };
  const uint32_t voff_lane = (lane_row * rw + col) * 4u;
  auto load_batch = [&](__amdgpu_buffer_rsrc_t rs, uint32_t b, uint32_t (&w)[R]) {
    uint32_t off = voff_lane + (k0 + b * BR) * rw * 4u;
    asm volatile("" : "+v"(off));
    if (X4) {
#pragma unroll
      for (uint32_t u = 0; u < RX; ++u) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, off + u * rw * 4u, 0, kStreamLoad);
        w[4 * u] = v[0]; w[4 * u + 1] = v[1]; w[4 * u + 2] = v[2]; w[4 * u + 3] = v[3];
      }
    } else {
#pragma unroll
      for (uint32_t u = 0; u < R; ++u)
        w[u] = uint32_t(__builtin_amdgcn_raw_buffer_load_b32(rs, off + u * rw * 4u, 0, kStreamLoad));
    }
  };

  uint32_t buf[D][R];
  float acc[kPer][2];
  uint32_t xbase = k0;
  __amdgpu_buffer_rsrc_t x_rs = words_rsrc(nullptr, 0u);  // AD: this instance's m x k values

  // one activation of A, as FP32
  auto x_val = [&](uint32_t r, uint32_t kk) -> float {
    const uint32_t flat = (flags & 1u) ? kk * mall + r0 + r : (r0 + r) * k + kk;
    if (AD)
      return __uint_as_float(uint32_t(__builtin_amdgcn_raw_buffer_load_b32(x_rs, flat * 4u, 0, 0)));
    const uint32_t v = flat / G;
    const uint32_t slot = (flags & 1u) ? (v >> 3) - a_base(0) : r * awn.per_row + (v >> 3) - a_base(r);
    const uint32_t code = (aw[slot] >> ((v & 7u) * 4u)) & 15u;
    return af[code * G + flat % G];
  };
  // Per-row L1 of x over the window of rows [w0, min(w0 + kRowWindow, kend)),
  // then each row's shift for that window in wsh (LDS: nothing of it lives
  // in registers through the main loop). Two barriers; flags a nonfinite x.
  auto window_scales = [&](uint32_t w0) __attribute__((always_inline)) {
    constexpr int kPerWin = kRowWindow / kRowThreads;
    const uint32_t w1 = (w0 + kRowWindow) < kend ? (w0 + kRowWindow) : kend;
    const uint32_t t = opaque(tid);
    bool bad = false;
#pragma unroll 1
    for (uint32_t r = 0; r < 2 * MP; ++r) {
      float lp = 0.0f, ln = 0.0f;  // the row's positive and negative masses
      if (r < m) {
        float v[kPerWin];
#pragma unroll
        for (int j = 0; j < kPerWin; ++j) {
          const uint32_t kk = w0 + t + j * kRowThreads;
          v[j] = kk < w1 ? x_val(r, kk) : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < kPerWin; ++j) {
          bad |= !finite_f32(v[j]);
          lp += fmaxf(v[j], 0.0f);
          ln += fmaxf(-v[j], 0.0f);
        }
      }
      lp = wave_sum(lp);
      ln = wave_sum(ln);
      if (lane == 0) {
        wl1[wave * 8 + r] = lp;
        wl1[(kRowThreads / 64 + wave) * 8 + r] = ln;
      }
    }
    if (AD && tile == 0 && __any(bad) && lane == 0) atomicOr(o.status, 1u);
    __syncthreads();
    if (t < 2 * MP) {
      float lp = 0.0f, ln = 0.0f;
#pragma unroll
      for (int w = 0; w < kRowThreads / 64; ++w) {
        lp += wl1[w * 8 + t];
        ln += wl1[(kRowThreads / 64 + w) * 8 + t];
      }
      // NaN when either mass is NaN or infinite (status bit 1 follows)
      const float l1 = fmaxf(lp, ln) + (lp - lp) + (ln - ln);
      wsh[t] = window_shift(l1);
      if (!(l1 <= FLT_MAX)) atomicOr(o.status, 1u);  // finite x whose L1 overflows FP32
    }
    __syncthreads();
  };
  // rows [xb0, xb0 + XR): per row and row pair, the 64-bit addend's two
  // halves, each quantised with its own row's scale
  auto stage_x = [&](uint32_t xb0) __attribute__((always_inline)) {
    for (uint32_t idx = opaque(tid); idx < XR * MP; idx += kRowThreads) {
      const uint32_t kk = xb0 + idx / MP, rp = idx % MP;
      int32_t lo = 0, hi = 0;
      if (kk < kend) {
        if (2 * rp < m) lo = quantize(x_val(2 * rp, kk), wsh[2 * rp]);
        if (2 * rp + 1 < m) hi = quantize(x_val(2 * rp + 1, kk), wsh[2 * rp + 1]);
      }
      sx[idx] = make_int2(lo, hi + (lo >> 31));
    }
  };
  // x pairs of one row of this lane's batch
  auto read_row = [&](uint32_t row, int2 (&xp)[MP]) __attribute__((always_inline)) {
    const int2* p = sx + (row - xbase) * MP;
#pragma unroll
    for (int rp = 0; rp < MP; ++rp) xp[rp] = p[rp];
  };
  auto flush = [&](bool clear) __attribute__((always_inline)) {
    const uint32_t ft = opaque(tid);
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint32_t bi = ft + i * kRowThreads;
      const uint32_t rp = (bi / kTileWords) % MP;  // bin (e, n8, rp, q)
      const int64_t v = bins[bi];
      const uint32_t lo = uint32_t(uint64_t(v)), hi = uint32_t(uint64_t(v) >> 32);
      acc[i][0] += unscale(float(int32_t(lo)), wsh[2 * rp]);
      acc[i][1] += unscale(float(int32_t(hi + (lo >> 31))), wsh[2 * rp + 1]);
      if (clear) bins[bi] = 0;
    }
  };
  // x pairs alternate between two register sets by row parity (R is even, so
  // the next batch's first row is read during this batch's last row)
  int2 xa[MP], xb[MP];
  auto stage = [&](uint32_t (&w)[R], uint32_t b, __amdgpu_buffer_rsrc_t rs_refill,
                   uint32_t b_refill) __attribute__((always_inline)) {
    asm volatile("" : "+s"(b));
    const uint32_t done = (b + 1) * BR;
    const bool last = b + 1 == nbp;
    const bool restage = k0 + done < kend && k0 + done - xbase >= XR;
    const bool wend = done % kRowWindow == 0 || last;
    if (b < nb) {  // padding batches (past the slice) bin nothing
      const uint32_t first = k0 + b * BR + lane_row;
#pragma unroll
      for (uint32_t u = 0; u < RX; ++u) {
        int2 (&cur)[MP] = (u & 1u) ? xb : xa;
        int2 (&nxt)[MP] = (u & 1u) ? xa : xb;
        // the next row's x is read ahead of this row's atomics (LDS operations
        // complete in order)
        if (u + 1 < RX) read_row(first + u + 1, nxt);
        else if (b + 1 < nb && !restage) read_row(first + BR, nxt);
        int64_t add[MP];
#pragma unroll
        for (int rp = 0; rp < MP; ++rp)
          add[rp] = int64_t((uint64_t(uint32_t(cur[rp].y)) << 32) | uint32_t(cur[rp].x));
        uint32_t r[X4 ? 4 : 1];
        if (X4) {
          const uint32_t a0 = rot1 ? w[4 * u + 1] : w[4 * u];
          const uint32_t a1 = rot1 ? w[4 * u + 2] : w[4 * u + 1];
          const uint32_t a2 = rot1 ? w[4 * u + 3] : w[4 * u + 2];
          const uint32_t a3 = rot1 ? w[4 * u] : w[4 * u + 3];
          r[0] = rot2 ? a2 : a0; r[X4 ? 1 : 0] = rot2 ? a3 : a1;
          r[X4 ? 2 : 0] = rot2 ? a0 : a2; r[X4 ? 3 : 0] = rot2 ? a1 : a3;
        } else {
          r[0] = w[u];
        }
#pragma unroll
        for (uint32_t t = 0; t < (X4 ? 4u : 1u); ++t) {
#pragma unroll
          for (uint32_t n8 = 0; n8 < 8; ++n8) {
            const uint32_t base = __builtin_amdgcn_ubfe(r[t], 4 * n8, 4) * (2048u * MP) + lq8[t];
#pragma unroll
            for (int rp = 0; rp < MP; ++rp) lds_add64(base + (n8 * MP + rp) * 256, add[rp]);
          }
        }
      }
    }
    load_batch(rs_refill, b_refill, w);
    __builtin_amdgcn_sched_barrier(0);
    if (wend) {
      __syncthreads();
      flush(!last);
      if (!last && !restage) __syncthreads();
    }
    if (restage) {
      if (!wend) __syncthreads();
      // a new window starts: its scales (the flush above used the old ones)
      if (done % kRowWindow == 0) window_scales(k0 + done);
      xbase = k0 + done;
      stage_x(xbase);
      __syncthreads();
      read_row(k0 + done + lane_row, xa);
      // settle here, so at the join the common path's x needs no wait behind
      // this batch's atomics
      __builtin_amdgcn_s_waitcnt(0xc07f);
    }
  };

  uint32_t item = blockIdx.z;
  RowAhead cur{}, nxt{};
  if (item < o.count) {
    cur = setup_loads(item);
    nxt = setup_loads(item + zn < o.count ? item + zn : item);
    const __amdgpu_buffer_rsrc_t r0 = batch_rsrc(item);
#pragma unroll
    for (uint32_t d = 0; d < D; ++d) load_batch(r0, d, buf[d]);
  }
  for (; item < o.count; item += zn) {
    const uint32_t next = item + zn;
    const __amdgpu_buffer_rsrc_t cur_rs = batch_rsrc(item);
    const __amdgpu_buffer_rsrc_t next_rs = batch_rsrc(next);
    // ---- set-up ----
    const uint32_t st = opaque(tid);
    __syncthreads();
    if (st < 16 * G) {
      if (!AD) af[st] = cur.a;
      bb[st] = cur.b;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (!AD && st + j * kRowThreads < kRowAWords) aw[st + j * kRowThreads] = cur.w[j];
    if (AD) x_rs = words_rsrc(item_ptr<float>(o.in[0], o.stride[0], item), mall * k * 4u);
#pragma unroll
    for (int i = 0; i < kPer; ++i) bins[st + i * kRowThreads] = 0;
    __syncthreads();
    if (tile == 0 && split == 0) sweep_books(AD ? bb : af, bb, 16 * G, o.status);
    window_scales(k0);
    xbase = k0;
    stage_x(xbase);
    __syncthreads();
    read_row(k0 + lane_row, xa);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // settle the first row's x before the loop
    cur = nxt;
    nxt = setup_loads(next + zn < o.count ? next + zn : item);
#pragma unroll
    for (int i = 0; i < kPer; ++i) acc[i][0] = acc[i][1] = 0.0f;

    for (uint32_t b0 = 0; b0 + D < nbp; b0 += D) {
#pragma unroll
      for (uint32_t d = 0; d < D; ++d) stage(buf[d], b0 + d, cur_rs, b0 + d + D);
    }
#pragma unroll
    for (uint32_t d = 0; d < D; ++d) stage(buf[d], nbp - D + d, next_rs, d);

    // ---- finalise: S[r][e][n8][q] in LDS, then y = C_B^T S per group ----
    const uint32_t ft = opaque(tid);
    float* ss = reinterpret_cast<float*>(smem);
    __syncthreads();  // every thread has flushed its bins
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const uint32_t bi = ft + i * kRowThreads;
      const uint32_t qq = bi % kTileWords, rest = bi / kTileWords;
      const uint32_t rp = rest % MP, rest2 = rest / MP;
      const uint32_t n8 = rest2 % 8, e = rest2 / 8;
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {
        const uint32_t r = 2 * rp + h;
        const float s = acc[i][h];  // scaled back at each flush
        if (gridDim.y == 1) {
          ss[((r * 16 + e) * 8 + n8) * kTileWords + qq] = s;
        } else if (r < m) {
          float* pp = partial + ((uint64_t(item) * gridDim.x + tile) * gridDim.y + split) *
                                    (m * 16 * kTileGroups);
          pp[r * 16 * kTileGroups + (qq * 8 + n8) * 16 + e] = s;
        }
      }
    }
    __syncthreads();
    if (gridDim.y == 1) {
      const uint32_t groups = (rw - tile * kTileWords) < kTileWords
                                  ? (rw - tile * kTileWords) * 8
                                  : kTileGroups;
      // thread ft always takes columns 4 tc .. 4 tc + 3 of its groups (tc = ft %
      // (G / 4)): each S value read serves four outputs
      const uint32_t tc = ft % (G / 4);
      float4 cb[16];
#pragma unroll
      for (uint32_t c = 0; c < 16; ++c)
        cb[c] = *reinterpret_cast<const float4*>(bb + c * G + 4 * tc);
      float* out = item_ptr_mut<float>(o.out, o.stride[4], item) + tile * kTileGroups * G;
      const bool vec = ((reinterpret_cast<uintptr_t>(out) | (uint64_t(n) * 4)) & 15u) == 0;
      bool bad = false;
      for (uint32_t idx = ft; idx < m * groups * (G / 4); idx += kRowThreads) {
        const uint32_t r = idx / (groups * (G / 4)), j = idx % (groups * (G / 4)) / (G / 4);
        const float* sj = ss + (r * 16 * 8 + j % 8) * kTileWords + j / 8;
        float4 y = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
        for (uint32_t c = 0; c < 16; ++c) {
          const float sv_ = sj[c * kTileGroups];
          y.x = fmaf(cb[c].x, sv_, y.x);
          y.y = fmaf(cb[c].y, sv_, y.y);
          y.z = fmaf(cb[c].z, sv_, y.z);
          y.w = fmaf(cb[c].w, sv_, y.w);
        }
        float* oy = out + uint64_t(r) * n + j * G + 4 * tc;
        if (vec) {
          *reinterpret_cast<float4*>(oy) = y;
        } else {
          oy[0] = y.x; oy[1] = y.y; oy[2] = y.z; oy[3] = y.w;
        }
        bad |= !finite_f32(y.x) || !finite_f32(y.y) || !finite_f32(y.z) || !finite_f32(y.w);
      }
      if (__any(bad) && (ft % warpSize) == 0) atomicOr(o.status, 1u);
    }
  }
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

// mrows > 1: the row instances of "gemv-row-pairs" (row_pairs_apply holds, so
// the instances fill the chip without splitting k).
template <int G, bool AD>
hipError_t launch_pairs(hipStream_t s, const Operands& o, uint32_t n, uint32_t k, uint32_t flags,
                        void* workspace, uint32_t mrows) {
  (void)flags;  // m = 1: A's flat index is the inner index either way; row instances: row-major A
  const uint32_t tiles = (n / (8 * G) + kTileWords - 1) / kTileWords;
  const uint32_t ninst = o.count * mrows;
  uint32_t ks, splits;
  pairs_slices(n, k, G, ninst, &ks, &splits);
  if (mrows > 1 && splits > 1) return hipErrorInvalidValue;  // excluded by row_pairs_apply
  // about one block per compute unit; each block walks its instances with the
  // next instance's first batches and set-up data already in flight
  const uint32_t per_z = tiles * splits;
  uint32_t zc = per_z >= 256 ? 1u : 256u / per_z;
  zc = zc < ninst ? zc : ninst;
  const size_t shmem = pairs_shmem(G);
  // one window; packed A also needs a slice length that is a multiple of 4
  // (x is read from the quantised book four rows at a time)
  const bool one_window = ks <= kPairWindow && (AD || k % 4 == 0);
  // 16-byte loads need rows of whole tiles (then every chunk is 16-byte aligned)
  const bool x4 = (n / (8 * G)) % kTileWords == 0;
  const void* fn = one_window
      ? (x4 ? reinterpret_cast<const void*>(&k_gemv_pairs<G, AD, true, true>)
            : reinterpret_cast<const void*>(&k_gemv_pairs<G, AD, true, false>))
      : (x4 ? reinterpret_cast<const void*>(&k_gemv_pairs<G, AD, false, true>)
            : reinterpret_cast<const void*>(&k_gemv_pairs<G, AD, false, false>));
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(shmem));
  if (e != hipSuccess) return e;
  dim3 grid(tiles, splits, zc);
  float* ws = static_cast<float*>(workspace);
  if (one_window && x4)
    k_gemv_pairs<G, AD, true, true><<<grid, kPairThreads, shmem, s>>>(o, n, k, ks, ws, mrows);
  else if (one_window)
    k_gemv_pairs<G, AD, true, false><<<grid, kPairThreads, shmem, s>>>(o, n, k, ks, ws, mrows);
  else if (x4)
    k_gemv_pairs<G, AD, false, true><<<grid, kPairThreads, shmem, s>>>(o, n, k, ks, ws, mrows);
  else
    k_gemv_pairs<G, AD, false, false><<<grid, kPairThreads, shmem, s>>>(o, n, k, ks, ws, mrows);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || splits == 1) return err;
  dim3 fgrid(tiles * kFinishParts, 1, zc);  // one row
  k_gemv_finish<G, 1><<<fgrid, 256, 0, s>>>(o, n, splits, tiles,
                                                 static_cast<const float*>(workspace));
  return hipGetLastError();
}

// Slices of k for GemvRows: gemv_splits' count in whole batches, and short
// enough that one slice's A words fit the staging area.
void rows_slices(uint32_t m, uint32_t mall, uint32_t n, uint32_t k, uint32_t group,
                 uint32_t flags, uint32_t count, uint32_t* ks, uint32_t* splits) {
  const uint32_t want = gemv_splits(n, k, group, count);
  uint32_t per = (k + want - 1) / want;
  per = (per + kRowBatchRows - 1) / kRowBatchRows * kRowBatchRows;
  while (per > kRowBatchRows && row_a_words(m, mall, per, group, flags).total > kRowAWords)
    per = (per / 2 + kRowBatchRows - 1) / kRowBatchRows * kRowBatchRows;
  *ks = per;
  *splits = (k + per - 1) / per;
}

template <int G, int MP, bool AD>
hipError_t launch_rows_mp(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                          uint32_t flags, void* workspace, uint32_t r0, uint32_t mall) {
  const uint32_t tiles = (n / (8 * G) + kTileWords - 1) / kTileWords;
  uint32_t ks, splits;
  rows_slices(m, mall, n, k, G, flags, o.count, &ks, &splits);
  const uint32_t per_z = tiles * splits;
  uint32_t zc = per_z >= 256 ? 1u : 256u / per_z;
  zc = zc < o.count ? zc : o.count;
  const size_t shmem = RowLds<G, MP>::total;
  // 16-byte loads need rows of whole tiles (then every chunk is 16-byte aligned)
  const bool x4 = (n / (8 * G)) % kTileWords == 0;
  const void* fn = x4 ? reinterpret_cast<const void*>(&k_gemv_rows<G, MP, AD, true>)
                      : reinterpret_cast<const void*>(&k_gemv_rows<G, MP, AD, false>);
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, int(shmem));
  if (e != hipSuccess) return e;
  Operands oc = o;  // this chunk's outputs start at row r0
  oc.out = static_cast<char*>(o.out) + uint64_t(r0) * n * sizeof(float);
  dim3 grid(tiles, splits, zc);
  float* ws = static_cast<float*>(workspace);
  if (x4)
    k_gemv_rows<G, MP, AD, true><<<grid, kRowThreads, shmem, s>>>(oc, m, n, k, flags, ks, ws, r0, mall);
  else
    k_gemv_rows<G, MP, AD, false><<<grid, kRowThreads, shmem, s>>>(oc, m, n, k, flags, ks, ws, r0, mall);
  e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  dim3 fgrid(tiles * kFinishParts, m, zc);  // a block row per row of A
  const float* part = static_cast<const float*>(workspace);
  switch (m) {
    case 1: k_gemv_finish<G, 1><<<fgrid, 256, 0, s>>>(oc, n, splits, tiles, part); break;
    case 2: k_gemv_finish<G, 2><<<fgrid, 256, 0, s>>>(oc, n, splits, tiles, part); break;
    case 3: k_gemv_finish<G, 3><<<fgrid, 256, 0, s>>>(oc, n, splits, tiles, part); break;
    case 4: k_gemv_finish<G, 4><<<fgrid, 256, 0, s>>>(oc, n, splits, tiles, part); break;
    case 5: k_gemv_finish<G, 5><<<fgrid, 256, 0, s>>>(oc, n, splits, tiles, part); break;
    case 6: k_gemv_finish<G, 6><<<fgrid, 256, 0, s>>>(oc, n, splits, tiles, part); break;
    case 7: k_gemv_finish<G, 7><<<fgrid, 256, 0, s>>>(oc, n, splits, tiles, part); break;
    default: k_gemv_finish<G, 8><<<fgrid, 256, 0, s>>>(oc, n, splits, tiles, part); break;
  }
  return hipGetLastError();
}

// A taller than kGemvMaxM rows runs as consecutive launches over chunks of
// kGemvMaxM rows (each re-reads B: the packed weight is small next to the
// general kernel's cost at these heights); the chunks share the workspace in
// stream order.
template <int G, bool AD>
hipError_t launch_rows(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                       uint32_t flags, void* workspace) {
  for (uint32_t r0 = 0; r0 < m; r0 += kGemvMaxM) {
    const uint32_t mc = (m - r0) < kGemvMaxM ? (m - r0) : kGemvMaxM;
    hipError_t e;
    switch ((mc + 1) / 2) {
      case 1: e = launch_rows_mp<G, 1, AD>(s, o, mc, n, k, flags, workspace, r0, m); break;
      case 2: e = launch_rows_mp<G, 2, AD>(s, o, mc, n, k, flags, workspace, r0, m); break;
      case 3: e = launch_rows_mp<G, 3, AD>(s, o, mc, n, k, flags, workspace, r0, m); break;
      default: e = launch_rows_mp<G, 4, AD>(s, o, mc, n, k, flags, workspace, r0, m); break;
    }
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

template <bool AD>
hipError_t launch_factorised(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                             uint32_t group, uint32_t flags, MatmulPath path, void* workspace) {
  if (path == MatmulPath::GemvPairs || path == MatmulPath::GemvRowPairs) {
    const uint32_t mrows = path == MatmulPath::GemvPairs ? 1u : m;
    if (group == 8) return launch_pairs<8, AD>(s, o, n, k, flags, workspace, mrows);
    if (group == 16) return launch_pairs<16, AD>(s, o, n, k, flags, workspace, mrows);
    return launch_pairs<32, AD>(s, o, n, k, flags, workspace, mrows);
  }
  if (group == 8) return launch_rows<8, AD>(s, o, m, n, k, flags, workspace);
  if (group == 16) return launch_rows<16, AD>(s, o, m, n, k, flags, workspace);
  return launch_rows<32, AD>(s, o, m, n, k, flags, workspace);
}

}  // namespace

const char* matmul_path_name(MatmulPath p) {
  switch (p) {
    case MatmulPath::General: return "general";
    case MatmulPath::GemvRows: return "gemv-rows";
    case MatmulPath::GemvPairs: return "gemv-pairs";
    case MatmulPath::GemvRowPairs: return "gemv-row-pairs";
    case MatmulPath::GemvTable: return "gemv-table";
    case MatmulPath::GramMfma: return "gram-mfma";
    case MatmulPath::OneHotMfma: return "onehot-mfma";
    case MatmulPath::GemvDirect: return "gemv-direct";
  }
  return "unknown";
}

MatmulPath choose_matmul_path(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                              uint32_t count, uint32_t policy) {
  if (policy == 1) return MatmulPath::General;
  if ((policy == 0 || m >= kOneHotMinRows) && onehot_applies(m, n, k, group, flags, count))
    return MatmulPath::OneHotMfma;
  if (gram_applies(m, n, k, group, flags, policy == 2)) return MatmulPath::GramMfma;
  if (policy == 0 && direct_applies(m, n, k, group, flags, count)) return MatmulPath::GemvDirect;
  if (row_pairs_apply(m, n, k, group, flags, count, false)) return MatmulPath::GemvRowPairs;
  if (rows_apply(m, n, k, group, flags))
    return m == 1 ? MatmulPath::GemvPairs : MatmulPath::GemvRows;
  return MatmulPath::General;
}

size_t matmul_workspace_bytes(MatmulPath p, uint32_t m, uint32_t n, uint32_t k, uint32_t group,
                              uint32_t flags, uint32_t count) {
  if (p == MatmulPath::OneHotMfma) return onehot_workspace_bytes(m, n, k, group);
  if (p == MatmulPath::GemvDirect) return direct_workspace_bytes(m, n, k, group, count);
  if (p != MatmulPath::GemvRows && p != MatmulPath::GemvPairs) return 0;
  uint32_t ks, splits;
  // the largest chunk of rows one launch bins; chunks reuse the partials
  const uint32_t mc = m < kGemvMaxM ? m : kGemvMaxM;
  uint32_t most = 1;
  if (p == MatmulPath::GemvPairs) {
    pairs_slices(n, k, group, count, &ks, &splits);
    most = splits;
  } else {
    for (uint32_t r0 = 0; r0 < m; r0 += kGemvMaxM) {
      rows_slices((m - r0) < kGemvMaxM ? (m - r0) : kGemvMaxM, m, n, k, group, flags, count, &ks,
                  &splits);
      most = splits > most ? splits : most;
    }
  }
  if (most == 1) return 0;
  const uint32_t tiles = (n / (8 * group) + kTileWords - 1) / kTileWords;
  return size_t(count) * most * tiles * mc * 16 * kTileGroups * sizeof(float);
}

hipError_t launch_matmul(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                         uint32_t group, uint32_t flags, MatmulPath path, void* workspace,
                         size_t workspace_bytes) {
  (void)workspace_bytes;
  if (path == MatmulPath::OneHotMfma) return launch_onehot(s, o, m, n, k, group, false, workspace);
  if (path == MatmulPath::GemvDirect)
    return launch_direct(s, o, m, n, k, group, flags, false, workspace);
  if (path == MatmulPath::GramMfma) return launch_gram(s, o, m, n, k, group);
  if (path == MatmulPath::GemvPairs || path == MatmulPath::GemvRows ||
      path == MatmulPath::GemvRowPairs)
    return launch_factorised<false>(s, o, m, n, k, group, flags, path, workspace);
  const uint32_t zc = o.count < 65535 ? o.count : 65535;
  dim3 grid((n + kGT - 1) / kGT, (m + kGT - 1) / kGT, zc);
  if (group == 8) k_matmul_general<8, false><<<grid, kGThreads, 0, s>>>(o, m, n, k, flags);
  else if (group == 16) k_matmul_general<16, false><<<grid, kGThreads, 0, s>>>(o, m, n, k, flags);
  else k_matmul_general<32, false><<<grid, kGThreads, 0, s>>>(o, m, n, k, flags);
  return hipGetLastError();
}

MatmulPath choose_dense_path(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                             uint32_t count, uint32_t policy) {
  if (policy == 1) return MatmulPath::General;
  if ((policy == 0 || m >= kOneHotMinRows) && onehot_applies_dense(m, n, k, group, flags, count))
    return MatmulPath::OneHotMfma;
  if (policy == 0 && direct_applies(m, n, k, group, flags, count)) return MatmulPath::GemvDirect;
  if (row_pairs_apply(m, n, k, group, flags, count, true)) return MatmulPath::GemvRowPairs;
  if (rows_apply(m, n, k, group, flags))
    return m == 1 ? MatmulPath::GemvPairs : MatmulPath::GemvRows;
  return MatmulPath::General;
}

// The factorised paths' split-k partials (the GEMV kernels take each window's
// scale from x themselves) and onehot-mfma's nibble columns and bf16 planes.
size_t dense_workspace_bytes(MatmulPath p, uint32_t m, uint32_t n, uint32_t k, uint32_t group,
                             uint32_t flags, uint32_t count) {
  if (p == MatmulPath::OneHotMfma) return onehot_dense_workspace_bytes(m, n, k, group);
  return matmul_workspace_bytes(p, m, n, k, group, flags, count);
}

hipError_t launch_matmul_dense(hipStream_t s, const Operands& o, uint32_t m, uint32_t n,
                               uint32_t k, uint32_t group, uint32_t flags, MatmulPath path,
                               void* workspace, size_t workspace_bytes) {
  (void)workspace_bytes;
  if (path == MatmulPath::OneHotMfma) return launch_onehot(s, o, m, n, k, group, true, workspace);
  if (path == MatmulPath::GemvDirect)
    return launch_direct(s, o, m, n, k, group, flags, true, workspace);
  if (path == MatmulPath::GemvPairs || path == MatmulPath::GemvRows ||
      path == MatmulPath::GemvRowPairs)
    return launch_factorised<true>(s, o, m, n, k, group, flags, path, workspace);
  const uint32_t zc = o.count < 65535 ? o.count : 65535;
  dim3 grid((n + kGT - 1) / kGT, (m + kGT - 1) / kGT, zc);
  if (group == 8) k_matmul_general<8, true><<<grid, kGThreads, 0, s>>>(o, m, n, k, flags);
  else if (group == 16) k_matmul_general<16, true><<<grid, kGThreads, 0, s>>>(o, m, n, k, flags);
  else k_matmul_general<32, true><<<grid, kGThreads, 0, s>>>(o, m, n, k, flags);
  return hipGetLastError();
}

}  // namespace ackvq
