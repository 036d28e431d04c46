// Large packed products with B grouped along n, on gfx950 matrix cores:
// "onehot-mfma".
//
// For C = A . B with B stored (k, n), its groups along n, and A row-major
// with its groups along k (op 2, flags 0 of
// src/alelyon_compute_kit/_kit/kernels/vq4.comp:165-176), output group j of
// row r is
//   y[r][G j + t] = sum_e S[r][(j, e)] C_B[e][t],
//   S[r][(j, e)]  = sum_kk A[r][kk] [b(kk, j) = e],
// so S = A . P with P[kk][(j, e)] the one-hot of B's code: a GEMM of inner
// dimension k and 16 n / G columns. It runs on v_mfma_f32_32x32x16_bf16:
//  - P is exact in bf16. Each lane builds its fragment (8 inner indices of one
//    (j, e) column) from one word of B's "nibble columns" (the 8 codes of group
//    j at 8 consecutive inner indices, written by a pre-pass) with a few
//    integer operations.
//  - A's values are rows of its book, so A's fragment (8 inner indices of one
//    row, inside one group) is read from an LDS table of the book scaled by a
//    power of two (largest magnitude below 2^15) and split into three bf16
//    terms hi + mid + lo: 24 significant bits with FP32's exponent range, so
//    every FP32 entry down to 2^-118 of the largest is carried exactly (the
//    last term stays a normal bf16; fp16 terms would stop at fp16's subnormal
//    floor, 2^-39 of the largest). Each 16-step of k costs three
//    MFMAs per 32 x 32 block and the accumulation is FP32.
// Then the 16-term products with C_B run on the VALU from S staged in LDS.
// Neither operand is decoded to memory.
//
// The sum order differs from the shader's sequential one; results agree to
// FP32 rounding (FP32 sums of exact A values, then 16 FP32 multiply-adds).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "kernels.hpp"

namespace ackvq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kOHThreads = 256;  // 4 waves, 2 x 2 over 64 X rows x 128 S columns
constexpr int kOHTerms = 3;           // bf16 terms of each scaled A value
// VALU operations the scheduler places after each MFMA of a step: with the
// next step's one-hot builds interleaved so, config 4's forward measured
// ~300 against ~310 us and an 8 x 4096 x 14336 g16 product 35.4 against
// 39.6 us (3, 4, 6 and 8 within noise of 5)
constexpr int kOHPipeValu = 5;
// X = 4 (256 rows per block) reuses each one-hot fragment over 12 MFMAs; X = 1
// (64 rows) gives four times the waves, for products whose 256-row grid would
// leave most of the chip idle.
constexpr uint32_t kOHBigGrid = 256;  // blocks of the X = 4 grid from which it is taken

__device__ __forceinline__ bool finite_f32(float x) { return fabsf(x) <= FLT_MAX; }

// The power of two that brings A's book below 2^15 (amax its largest finite
// magnitude): 15 - e for amax in [2^(e-1), 2^e), 0 for an all-zero book.
__device__ __forceinline__ int book_shift(float amax) {
  if (!(amax > 0.0f)) return 0;
  int ex;
  frexpf(amax, &ex);
  const int shift = 15 - ex;
  return shift < -126 ? -126 : (shift > 126 ? 126 : shift);
}

// Nibbles of vectors v .. v+7 (vector v in bits 0..3). Both loads are
// unconditional: the word index is clamped to the array (a clamped word only
// supplies nibbles past the last vector, which the caller never uses).
__device__ __forceinline__ uint32_t nibbles8(const uint32_t* codes, uint64_t v, uint64_t last) {
  const uint64_t w = v >> 3;
  const uint32_t lo = codes[w < last ? w : last];
  const uint32_t hi = codes[w + 1 < last ? w + 1 : last];
  return __builtin_amdgcn_alignbit(hi, lo, uint32_t(v & 7u) * 4u);
}

// One-hot fragment from a nibble-column word w (nibble i: B's code at inner
// index kk0 + i): bf16 element i is 1.0 where nibble i equals the lane's code
// c; ee = c * 0x11111111.
__device__ __forceinline__ bf16x8 one_hot_column(uint32_t w, uint32_t ee) {
  const uint32_t z = w ^ ee;  // nibble i is zero where it matches
  uint32_t t = z | (z >> 1);
  t |= t >> 2;                                          // bit 4i: nibble i nonzero
  const uint32_t g = (t & 0x11111111u) ^ 0x11111111u;   // bit 4i: nibble i matches
  const uint32_t fe = g & 0x01010101u, fo = (g >> 4) & 0x01010101u;
  // 0xFF bytes where fe, fo hold a 1 (even, odd nibbles). The shifted copies
  // are opaque so that the compiler keeps a shift and a subtract (full rate)
  // instead of folding them into v_mul_lo_u32 (quarter rate).
  uint32_t fe8 = fe << 8, fo8 = fo << 8;
  asm("" : "+v"(fe8), "+v"(fo8));
  const uint32_t FE = fe8 - fe, FO = fo8 - fo;
  // dword d: element 0 from nibble 2d (byte d of FE in both of its bytes),
  // element 1 from nibble 2d + 1 (of FO); bf16 1.0 is 0x3F80
  u32x4 v;
  v[0] = __builtin_amdgcn_perm(FO, FE, 0x04040000u) & 0x3F803F80u;
  v[1] = __builtin_amdgcn_perm(FO, FE, 0x05050101u) & 0x3F803F80u;
  v[2] = __builtin_amdgcn_perm(FO, FE, 0x06060202u) & 0x3F803F80u;
  v[3] = __builtin_amdgcn_perm(FO, FE, 0x07070303u) & 0x3F803F80u;
  return __builtin_bit_cast(bf16x8, v);
}

// Dense activations: 8 FP32 values split into three bf16 terms hi + mid + lo
// (each the bf16 rounding of what the previous ones leave; the differences are
// exact in FP32 and the last term holds the rest exactly for values of at
// least 2^-103, so no scale is needed). hi is the rounding of x clamped to the
// largest bf16 (0x1.fep127): a finite x past it would otherwise round hi up to
// infinity; its rest, below 2^121, still splits exactly into mid and lo. A NaN
// or infinite x leaves a NaN or infinite rest, which reaches the output and
// raises status bit 1. The main loop adds lo, then mid, then hi, so a partial
// sum of one value's terms never passes the value itself (hi + mid alone can:
// FLT_MAX splits into the largest bf16 + 2^120 - 2^104, and hi + mid is 2^128).
constexpr float kBf16Max = 0x1.fep127f;
__device__ __forceinline__ void split_bf16x3(const float4 a, const float4 b, bool zero,
                                             bf16x8 (&d)[3]) {
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float x = zero ? 0.0f : v[i];
    const __bf16 hi = __bf16(fminf(fmaxf(x, -kBf16Max), kBf16Max));
    const float r1 = x - float(hi);
    const __bf16 mid = __bf16(r1);
    d[0][i] = hi;
    d[1][i] = mid;
    d[2][i] = __bf16(r1 - float(mid));
  }
}

// Nibble columns of B: nc[j * (k / 8) + kk8] holds the codes of group j at
// inner indices 8 kk8 .. 8 kk8 + 7 (nibble i: index 8 kk8 + i). A block reads
// 16 rows of 32 word columns (coalesced) into LDS and writes the 256 groups'
// 2 words each: small tiles, so that even a 4096-row weight spreads over 256
// blocks (with 64-row tiles the pre-pass took 4.8 of a 128-row chunk's
// 19.1 us; 16-row tiles: 18.3 us). Requires k % 8 == 0.
constexpr uint32_t kNCRows = 16, kNCCols = 32;
__global__ __launch_bounds__(256) void k_nibble_columns(const uint32_t* __restrict__ codes,
                                                        uint32_t* __restrict__ nc, uint32_t k,
                                                        uint32_t rw) {
  __shared__ uint32_t tile[kNCRows][kNCCols + 1];
  const uint32_t q0 = blockIdx.x * kNCCols, k0 = blockIdx.y * kNCRows;
  const uint32_t tid = threadIdx.x;
  for (uint32_t i = tid; i < kNCRows * kNCCols; i += 256) {
    const uint32_t r = i / kNCCols, c = i % kNCCols;
    tile[r][c] = (k0 + r < k && q0 + c < rw) ? codes[uint64_t(k0 + r) * rw + q0 + c] : 0u;
  }
  __syncthreads();
  const uint32_t c = tid / 8, p = tid % 8;  // word column q0 + c, nibble p: group 8 (q0 + c) + p
  if (q0 + c >= rw) return;
  const uint32_t k8 = k / 8;
  uint32_t* dst = nc + uint64_t(8 * (q0 + c) + p) * k8 + k0 / 8;
#pragma unroll
  for (uint32_t r8 = 0; r8 < kNCRows / 8; ++r8) {
    if (k0 / 8 + r8 >= k8) break;
    uint32_t w = 0;
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i)
      w |= __builtin_amdgcn_ubfe(tile[8 * r8 + i][c], 4 * p, 4) << (4 * i);
    dst[r8] = w;
  }
}

// grid: (n / (8 G) word columns of B, ceil(m / (64 X))). A block covers 64 X
// rows of A and the 8 groups of one word column of B (128 S columns); wave
// (wy, wx) takes rows 32 X wy .. +32 X - 1 and groups 4 wx .. 4 wx + 3.
// Requires k % 16 == 0, k % G == 0 (packed A) and n % (8 G) == 0; one
// instance. AD: A is dense FP32 in in[0], split into three bf16 terms as it is
// read (a nonfinite x reaches every output of its row, which sets status bit 1).
// Split k (small grids): block z covers inner indices [z kpart, (z + 1) kpart)
// (kpart a multiple of 8 G) and writes its S, still scaled by 2^shift, to
// partial[z][r][16 j + e] instead of finishing the product; k_onehot_finish
// adds the splits in order and applies C_B. partial is null when k is not
// split (gridDim.z 1, kpart k).
// S rows a wave stages per epilogue round: one or two 32-row blocks
template <int X>
constexpr uint32_t oh_chunk_rows() { return X % 2 ? 32 : 64; }

// A's table: [term][8-entry chunk of the group][code][8]; code 16 is empty
// (rows past m). The 16 lanes of a read phase read one chunk, so distinct
// codes land in distinct banks.
template <int G>
using OHTable = __bf16[kOHTerms][G / 8][17][8];

// One block of k_onehot_mfma: word column q, rows rowb .. rowb + 64 X - 1,
// split part z. The LDS areas come from the kernel: sS holds at least
// 4 oh_chunk_rows<X>() x 64 floats (one wave's S, a round at a time).
template <int G, int X, bool AD>
__device__ __forceinline__ void onehot_block(const Operands& o, uint32_t m, uint32_t n,
                                             uint32_t k, const uint32_t* __restrict__ nc,
                                             uint32_t kpart, float* __restrict__ partial,
                                             uint32_t q, uint32_t rowb, uint32_t z,
                                             bool check_books, OHTable<G>& tabA, float* sS,
                                             float* sbook, float* sred) {
  static_assert(G == 16 || G == 32 || (AD && G == 8), "a 16-step of k lies in one group of A");
  static_assert(X >= 1 && X <= 4, "row blocks per wave");
  constexpr int kOHX = X;
  constexpr uint32_t kChunkRows = oh_chunk_rows<X>();
  const uint32_t tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const uint32_t i32 = lane % 32, h = lane / 32;
  const uint32_t wy = wave / 2, wx = wave % 2;
  const uint32_t row0 = rowb + 32 * X * wy;
  const uint32_t J = k / G;
  const uint64_t a_last = (uint64_t(m) * J + 7) / 8 - 1;
  const uint32_t* a_codes = static_cast<const uint32_t*>(o.in[0]);
  const float* xa = static_cast<const float*>(o.in[0]);
  const float* a_book = static_cast<const float*>(o.in[1]);
  const float* b_book = static_cast<const float*>(o.in[3]);
  float* out = static_cast<float*>(o.out);
  // Rows past m read the last row's codes and use the empty table entry.
  uint64_t av[kOHX];
  bool dead[kOHX];
#pragma unroll
  for (int x = 0; x < kOHX; ++x) {
    const uint32_t r = row0 + 32 * x + i32;
    av[x] = uint64_t(r < m ? r : m - 1) * J;
    dead[x] = r >= m;
  }
  // The lane's S columns: code i32 % 16 of groups 8 q + 4 wx + 2 y + i32 / 16
  // (y = 0, 1), and its nibble-column words (K entries 8 h .. 8 h + 7).
  const uint32_t ee = (i32 % 16) * 0x11111111u;
  const uint32_t k8 = k / 8;
  const uint32_t* nc0 = nc + uint64_t(8 * q + 4 * wx + i32 / 16) * k8 + h;
  const uint32_t* nc1 = nc0 + 2 * uint64_t(k8);
  // this block's inner indices [kb, ke)
  const uint32_t kb = z * kpart;
  const uint32_t ke = (kb + kpart) < k ? (kb + kpart) : k;

  // ---- tables: B's book as is; A's scaled below 2^15 and split into three
  // bf16 terms (each the bf16 rounding of what the previous ones leave; the
  // differences are exact in FP32, and the last one holds the rest exactly)
  bool bad = false;
  float amax = 0.0f;
  for (uint32_t i = tid; i < 16 * G; i += kOHThreads) {
    const float a = AD ? 0.0f : a_book[i], b = b_book[i];
    sbook[i] = b;
    if (check_books) bad |= !finite_f32(a) || !finite_f32(b);
    amax = fmaxf(amax, finite_f32(a) ? fabsf(a) : 0.0f);
  }
  for (int off = 1; off < 64; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
  if (lane == 0) sred[wave] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(sred[0], sred[1]), fmaxf(sred[2], sred[3]));
  const int shift = book_shift(amax);
  for (uint32_t i = tid; i < (AD ? 0u : 17u * G); i += kOHThreads) {
    const float scaled = i < 16 * G ? ldexpf(a_book[i], shift) : 0.0f;
    const __bf16 hi = __bf16(scaled);
    const float r1 = scaled - float(hi);
    const __bf16 mid = __bf16(r1);
    tabA[0][(i % G) / 8][i / G][i % 8] = hi;
    tabA[1][(i % G) / 8][i / G][i % 8] = mid;
    tabA[2][(i % G) / 8][i / G][i % 8] = __bf16(r1 - float(mid));
  }
  __syncthreads();

  // ---- main loop: passes over 8 groups of A (8 G inner indices, G / 2 steps
  // of 16), A's code words one pass ahead, B's words three steps ahead in a
  // ring of four, the next step's one-hot fragments built between this step's
  // MFMAs, and term t of the next step's A fragments read as soon as this
  // step's term-t MFMAs are issued, into the same registers
  f32x16 acc[kOHX][2];
#pragma unroll
  for (int x = 0; x < kOHX; ++x)
#pragma unroll
    for (int y = 0; y < 2; ++y) acc[x][y] = (f32x16)0.0f;
  constexpr uint32_t kSteps = G / 2;
  constexpr uint32_t kChunk = 17 * 16;          // bytes of one chunk's table
  constexpr uint32_t kTerm = (G / 8) * kChunk;  // bytes of one term's table
  static_assert(kSteps % 4 == 0, "the B ring position repeats every pass");
  const char* tab_lane = reinterpret_cast<const char*>(&tabA[0][0][0][0]) + h * kChunk;
  uint32_t aw[kOHX], an[kOHX];
#pragma unroll
  for (int x = 0; x < kOHX; ++x) an[x] = AD ? 0u : nibbles8(a_codes, av[x] + kb / G, a_last);
  uint32_t wb[4][2];
  wb[0][0] = nc0[kb / 8];
  wb[0][1] = nc1[kb / 8];
  wb[1][0] = nc0[(kb + 16 < ke ? kb + 16 : kb) / 8];
  wb[1][1] = nc1[(kb + 16 < ke ? kb + 16 : kb) / 8];
  wb[2][0] = nc0[(kb + 32 < ke ? kb + 32 : kb) / 8];
  wb[2][1] = nc1[(kb + 32 < ke ? kb + 32 : kb) / 8];
  // one-hot fragments of the current step; the next step's are built between
  // this step's MFMAs
  bf16x8 bfc[2];
  bfc[0] = one_hot_column(wb[0][0], ee);
  bfc[1] = one_hot_column(wb[0][1], ee);
  // the table row of step s_ (both halves of the wave are in one group; the
  // lane's chunk is c8 + h)
  auto a_ptr = [&](const uint32_t (&wd)[kOHX], uint32_t s_, int x) __attribute__((always_inline)) {
    const uint32_t g_in = (16 * s_) / G, c8 = (16 * s_ % G) / 8;
    const uint32_t code = dead[x] ? 16u : __builtin_amdgcn_ubfe(wd[x], 4 * g_in, 4);
    return tab_lane + c8 * kChunk + code * 16;
  };
  bf16x8 af[kOHX][kOHTerms];
  // AD: the lane's 8 values of each row, one step ahead (rows past m read the
  // last row and are zeroed by the split)
  const float* xr[kOHX];
  float4 xn[kOHX][2];
#pragma unroll
  for (int x = 0; x < kOHX; ++x) {
    if (AD) {
      const uint32_t r = row0 + 32 * x + i32;
      xr[x] = xa + uint64_t(r < m ? r : m - 1) * k + 8 * h;
      xn[x][0] = *reinterpret_cast<const float4*>(xr[x] + kb);
      xn[x][1] = *reinterpret_cast<const float4*>(xr[x] + kb + 4);
    } else {
      const char* pa = a_ptr(an, 0, x);
#pragma unroll
      for (int t = 0; t < kOHTerms; ++t)
        af[x][t] = *reinterpret_cast<const bf16x8*>(pa + t * kTerm);
    }
  }
  // Every load of a step is issued unconditionally (indices past the last
  // step are clamped to it, and the A table and nibbles8 stay in bounds), and
  // only the ragged last pass can leave the unrolled loop early: a load behind
  // a branch leaves the compiler unable to count the loads in flight, and it
  // then waits for all of them, the ones just issued for later steps included.
  const uint32_t klast = ke - 16;  // the last step's first inner index
  auto pass = [&](uint32_t p0, bool ragged) __attribute__((always_inline)) {
#pragma unroll
    for (int x = 0; x < kOHX; ++x) {
      aw[x] = an[x];
      if (!AD) an[x] = nibbles8(a_codes, av[x] + (p0 + 8 * G) / G, a_last);
    }
#pragma unroll
    for (uint32_t s = 0; s < kSteps; ++s) {
      const uint32_t kk0 = p0 + 16 * s;
      if (ragged && kk0 >= ke) break;
      const uint32_t kw = kk0 + 48 < klast ? kk0 + 48 : klast;
      wb[(s + 3) % 4][0] = nc0[kw / 8];
      wb[(s + 3) % 4][1] = nc1[kw / 8];
      const uint32_t kn = kk0 + 16 < klast ? kk0 + 16 : klast;
      const char* pn[kOHX];
#pragma unroll
      for (int x = 0; x < kOHX; ++x) {
        if (AD) {
          split_bf16x3(xn[x][0], xn[x][1], dead[x], af[x]);
          xn[x][0] = *reinterpret_cast<const float4*>(xr[x] + kn);
          xn[x][1] = *reinterpret_cast<const float4*>(xr[x] + kn + 4);
        } else {
          pn[x] = s + 1 < kSteps ? a_ptr(aw, s + 1, x) : a_ptr(an, 0, x);
        }
      }
      // the loads for later steps go out before this step's work (left to
      // itself the scheduler sinks them next to their use and waits on them)
      __builtin_amdgcn_sched_barrier(0);
      bf16x8 bfn[2];
      bfn[0] = one_hot_column(wb[(s + 1) % 4][0], ee);
      bfn[1] = one_hot_column(wb[(s + 1) % 4][1], ee);
      // terms smallest first: lo, mid, hi
#pragma unroll
      for (int t = kOHTerms - 1; t >= 0; --t) {
#pragma unroll
        for (int x = 0; x < kOHX; ++x)
#pragma unroll
          for (int y = 0; y < 2; ++y)
            acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[x][t], bfc[y], acc[x][y], 0, 0, 0);
        if (!AD) {
#pragma unroll
          for (int x = 0; x < kOHX; ++x)
            af[x][t] = *reinterpret_cast<const bf16x8*>(pn[x] + t * kTerm);
        }
      }
      // each MFMA followed by up to kOHPipeValu VALU operations (the next
      // step's one-hot builds, addresses), each term's table reads after its
      // MFMAs: the matrix pipe stays fed by this wave alone
#pragma unroll
      for (int t = 0; t < kOHTerms; ++t) {
#pragma unroll
        for (int i = 0; i < 2 * kOHX; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x002, kOHPipeValu, 0);
        }
        if (!AD) __builtin_amdgcn_sched_group_barrier(0x100, kOHX, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      bfc[0] = bfn[0];
      bfc[1] = bfn[1];
    }
  };
  const uint32_t whole = kb + (ke - kb) / (8 * G) * (8 * G);  // end of the whole passes
  for (uint32_t p0 = kb; p0 < whole; p0 += 8 * G) pass(p0, false);
  if (whole < ke) pass(whole, true);

  if (partial != nullptr) {  // this split's S, scaled, for k_onehot_finish
    const uint32_t cols = 16 * (n / G);
    float* pz = partial + uint64_t(z) * m * cols + 16 * (8 * q + 4 * wx) + i32;
#pragma unroll
    for (int x = 0; x < kOHX; ++x)
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const uint32_t r = row0 + 32 * x + (t % 4) + 4 * h + 8 * (t / 4);
        if (r < m) {
          pz[uint64_t(r) * cols] = acc[x][0][t];
          pz[uint64_t(r) * cols + 32] = acc[x][1][t];
        }
      }
    if (__any(bad) && lane == 0) atomicOr(o.status, 1u);
    return;
  }

  // ---- S to LDS, kChunkRows rows at a time (lane: column i32, item t holds
  // row (t % 4) + 4 h + 8 (t / 4) of its 32-row block), then
  // y[r][G j + t] = sum_e S[r][(j, e)] C_B[e][t], e ascending; a lane's t is
  // fixed (the row stride 64 is a multiple of G). S stays scaled by 2^shift
  // through the product and y is unscaled last (one ldexp, exact unless y is
  // subnormal), so A values near FLT_MAX / k cannot overflow a bucket sum
  // whose products with C_B are finite.
  const uint32_t tc = lane % G;
  float cb[16];
#pragma unroll
  for (int f = 0; f < 16; ++f) cb[f] = sbook[f * G + tc];
  constexpr int kTilesPerRound = kChunkRows / 32;
#pragma unroll
  for (int hv = 0; hv < X / kTilesPerRound; ++hv) {
    if (hv) __syncthreads();  // the previous round has been read
#pragma unroll
    for (int x = 0; x < kTilesPerRound; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y)
#pragma unroll
        for (int t = 0; t < 16; ++t)
          sS[(wave * kChunkRows + 32 * x + (t % 4) + 4 * h + 8 * (t / 4)) * 64 + 32 * y + i32] =
              acc[kTilesPerRound * hv + x][y][t];
    __syncthreads();
    for (uint32_t idx = lane; idx < kChunkRows * 4 * G; idx += 64) {
      const uint32_t row = idx / (4 * G), jl = (idx % (4 * G)) / G;
      const uint32_t r = row0 + kChunkRows * hv + row;
      if (r >= m) break;
      const float4* sp = reinterpret_cast<const float4*>(&sS[(wave * kChunkRows + row) * 64 + 16 * jl]);
      const float4 s0 = sp[0], s1 = sp[1], s2 = sp[2], s3 = sp[3];
      float y = 0.0f;
      y = fmaf(s0.x, cb[0], y);
      y = fmaf(s0.y, cb[1], y);
      y = fmaf(s0.z, cb[2], y);
      y = fmaf(s0.w, cb[3], y);
      y = fmaf(s1.x, cb[4], y);
      y = fmaf(s1.y, cb[5], y);
      y = fmaf(s1.z, cb[6], y);
      y = fmaf(s1.w, cb[7], y);
      y = fmaf(s2.x, cb[8], y);
      y = fmaf(s2.y, cb[9], y);
      y = fmaf(s2.z, cb[10], y);
      y = fmaf(s2.w, cb[11], y);
      y = fmaf(s3.x, cb[12], y);
      y = fmaf(s3.y, cb[13], y);
      y = fmaf(s3.z, cb[14], y);
      y = fmaf(s3.w, cb[15], y);
      if (!AD) y = ldexpf(y, -shift);
      out[uint64_t(r) * n + (8 * q + 4 * wx + jl) * G + tc] = y;
      bad |= !finite_f32(y);
    }
  }
  if (__any(bad) && lane == 0) atomicOr(o.status, 1u);
}

// grid: (n / (8 G), ceil(m / (64 X)), split parts)
template <int G, int X, bool AD>
__global__ __launch_bounds__(kOHThreads, X == 1 ? 4 : 2) void k_onehot_mfma(
    Operands o, uint32_t m, uint32_t n, uint32_t k, const uint32_t* __restrict__ nc,
    uint32_t kpart, float* __restrict__ partial) {
  __shared__ __align__(16) OHTable<G> tabA;
  __shared__ __align__(16) float sS[4 * oh_chunk_rows<X>() * 64];
  __shared__ float sbook[16 * G];
  __shared__ float sred[4];
  onehot_block<G, X, AD>(o, m, n, k, nc, kpart, partial, blockIdx.x, blockIdx.y * (64 * X),
                         blockIdx.z, blockIdx.x == 0 && blockIdx.y == 0, tabA, sS, sbook, sred);
}

// Packed A on a grid with fewer 256-row blocks than the chip holds (two per
// compute unit, kOHSlots), where whole 256-row blocks would leave slots idle
// for the whole product (config 4: 448 blocks for 512 slots): the rows of
// each word column are cut into 256-row (X = 4) and 192-row (X = 3) blocks, as
// many of each as half the slots, so that each compute unit can hold one of
// each and every unit does the same work. Columns 0 .. c1 - 1 hold a1 blocks
// of 256 rows then b1 of 192; columns c1 .. hold a2 and b2. Blocks
// 0 .. n4 - 1 are the 256-row ones, column-major; the rest the 192-row ones.
struct OHMixed {
  uint32_t c1, a1, b1, a2, b2;
};

template <int G>
__global__ __launch_bounds__(kOHThreads, 2) void k_onehot_mixed(Operands o, uint32_t m, uint32_t n,
                                                                uint32_t k,
                                                                const uint32_t* __restrict__ nc,
                                                                OHMixed mx) {
  __shared__ __align__(16) OHTable<G> tabA;
  __shared__ __align__(16) float sS[4 * 64 * 64];
  __shared__ float sbook[16 * G];
  __shared__ float sred[4];
  const uint32_t b = blockIdx.x, n4 = mx.c1 * mx.a1 + (n / (8 * G) - mx.c1) * mx.a2;
  if (b < n4) {
    const uint32_t first = mx.c1 * mx.a1;
    const uint32_t q = b < first ? b / mx.a1 : mx.c1 + (b - first) / mx.a2;
    const uint32_t slot = b < first ? b % mx.a1 : (b - first) % mx.a2;
    onehot_block<G, 4, false>(o, m, n, k, nc, k, nullptr, q, 256 * slot, 0, b == 0, tabA, sS,
                              sbook, sred);
  } else {
    const uint32_t j = b - n4, first = mx.c1 * mx.b1;
    const uint32_t q = j < first ? j / mx.b1 : mx.c1 + (j - first) / mx.b2;
    const uint32_t slot = j < first ? j % mx.b1 : (j - first) % mx.b2;
    const uint32_t above = 256 * (j < first ? mx.a1 : mx.a2);  // the column's 256-row blocks
    onehot_block<G, 3, false>(o, m, n, k, nc, k, nullptr, q, above + 192 * slot, 0, false, tabA,
                              sS, sbook, sred);
  }
}

// Split k, second half: S[r][(j, e)] = the splits' partial sums added in split
// order, then k_onehot_mfma's epilogue, y[r][G j + t] = sum_e S[r][(j, e)]
// C_B[e][t] (e ascending), unscaled by 2^-shift for packed A. grid:
// (ceil(n / 256), m): block (x, r) finishes columns 256 x .. 256 x + 255 of row
// r. Its threads first sum the block's 16 (256 / G) S entries over the splits
// (each entry read once, coalesced, the loads of four splits issued before
// their adds), then one thread per output takes its group's 16 from LDS.
template <int G, bool AD>
__global__ __launch_bounds__(256) void k_onehot_finish(Operands o, uint32_t m, uint32_t n,
                                                       uint32_t splits,
                                                       const float* __restrict__ partial) {
  constexpr uint32_t kS = 16 * 256 / G;  // S entries of the block's 256 columns
  __shared__ float sred[4];
  __shared__ float sS[kS];
  const uint32_t tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  int shift = 0;
  if (!AD) {
    const float* a_book = static_cast<const float*>(o.in[1]);
    float amax = 0.0f;
    for (uint32_t i = tid; i < 16 * G; i += 256) {
      const float a = a_book[i];
      amax = fmaxf(amax, finite_f32(a) ? fabsf(a) : 0.0f);
    }
    for (int off = 1; off < 64; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if (lane == 0) sred[wave] = amax;
    __syncthreads();
    shift = book_shift(fmaxf(fmaxf(sred[0], sred[1]), fmaxf(sred[2], sred[3])));
  }
  const uint32_t r = blockIdx.y, c0 = blockIdx.x * 256;
  const uint32_t cols = 16 * (n / G);                 // S entries per row
  const uint32_t s0 = 16 * (c0 / G);                  // the block's first S entry
  const uint64_t zstride = uint64_t(m) * cols;
  for (uint32_t i = tid; i < kS; i += 256) {
    if (s0 + i >= cols) break;
    const float* p = partial + uint64_t(r) * cols + s0 + i;
    float sum = 0.0f;
    uint32_t z = 0;
    for (; z + 4 <= splits; z += 4) {
      const float a0 = p[z * zstride], a1 = p[(z + 1) * zstride];
      const float a2 = p[(z + 2) * zstride], a3 = p[(z + 3) * zstride];
      sum += a0;
      sum += a1;
      sum += a2;
      sum += a3;
    }
    for (; z < splits; ++z) sum += p[z * zstride];
    sS[i] = sum;
  }
  __syncthreads();
  const uint32_t col = c0 + tid;
  if (col >= n) return;
  const uint32_t jl = tid / G, tc = col % G;
  const float* b_book = static_cast<const float*>(o.in[3]);
  float y = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) y = fmaf(sS[16 * jl + e], b_book[e * G + tc], y);
  if (!AD) y = ldexpf(y, -shift);
  static_cast<float*>(o.out)[uint64_t(r) * n + col] = y;
  if (__any(!finite_f32(y)) && lane == 0) atomicOr(o.status, 1u);
}

// ---- dense activations on large grids: bf16 planes -------------------------
// Splitting x as it is read repeats the split for every column block that
// reads the same rows (56 of them at config 4), and that VALU work outweighs
// the MFMAs. So a pre-pass splits every value once into three bf16 planes
// (t = hi, mid, lo; rows m .. mp - 1 zero), stored in the MFMA's fragment
// order: for 32-row block rb and 16-step s of k, one 1 KiB chunk per term in
// which lane l = (r % 32) + 32 h holds the 8 values of row 32 rb + (r % 32)
// at inner indices 16 s + 8 h .. + 7. A wave's fragment is then one
// contiguous 1 KiB read (row-major planes would touch 32 cache lines for 32
// bytes each, four times the bytes through L2).
__device__ __forceinline__ uint64_t plane_chunk(uint32_t rb, uint32_t s, uint32_t steps) {
  return (uint64_t(rb) * steps + s) * 512;  // in bf16 elements: 64 lanes x 8
}

// One thread per destination lane: chunk i (of mp / 32 * steps) and lane l.
__global__ __launch_bounds__(256) void k_split_planes(const float* __restrict__ x,
                                                      __bf16* __restrict__ planes, uint32_t m,
                                                      uint32_t mp, uint32_t k) {
  const uint32_t steps = k / 16;
  const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= uint64_t(mp) * steps * 2) return;  // (mp / 32) * steps chunks of 64 lanes
  const uint32_t lane = uint32_t(i % 64);
  const uint64_t chunk = i / 64;
  const uint32_t rb = uint32_t(chunk / steps), s = uint32_t(chunk % steps);
  const uint32_t r = 32 * rb + lane % 32, kk = 16 * s + 8 * (lane / 32);
  float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b = a;
  if (r < m) {
    const float4* p = reinterpret_cast<const float4*>(x + uint64_t(r) * k + kk);
    a = p[0];
    b = p[1];
  }
  bf16x8 d[3];
  split_bf16x3(a, b, false, d);
  const uint64_t plane = uint64_t(mp) * k, at = plane_chunk(rb, s, steps) + 8 * lane;
#pragma unroll
  for (int t = 0; t < kOHTerms; ++t) *reinterpret_cast<bf16x8*>(planes + t * plane + at) = d[t];
}

// grid: n / (8 G) word columns of B x mp / (128 X) row blocks, one
// dimension. Blocks go to the 8 XCDs in turn (block b to XCD b mod 8), so when
// the row blocks are a multiple of 8, block b takes row block b mod 8 + 8 j and
// word column i mod C (i = b / 8, j = i / C): every block of an XCD reads its
// eighth of the planes, which that XCD's L2 then serves to all the columns
// (config 4: 8 row blocks of 256 rows, 56 columns). Otherwise columns vary
// fastest. The block's 4 waves
// stack along rows: wave w takes rows 32 X w .. 32 X w + 32 X - 1 of the
// block's 128 X and all 8 groups of word column q (128 S columns, four 32 x 32
// blocks y), so each A fragment read from the planes feeds four MFMAs per
// term and each one-hot fragment X. A fragments are read one step ahead, B's
// nibble-column words two steps ahead in a ring of four. The epilogue is that
// of k_onehot_mfma: S through LDS, 32 rows at a time, then the 16-term
// products with C_B (no scale: the planes hold x itself).
// Requires k % 16 == 0, n % (8 G) == 0, mp a multiple of 128 X; one instance.
constexpr uint32_t kPlaneSRow = 132;  // sS row stride in floats: the two row halves of
                                      // an accumulator write land 16 banks apart
template <int G, int X>
__global__ __launch_bounds__(kOHThreads, 2) void k_onehot_planes(
    Operands o, uint32_t m, uint32_t n, uint32_t k, uint32_t mp, const uint32_t* __restrict__ nc,
    const __bf16* __restrict__ planes) {
  static_assert(G == 8 || G == 16 || G == 32, "groups of B");
  static_assert(X == 1 || X == 2, "row blocks per wave");
  __shared__ __align__(16) float sS[4][32][kPlaneSRow];
  __shared__ float sbook[16 * G];
  const uint32_t tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const uint32_t i32 = lane % 32, h = lane / 32;
  const uint32_t cols = n / (8 * G), rblocks = mp / (128 * X), bid = blockIdx.x;
  uint32_t q, rb;
  if (rblocks % 8 == 0) {
    const uint32_t i = bid / 8;
    rb = bid % 8 + 8 * (i / cols);
    q = i % cols;
  } else {
    rb = bid / cols;
    q = bid % cols;
  }
  const uint32_t row0 = rb * (128 * X) + 32 * X * wave;
  const float* b_book = static_cast<const float*>(o.in[3]);
  float* out = static_cast<float*>(o.out);
  bool bad = false;
  for (uint32_t i = tid; i < 16 * G; i += kOHThreads) {
    const float b = b_book[i];
    sbook[i] = b;
    if (bid == 0) bad |= !finite_f32(b);
  }
  // the lane's S columns: code i32 % 16 of groups 8 q + 2 y + i32 / 16
  const uint32_t ee = (i32 % 16) * 0x11111111u;
  const uint32_t k8 = k / 8;
  const uint32_t* ncl = nc + uint64_t(8 * q + i32 / 16) * k8 + h;  // group of y: + 2 y k8
  // the lane's 16 bytes of each fragment chunk; block x: + x steps chunks,
  // step s: + s chunks, term t: + t planes
  const uint64_t plane = uint64_t(mp) * k;
  const uint32_t steps = k / 16;
  const __bf16* pa = planes + plane_chunk(row0 / 32, 0, steps) + 8 * lane;
  const uint64_t xstride = plane_chunk(1, 0, steps);

  f32x16 acc[X][4];
#pragma unroll
  for (int x = 0; x < X; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y) acc[x][y] = (f32x16)0.0f;
  // Loads as in k_onehot_mfma: unconditional (indices clamped to the last
  // step), and only the last 0-3 steps, past the whole groups of four, are
  // taken outside the unrolled loop. B's nibble-column words are read three
  // steps ahead (a ring of four), A's fragments one step ahead, and the
  // one-hot fragments of the next step are built between this step's MFMAs,
  // so their VALU work runs while the matrix core is busy.
  const uint32_t klast = k - 16;
  uint32_t wb[4][4];
  bf16x8 fa[2][X][kOHTerms];
  bf16x8 bf[2][4];
#pragma unroll
  for (int y = 0; y < 4; ++y) {
#pragma unroll
    for (uint32_t s = 0; s < 3; ++s) wb[s][y] = ncl[2 * y * k8 + (16 * s < k ? 2 * s : 0)];
    bf[0][y] = one_hot_column(wb[0][y], ee);
  }
#pragma unroll
  for (int x = 0; x < X; ++x)
#pragma unroll
    for (int t = 0; t < kOHTerms; ++t)
      fa[0][x][t] = *reinterpret_cast<const bf16x8*>(pa + t * plane + x * xstride);
  auto step = [&](uint32_t kk0, uint32_t s) __attribute__((always_inline)) {
    const uint32_t kb = kk0 + 48 < klast ? kk0 + 48 : klast;
#pragma unroll
    for (int y = 0; y < 4; ++y) wb[(s + 3) % 4][y] = ncl[2 * y * k8 + kb / 8];
    const uint32_t kn = kk0 + 16 < klast ? kk0 + 16 : klast;
#pragma unroll
    for (int x = 0; x < X; ++x)
#pragma unroll
      for (int t = 0; t < kOHTerms; ++t)
        fa[(s + 1) % 2][x][t] = *reinterpret_cast<const bf16x8*>(
            pa + t * plane + x * xstride + plane_chunk(0, kn / 16, steps));
    // keep the loads for later steps ahead of this step's work: left to
    // itself the scheduler sinks them next to their use and waits on them
    __builtin_amdgcn_sched_barrier(0);
    // terms smallest first: lo, mid, hi
#pragma unroll
    for (int t = kOHTerms - 1; t >= 0; --t)
#pragma unroll
      for (int x = 0; x < X; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y)
          acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[s % 2][x][t], bf[s % 2][y],
                                                              acc[x][y], 0, 0, 0);
#pragma unroll
    for (int y = 0; y < 4; ++y) bf[(s + 1) % 2][y] = one_hot_column(wb[(s + 1) % 4][y], ee);
    // interleave: one MFMA, then up to four VALU instructions
#pragma unroll
    for (int i = 0; i < kOHTerms * X * 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  const uint32_t four = steps / 4 * 4;
  for (uint32_t k0 = 0; k0 < 16 * four; k0 += 64) {
#pragma unroll
    for (uint32_t s = 0; s < 4; ++s) step(k0 + 16 * s, s);
  }
#pragma unroll
  for (uint32_t s = 0; s < 3; ++s)
    if (four + s < steps) step(16 * (four + s), s);

  // ---- S to LDS one 32-row block at a time (item t of acc[x][y] is row
  // (t % 4) + 4 h + 8 (t / 4), column 32 y + i32), then
  // y[r][G j + t] = sum_e S[r][(j, e)] C_B[e][t], e ascending; a lane's t is
  // fixed (64 is a multiple of G)
  __syncthreads();  // sbook
  const uint32_t tc = lane % G;
  float cb[16];
#pragma unroll
  for (int f = 0; f < 16; ++f) cb[f] = sbook[f * G + tc];
#pragma unroll
  for (int x = 0; x < X; ++x) {
    if (x) __syncthreads();  // the previous block's S has been read
#pragma unroll
    for (int y = 0; y < 4; ++y)
#pragma unroll
      for (int t = 0; t < 16; ++t)
        sS[wave][(t % 4) + 4 * h + 8 * (t / 4)][32 * y + i32] = acc[x][y][t];
    __syncthreads();
    for (uint32_t idx = lane; idx < 32 * 8 * G; idx += 64) {
      const uint32_t row = idx / (8 * G), j = (idx / G) % 8;
      const uint32_t r = row0 + 32 * x + row;
      if (r >= m) break;
      const float4* sp = reinterpret_cast<const float4*>(&sS[wave][row][16 * j]);
      const float4 s0 = sp[0], s1 = sp[1], s2 = sp[2], s3 = sp[3];
      float yv = 0.0f;
      yv = fmaf(s0.x, cb[0], yv);
      yv = fmaf(s0.y, cb[1], yv);
      yv = fmaf(s0.z, cb[2], yv);
      yv = fmaf(s0.w, cb[3], yv);
      yv = fmaf(s1.x, cb[4], yv);
      yv = fmaf(s1.y, cb[5], yv);
      yv = fmaf(s1.z, cb[6], yv);
      yv = fmaf(s1.w, cb[7], yv);
      yv = fmaf(s2.x, cb[8], yv);
      yv = fmaf(s2.y, cb[9], yv);
      yv = fmaf(s2.z, cb[10], yv);
      yv = fmaf(s2.w, cb[11], yv);
      yv = fmaf(s3.x, cb[12], yv);
      yv = fmaf(s3.y, cb[13], yv);
      yv = fmaf(s3.z, cb[14], yv);
      yv = fmaf(s3.w, cb[15], yv);
      out[uint64_t(r) * n + (8 * q + j) * G + tc] = yv;
      bad |= !finite_f32(yv);
    }
  }
  if (__any(bad) && lane == 0) atomicOr(o.status, 1u);
}

// Dense activations take the bf16 planes (k_onehot_planes) once the grid of
// 128 X-row blocks has kOHBigGrid blocks: X = 2 (256 rows) where that grid is
// large enough, else X = 1 (128 rows); smaller grids split x as they read it
// (k_onehot_mfma with 64-row blocks), where the pre-pass would not pay.
uint32_t dense_planes_x(uint32_t m, uint32_t n, uint32_t group) {
  const uint64_t cols = n / (8 * group);
  if (cols * ((m + 255) / 256) >= kOHBigGrid) return 2;
  if (cols * ((m + 127) / 128) >= kOHBigGrid) return 1;
  return 0;
}

uint32_t planes_rows(uint32_t m, uint32_t px) { return (m + 128 * px - 1) / (128 * px) * (128 * px); }

size_t nc_bytes(uint32_t n, uint32_t k, uint32_t group) {
  return (size_t(n / group) * (k / 8) * 4 + 255) / 256 * 256;
}

uint64_t big_grid(uint32_t m, uint32_t n, uint32_t group) {
  return uint64_t(n / (8 * group)) * ((m + 255) / 256);
}

// Split k for the 64-row grid (packed A below kOHBigGrid blocks of 256 rows,
// dense A below the planes' grid): with fewer than kOHSplitBlocks blocks the
// chip idles while each block walks all of k, so k is cut into `count` parts
// of `kpart` inner indices (whole passes of 8 G, at least two each) run as
// blocks z of a 3D grid, their partial S in the workspace (at most
// kOHPartialMax bytes) and k_onehot_finish adding them.
constexpr uint32_t kOHSplitBlocks = 256;
constexpr size_t kOHPartialMax = size_t(8) << 20;

struct Split {
  uint32_t count, kpart;
};

Split onehot_split(uint32_t m, uint32_t n, uint32_t k, uint32_t group, bool dense) {
  const bool x1 = dense ? dense_planes_x(m, n, group) == 0 : big_grid(m, n, group) < kOHBigGrid;
  const uint64_t blocks = uint64_t(n / (8 * group)) * ((m + 63) / 64);
  const uint32_t pass = 8 * group, passes = (k + pass - 1) / pass;
  const size_t per_split = size_t(m) * (16 * (n / group)) * sizeof(float);
  uint64_t want = (kOHSplitBlocks + blocks - 1) / blocks;
  if (want > passes / 2) want = passes / 2;
  if (want > kOHPartialMax / per_split) want = kOHPartialMax / per_split;
  if (!x1 || want < 2) return {1, k};
  const uint32_t per = (passes + uint32_t(want) - 1) / uint32_t(want);  // passes per split
  return {(passes + per - 1) / per, per * pass};
}

// The mixed 256/192-row tiling of k_onehot_mixed: per word column, a 256-row
// and b 192-row blocks with 4 a + 3 b = m / 64, two column classes, and
// kOHSlots / 2 blocks of each size in all. False when the grid has no tail or
// no such split exists (m not a multiple of 64, or no two classes fit).
constexpr uint32_t kOHSlots = 512;  // blocks the chip holds at once: two per compute unit

bool onehot_mixed_plan(uint32_t m, uint32_t n, uint32_t group, OHMixed* out) {
  const uint32_t cols = n / (8 * group);
  const uint64_t tiles = big_grid(m, n, group);
  if (group == 8 || tiles < kOHBigGrid || tiles >= kOHSlots || m % 64 != 0) return false;
  const uint32_t half = kOHSlots / 2, u = m / 64;
  for (uint32_t a1 = 0; 4 * a1 <= u; ++a1) {
    if ((u - 4 * a1) % 3 != 0) continue;
    const uint32_t b1 = (u - 4 * a1) / 3;
    for (uint32_t a2 = 0; 4 * a2 <= u; ++a2) {
      if ((u - 4 * a2) % 3 != 0) continue;
      const uint32_t b2 = (u - 4 * a2) / 3;
      for (uint32_t c1 = 0; c1 <= cols; ++c1) {
        const uint32_t c2 = cols - c1;
        if (c1 * a1 + c2 * a2 == half && c1 * b1 + c2 * b2 == half) {
          *out = OHMixed{c1, a1, b1, a2, b2};
          return true;
        }
      }
    }
  }
  return false;
}

}  // namespace

// From kOneHotMinRows rows of A always; from 8 rows when B holds at least
// 2^20 values (smaller products keep the bit-exact general kernel or the
// GEMVs). Small grids split k, so the path's time hardly grows with m below 64
// rows, where the GEMVs' grows with every row (one product, µs, one-hot against
// the automatic choice before): 8 x 4096 x 14336 g16 36 against 58 (gemv-rows),
// 8 x 4096^2 g16 17.5 against 21.4 (gemv-direct), 9 x 4096^2 g16 18 against 62,
// 48 x 4096 x 14336 g16 40 against 346; at 4 rows the GEMVs still win 2 of 4
// shapes.
bool onehot_applies(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                    uint32_t count) {
  if (count != 1 || flags != 0 || (group != 16 && group != 32) || n % (8 * group) != 0 ||
      k % 16 != 0 || k % group != 0)
    return false;
  if (m >= kOneHotMinRows) return true;
  return m >= kOneHotMinRowsSmall && uint64_t(n) * k >= (uint64_t(1) << 20);
}

// Workspace: B's nibble columns, then the planes (dense A on a large grid) or
// the split partial sums.
size_t onehot_workspace_bytes(uint32_t m, uint32_t n, uint32_t k, uint32_t group) {
  const Split sp = onehot_split(m, n, k, group, false);
  if (sp.count == 1) return size_t(n / group) * (k / 8) * 4;
  return nc_bytes(n, k, group) + size_t(sp.count) * m * (16 * (n / group)) * sizeof(float);
}

size_t onehot_dense_workspace_bytes(uint32_t m, uint32_t n, uint32_t k, uint32_t group) {
  const uint32_t px = dense_planes_x(m, n, group);
  if (px != 0)
    return nc_bytes(n, k, group) + size_t(kOHTerms) * planes_rows(m, px) * k * sizeof(__bf16);
  const Split sp = onehot_split(m, n, k, group, true);
  if (sp.count == 1) return size_t(n / group) * (k / 8) * 4;
  return nc_bytes(n, k, group) + size_t(sp.count) * m * (16 * (n / group)) * sizeof(float);
}

namespace {

template <int G, int X, bool AD>
void launch_onehot_x(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                     const uint32_t* nc, float* partial) {
  const Split sp = X == 1 ? onehot_split(m, n, k, G, AD) : Split{1, k};
  dim3 grid(n / (8 * G), (m + 64 * X - 1) / (64 * X), sp.count);
  k_onehot_mfma<G, X, AD><<<grid, kOHThreads, 0, s>>>(o, m, n, k, nc, sp.kpart,
                                                      sp.count > 1 ? partial : nullptr);
  if (sp.count > 1)
    k_onehot_finish<G, AD><<<dim3((n + 255) / 256, m), 256, 0, s>>>(o, m, n, sp.count, partial);
}

template <int G>
void launch_planes(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                   uint32_t px, const uint32_t* nc, __bf16* planes) {
  const uint32_t mp = planes_rows(m, px);
  const uint64_t lanes = uint64_t(mp) * (k / 16) * 2;  // 64 lanes per (32 rows, 16-step)
  k_split_planes<<<dim3(uint32_t((lanes + 255) / 256)), 256, 0, s>>>(
      static_cast<const float*>(o.in[0]), planes, m, mp, k);
  dim3 grid((n / (8 * G)) * (mp / (128 * px)));
  if (px == 2) k_onehot_planes<G, 2><<<grid, kOHThreads, 0, s>>>(o, m, n, k, mp, nc, planes);
  else k_onehot_planes<G, 1><<<grid, kOHThreads, 0, s>>>(o, m, n, k, mp, nc, planes);
}

template <int G>
void launch_onehot_g(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                     bool dense, const uint32_t* nc, void* rest) {
  float* partial = static_cast<float*>(rest);
  if (dense) {
    if (const uint32_t px = dense_planes_x(m, n, G))
      launch_planes<G>(s, o, m, n, k, px, nc, static_cast<__bf16*>(rest));
    else launch_onehot_x<G, 1, true>(s, o, m, n, k, nc, partial);
  } else if (big_grid(m, n, G) >= kOHBigGrid) {
    OHMixed mx;
    if (onehot_mixed_plan(m, n, G, &mx))
      k_onehot_mixed<G><<<dim3(kOHSlots), kOHThreads, 0, s>>>(o, m, n, k, nc, mx);
    else launch_onehot_x<G, 4, false>(s, o, m, n, k, nc, nullptr);
  } else {
    launch_onehot_x<G, 1, false>(s, o, m, n, k, nc, partial);
  }
}

// Group 8 is admitted for dense activations only (packed A's 16-steps of k
// would straddle its groups).
template <>
void launch_onehot_g<8>(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                        bool dense, const uint32_t* nc, void* rest) {
  (void)dense;
  if (const uint32_t px = dense_planes_x(m, n, 8))
    launch_planes<8>(s, o, m, n, k, px, nc, static_cast<__bf16*>(rest));
  else launch_onehot_x<8, 1, true>(s, o, m, n, k, nc, static_cast<float*>(rest));
}

}  // namespace

// Dense activations (no A groups to straddle, so group 8 as well): from 64
// rows, and from 9 with B of at least 2^20 values. x is split into three bf16
// terms as it is read, VALU work that the packed path's table reads do not
// have, so at 8 rows the GEMVs still win some shapes (µs, gemv-rows against
// one-hot): 8 x 8192^2 g16 47.7 against 55.8, 8 x 4096 x 14336 g16 55.0
// against 49.9.
bool onehot_applies_dense(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                          uint32_t count) {
  if (count != 1 || flags != 0 || n % (8 * group) != 0 || k % 16 != 0) return false;
  if (m >= kOneHotMinRows) return true;
  return m >= kOneHotMinRowsDense && uint64_t(n) * k >= (uint64_t(1) << 20);
}

hipError_t launch_onehot(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                         uint32_t group, bool dense, void* workspace) {
  const uint32_t rw = n / (8 * group);
  uint32_t* nc = static_cast<uint32_t*>(workspace);
  dim3 ngrid((rw + kNCCols - 1) / kNCCols, (k + kNCRows - 1) / kNCRows);
  k_nibble_columns<<<ngrid, 256, 0, s>>>(static_cast<const uint32_t*>(o.in[2]), nc, k, rw);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  void* rest = static_cast<char*>(workspace) + nc_bytes(n, k, group);  // planes or partial sums
  if (group == 8) launch_onehot_g<8>(s, o, m, n, k, dense, nc, rest);
  else if (group == 16) launch_onehot_g<16>(s, o, m, n, k, dense, nc, rest);
  else launch_onehot_g<32>(s, o, m, n, k, dense, nc, rest);
  return hipGetLastError();
}

}  // namespace ackvq
