// Large packed products whose operands are both grouped along the inner
// dimension, on gfx950 matrix cores: "gram-mfma".
//
// With B stored (n, k) (op 2, flags 2 of
// src/alelyon_compute_kit/_kit/kernels/vq4.comp:165-176 -- the dY . W^T of a
// backward pass) and k a multiple of the group G, inner index kk = j*G + t
// lies in group j of A's row r and of B's row c, so
//   C[r][c] = sum_j sum_t C_A[a(r,j)][t] * C_B[b(c,j)][t]
//           = sum_j Gram[a(r,j)][b(c,j)],   Gram = C_A . C_B^T  (16 x 16).
// That is a GEMM with inner dimension 16 * k / G:
//   C = P . Q,  P[r][(j,e)] = [a(r,j) == e],  Q[(j,e)][c] = Gram[e][b(c,j)],
// and it runs on v_mfma_f32_32x32x16_bf16 with one 16-step of K per group j:
// P is a one-hot row (exact in bf16), and Q is Gram scaled by a power of two
// and split into three bf16 terms hi + mid + lo (24 significant bits with
// FP32's exponent range: every FP32 Gram entry down to 2^-118 of the largest
// is carried exactly, the last term staying a normal bf16), so each j costs
// three MFMAs per 32 x 32 output
// block and the accumulation is FP32. Neither operand is decoded:
// P's fragments are read from a 768-byte LDS table of the one-hot rows
// addressed by A's nibble, Q's from a 1.5 KiB LDS table addressed by B's.
//
// The sum order differs from the shader's sequential one; results agree to
// FP32 rounding (k/G FP32 accumulations of exact Gram entries).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "kernels.hpp"

namespace ackvq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kGramThreads = 256;  // 4 waves, 2 x 2 over the block tile
constexpr uint32_t kWaveTile = 64;      // each wave: 64 rows x 64 columns (2 x 2 MFMA blocks)
constexpr uint32_t kBlockTile = 128;

__device__ __forceinline__ bool finite_f32(float x) { return fabsf(x) <= FLT_MAX; }

template <typename T>
__device__ __forceinline__ const T* item_ptr(const void* base, uint64_t stride, uint32_t item) {
  return reinterpret_cast<const T*>(static_cast<const char*>(base) + stride * item);
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

// One-hot MFMA A operand: this lane holds K entries 8h .. 8h+7 of its row;
// d = code - 8h selects the entry set to 1.0 (none when d is outside 0..7).
__device__ __forceinline__ bf16x8 one_hot(uint32_t d) {
  const uint32_t one = (d & 1u) ? 0x3F800000u : 0x00003F80u;  // bf16 1.0 in the low or high half
  const uint32_t pair = d >> 1;
  u32x4 v;
  v.x = pair == 0 ? one : 0u;
  v.y = pair == 1 ? one : 0u;
  v.z = pair == 2 ? one : 0u;
  v.w = pair == 3 ? one : 0u;
  return __builtin_bit_cast(bf16x8, v);
}

constexpr int kGramTerms = 3;  // bf16 terms of each scaled Gram entry

struct GramTile {
  f32x16 acc[2][2];
};

// One group j: two one-hot A fragments (rows) and hi, mid and lo B fragments
// for two column blocks, all from LDS tables, then twelve MFMAs. sel0/sel1 are
// the lanes' one-hot table bases (16 h for the lane's half h of K, 32 for a
// row past the matrix, whose entries are empty), OR-ed with the A nibble.
__device__ __forceinline__ void gram_step(GramTile& t, uint32_t aw0, uint32_t aw1, uint32_t bw0,
                                          uint32_t bw1, uint32_t jj, uint32_t sel0, uint32_t sel1,
                                          const char* tab_lane, const char* lut) {
  bf16x8 af[2];
  af[0] = *reinterpret_cast<const bf16x8*>(lut + 16 * (__builtin_amdgcn_ubfe(aw0, 4 * jj, 4) | sel0));
  af[1] = *reinterpret_cast<const bf16x8*>(lut + 16 * (__builtin_amdgcn_ubfe(aw1, 4 * jj, 4) | sel1));
  bf16x8 bf[2][kGramTerms];
  const char* p0 = tab_lane + 16 * __builtin_amdgcn_ubfe(bw0, 4 * jj, 4);
  const char* p1 = tab_lane + 16 * __builtin_amdgcn_ubfe(bw1, 4 * jj, 4);
#pragma unroll
  for (int s = 0; s < kGramTerms; ++s) {
    bf[0][s] = *reinterpret_cast<const bf16x8*>(p0 + 512 * s);
    bf[1][s] = *reinterpret_cast<const bf16x8*>(p1 + 512 * s);
  }
#pragma unroll
  for (int s = 0; s < kGramTerms; ++s)
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y)
        t.acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[x], bf[y][s], t.acc[x][y], 0, 0, 0);
}

// grid: (ceil(n / 128), ceil(m / 128), instances). Requires k % G == 0.
template <int G>
__global__ __launch_bounds__(kGramThreads, 2) void k_gram_mfma(Operands o, uint32_t m, uint32_t n,
                                                               uint32_t k) {
  __shared__ float sa[16 * G];
  __shared__ float sb[16 * G];
  // [term][A code / 8][B code][A code % 8], scaled Gram: a lane reads the 8
  // entries of its half (h = A code / 8) for its column's B code, and for one
  // half the 16 B codes' 16-byte rows fill the 64 banks once, so the 16 lanes
  // of a pass (one h) never conflict (equal codes broadcast)
  __shared__ __align__(16) __bf16 tab[kGramTerms][2][16][8];
  __shared__ float sred[kGramThreads / 64];
  // one-hot A fragments: entry 16 h + code holds one_hot(code - 8 h), entries
  // 32..47 (dead rows) are empty
  __shared__ __align__(16) u32x4 ohlut[48];
  const uint32_t J = k / G;
  const uint32_t tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const uint32_t i32 = lane % 32, h = lane / 32;
  const uint32_t row0 = blockIdx.y * kBlockTile + (wave / 2) * kWaveTile;
  const uint32_t col0 = blockIdx.x * kBlockTile + (wave % 2) * kWaveTile;
  const uint64_t a_last = (uint64_t(m) * J + 7) / 8 - 1;
  const uint64_t b_last = (uint64_t(n) * J + 7) / 8 - 1;
  // Rows and columns past the matrix read the last row's (column's) codes;
  // a dead row's one-hot is forced empty, a dead column is never stored.
  uint64_t av[2], bv[2];
  uint32_t sel[2];
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    const uint32_t r = row0 + 32 * x + i32, c = col0 + 32 * x + i32;
    av[x] = uint64_t(r < m ? r : m - 1) * J;
    bv[x] = uint64_t(c < n ? c : n - 1) * J;
    sel[x] = r < m ? 16u * h : 32u;  // the lane's one-hot table base
  }
  if (tid < 48)
    ohlut[tid] = tid < 32 ? __builtin_bit_cast(u32x4, one_hot((tid % 16) - 8u * (tid / 16)))
                          : u32x4{0u, 0u, 0u, 0u};

  for (uint32_t item = blockIdx.z; item < o.count; item += gridDim.z) {
    const uint32_t* a_codes = item_ptr<uint32_t>(o.in[0], o.stride[0], item);
    const float* a_book = item_ptr<float>(o.in[1], o.stride[1], item);
    const uint32_t* b_codes = item_ptr<uint32_t>(o.in[2], o.stride[2], item);
    const float* b_book = item_ptr<float>(o.in[3], o.stride[3], item);
    float* out = reinterpret_cast<float*>(static_cast<char*>(o.out) + o.stride[4] * item);

    // ---- Gram table: entry (e, f) per thread, in float64, then scaled so
    // the largest magnitude is below 2^15 and split into bf16 hi + mid + lo
    // (each term the bf16 rounding of what the previous ones leave; the
    // differences are exact in FP32, and the last term holds the rest exactly).
    __syncthreads();  // the previous instance's table is no longer read
    for (uint32_t i = tid; i < 16 * G; i += kGramThreads) {
      sa[i] = a_book[i];
      sb[i] = b_book[i];
    }
    __syncthreads();
    bool bad = false;
    if (blockIdx.x == 0 && blockIdx.y == 0)
      for (uint32_t i = tid; i < 16 * G; i += kGramThreads)
        bad |= !finite_f32(sa[i]) || !finite_f32(sb[i]);
    const uint32_t e = tid / 16, f = tid % 16;
    double dot = 0.0;
#pragma unroll 8
    for (int t = 0; t < G; ++t) dot = fma(double(sa[e * G + t]), double(sb[f * G + t]), dot);
    const float gv = float(dot);
    bad |= !finite_f32(gv);
    float gmax = finite_f32(gv) ? fabsf(gv) : 0.0f;
    for (int off = 1; off < 64; off <<= 1) gmax = fmaxf(gmax, __shfl_xor(gmax, off));
    if (lane == 0) sred[wave] = gmax;
    __syncthreads();
    gmax = fmaxf(fmaxf(sred[0], sred[1]), fmaxf(sred[2], sred[3]));
    int shift = 0;
    if (gmax > 0.0f) {
      int ex;
      frexpf(gmax, &ex);  // gmax < 2^ex
      shift = 15 - ex;
      shift = shift < -126 ? -126 : (shift > 126 ? 126 : shift);
    }
    const float scaled = ldexpf(gv, shift);
    const __bf16 hi = __bf16(scaled);
    const float r1 = scaled - float(hi);
    const __bf16 mid = __bf16(r1);
    tab[0][e / 8][f][e % 8] = hi;
    tab[1][e / 8][f][e % 8] = mid;
    tab[2][e / 8][f][e % 8] = __bf16(r1 - float(mid));
    const float unscale = ldexpf(1.0f, -shift);
    __syncthreads();

    // ---- main loop: 8 groups per pass, code words prefetched one pass ahead
    GramTile tile;
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y) tile.acc[x][y] = (f32x16)0.0f;
    const char* tab_lane = reinterpret_cast<const char*>(&tab[0][0][0][0]) + 256 * h;
    uint32_t an0 = nibbles8(a_codes, av[0], a_last), an1 = nibbles8(a_codes, av[1], a_last);
    uint32_t bn0 = nibbles8(b_codes, bv[0], b_last), bn1 = nibbles8(b_codes, bv[1], b_last);
    const uint32_t full = J / 8 * 8;
    uint32_t j0 = 0;
    for (; j0 < full; j0 += 8) {
      const uint32_t aw0 = an0, aw1 = an1, bw0 = bn0, bw1 = bn1;
      if (j0 + 8 < J) {
        an0 = nibbles8(a_codes, av[0] + j0 + 8, a_last);
        an1 = nibbles8(a_codes, av[1] + j0 + 8, a_last);
        bn0 = nibbles8(b_codes, bv[0] + j0 + 8, b_last);
        bn1 = nibbles8(b_codes, bv[1] + j0 + 8, b_last);
      }
#pragma unroll
      for (uint32_t jj = 0; jj < 8; ++jj)
        gram_step(tile, aw0, aw1, bw0, bw1, jj, sel[0], sel[1], tab_lane,
                  reinterpret_cast<const char*>(ohlut));
    }
    for (uint32_t jj = 0; j0 + jj < J; ++jj)
      gram_step(tile, an0, an1, bn0, bn1, jj, sel[0], sel[1], tab_lane,
                reinterpret_cast<const char*>(ohlut));

    // ---- store: lane (column i32, half h), item t holds row (t%4) + 4h + 8(t/4)
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int y = 0; y < 2; ++y) {
        const uint32_t c = col0 + 32 * y + i32;
#pragma unroll
        for (int t = 0; t < 16; ++t) {
          const uint32_t r = row0 + 32 * x + (t % 4) + 4 * h + 8 * (t / 4);
          const float v = tile.acc[x][y][t] * unscale;
          if (r < m && c < n) {
            out[uint64_t(r) * n + c] = v;
            bad |= !finite_f32(v);
          }
        }
      }
    if (__any(bad) && lane == 0) atomicOr(o.status, 1u);
  }
}

}  // namespace

// Below kGramMinMacs the general kernel, bit-identical to the shader, is
// fast enough; `any_size` (the test policy) lifts the bound.
constexpr uint64_t kGramMinMacs = 1ull << 22;

bool gram_applies(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                  bool any_size) {
  return flags == 2 && k % group == 0 && (any_size || uint64_t(m) * n * k >= kGramMinMacs);
}

hipError_t launch_gram(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                       uint32_t group) {
  const uint32_t zc = o.count < 65535 ? o.count : 65535;
  dim3 grid((n + kBlockTile - 1) / kBlockTile, (m + kBlockTile - 1) / kBlockTile, zc);
  if (group == 8) k_gram_mfma<8><<<grid, kGramThreads, 0, s>>>(o, m, n, k);
  else if (group == 16) k_gram_mfma<16><<<grid, kGramThreads, 0, s>>>(o, m, n, k);
  else k_gram_mfma<32><<<grid, kGramThreads, 0, s>>>(o, m, n, k);
  return hipGetLastError();
}

}  // namespace ackvq
