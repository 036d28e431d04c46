// vq4/v1 codec kernels for gfx950: encode (op 0), decode (op 1), AdamW from
// four packed states (op 3), and the passes of the fused VQAdamW step.
//
// Numerics follow src/alelyon_compute_kit/_kit/kernels/vq4.comp exactly. The
// library is compiled with -ffp-contract=off, so every `a * b + c` below is a
// rounded multiply followed by a rounded add, as GLSL `precise` demands; FP32
// division and square root are IEEE correctly rounded.
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "fit_device.hpp"
#include "kernels.hpp"

namespace ackvq {
namespace {

constexpr int kThreads = 256;
constexpr uint32_t kMaxGridX = 16384;

__device__ __forceinline__ bool finite_f32(float x) { return fabsf(x) <= FLT_MAX; }

__device__ __forceinline__ uint32_t nibble(const uint32_t* codes, uint32_t vector) {
  return (codes[vector >> 3] >> ((vector & 7u) * 4u)) & 15u;
}

__device__ __forceinline__ uint32_t words_for(uint32_t values, uint32_t group) {
  uint32_t vectors = values / group + (values % group != 0);
  return vectors / 8 + (vectors % 8 != 0);
}

template <typename T>
__device__ __forceinline__ const T* item_ptr(const void* base, uint64_t stride, uint32_t item) {
  return reinterpret_cast<const T*>(static_cast<const char*>(base) + stride * item);
}
template <typename T>
__device__ __forceinline__ T* item_ptr_mut(void* base, uint64_t stride, uint32_t item) {
  return reinterpret_cast<T*>(static_cast<char*>(base) + stride * item);
}

// Status sweep over a codebook (vq4.comp:153-158): any nonfinite value sets
// bit 1. Run by one block per instance.
__device__ void sweep_book(const float* book, uint32_t values, uint32_t* status) {
  bool bad = false;
  for (uint32_t i = threadIdx.x; i < values; i += blockDim.x) bad |= !finite_f32(book[i]);
  if (__any(bad) && (threadIdx.x % warpSize) == 0) atomicOr(status, 1u);
}

// Argmin of vq4.comp:118-144 for one vector: for each code ascending, the
// FP32 distance accumulated as d = d + (x_j - c_j)^2 with every operation
// rounded, j ascending over the valid components; strict `<` keeps the
// lowest index; best starts at +inf, selected at 0. `bad` reports a
// nonfinite final distance (a nonfinite partial distance stays nonfinite
// when values and book are finite, so this equals the shader's per-step
// test; nonfinite values and books are reported by their own checks).
template <int G, bool Full>
__device__ __forceinline__ uint32_t argmin32(const float (&x)[G], uint32_t valid,
                                             const float* sbook, bool& bad) {
  float best = __int_as_float(0x7f800000);
  uint32_t selected = 0;
#pragma unroll 2
  for (uint32_t code = 0; code < 16; ++code) {
    const float* c = sbook + code * G;
    float d = 0.0f;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if (Full || uint32_t(j) < valid) {
        const float delta = x[j] - c[j];
        const float sq = delta * delta;
        d = d + sq;
      }
    }
    bad |= !finite_f32(d);
    if (d < best) {
      best = d;
      selected = code;
    }
  }
  return selected;
}

// Screen in front of argmin32 for whole vectors: it ranks the codes by
// A_c = |c|^2 - 2 x.c, one FMA per component from -2c and |c|^2 prepared in
// LDS, and proves when its best code is also the shader's. With X = |x|^2 and
// u = 2^-24, the shader's computed distance d_c lies within (G + 2) u D_c of
// the exact D_c <= 2 (X + |c|^2), and A_c within G u (X + 3.01 |c|^2) of
// D_c - X, so |A_c + X - d_c| <= 5.01 (G + 2) u (X + |c|^2). E below takes
// 8 (G + 2) u (xn + cmax), where xn and cmax (the largest |c|^2) are the FP32
// sums (relative error G u), which also covers the rounding of E and of the
// gap; 2^-140 bounds the absolute error that subnormal results add (2^-150
// per operation). If the runner-up's A exceeds the best's by more than 2E,
// then d(best) < d(c) for every other code: the best is the shader's strict
// argmin. The screen applies while the book is finite and xn, cmax < 2^120
// (then every d_c is finite, so no status bit is due); otherwise, or on a
// narrower gap, the caller runs argmin32.
struct Screen {
  const float* m2;  // -2 c, [16][G]
  const float* cn;  // |c|^2 per code, +inf where the entry is not finite
  float base;       // 2 E's part from the book: 16 (G + 2) u cmax + 2^-139
  bool on;
};

// -2 c and |c|^2 of `books` consecutive 16-entry books; then a barrier.
template <int G>
__device__ __forceinline__ void screen_prepare(const float* sbook, float* m2, float* cn,
                                               uint32_t books) {
  for (uint32_t i = threadIdx.x; i < books * 16 * G; i += blockDim.x) m2[i] = -2.0f * sbook[i];
  for (uint32_t t = threadIdx.x; t < books * 16; t += blockDim.x) {
    float n = 0.0f;
    bool ok = true;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const float c = sbook[t * G + j];
      ok &= finite_f32(c);
      n = fmaf(c, c, n);
    }
    cn[t] = ok ? n : __int_as_float(0x7f800000);
  }
}

template <int G>
__device__ __forceinline__ Screen screen_load(const float* m2, const float* cn) {
  float cmax = 0.0f;
#pragma unroll
  for (int t = 0; t < 16; ++t) cmax = fmaxf(cmax, cn[t]);
  constexpr float k2 = float(16 * (G + 2)) * 0x1p-24f;
  return Screen{m2, cn, fmaf(k2, cmax, 0x1p-139f), cmax < 0x1p120f};
}

// The screened code of a whole vector, or kNoScreen when argmin32 must decide.
constexpr uint32_t kNoScreen = 16;
template <int G>
__device__ __forceinline__ uint32_t argmin_screen(const float (&x)[G], const Screen& s) {
  constexpr float k2 = float(16 * (G + 2)) * 0x1p-24f;
  float xn = 0.0f;
#pragma unroll
  for (int j = 0; j < G; ++j) xn = fmaf(x[j], x[j], xn);
  float b1 = __int_as_float(0x7f800000), b2 = b1;
  uint32_t i1 = 0;
  // 32 book values in flight per step at any G (more spills the fused step's kernel)
#pragma unroll(32 / G)
  for (uint32_t code = 0; code < 16; ++code) {
    const float* c = s.m2 + code * G;
    float r = s.cn[code];
#pragma unroll
    for (int j = 0; j < G; ++j) r = fmaf(x[j], c[j], r);
    const bool lt = r < b1;
    b2 = __builtin_amdgcn_fmed3f(b1, b2, r);  // the runner-up (b1 <= b2)
    b1 = lt ? r : b1;
    i1 = lt ? code : i1;
  }
  const bool proven = s.on && xn < 0x1p120f && (b2 - b1) > fmaf(k2, xn, s.base);
  return proven ? i1 : kNoScreen;
}

// The same screen with the dot products on the matrix core, for a wave whose
// 64 vectors are whole: v_mfma_f32_16x16x4f32 takes A = -2 c (16 codes x 4
// components), B = x (4 components x 16 vectors) and C = |c|^2, so one chain of
// G / 4 instructions gives A_c for 16 codes of 16 vectors. Lane l feeds
// A[l % 16][l / 16] and B[l / 16][l % 16] and holds D[4 (l / 16) + r][l % 16];
// it loads components P (l / 16) .. P (l / 16) + P - 1 (P = G / 4) of vector
// l % 16 of each of the wave's four 16-vector sets, and instruction t of a
// chain takes component P k + t at row k of the product. A 4 x 4 transpose of
// 4-code blocks across the lane rows (v_permlane32_swap, then
// v_permlane16_swap) leaves lane l with all 16 A_c of vector l, which it ranks
// as argmin_screen does. Error: the matrix core's sum of 4 products and the
// accumulator is taken as within 8 u of the sum of their magnitudes (measured
// worst 3.4 u over 16,384 random tiles with spread exponents and cancellation;
// rounding each operation to nearest gives 5 u at most; subnormal operands and
// results measured exact). Over the chain that is 2 G u (X + 2 |c|^2), with G u
// |c|^2 more from |c|^2 itself, so |A_c + X - d_c| <= (7 G + 4) u (X + |c|^2),
// within the E of argmin_screen (8 (G + 2) u (xn + cmax)) at G = 8, 16 and 32.
typedef float F4 __attribute__((ext_vector_type(4)));  // 16-byte vector

template <int G>
struct MfmaScreen {
  float a[G / 4];  // -2 c[l % 16][(G / 4) (l / 16) + t]
  float cn[4];     // |c|^2 of codes 4 (l / 16) + r
};

template <int G>
__device__ __forceinline__ MfmaScreen<G> mfma_screen_load(const Screen& s) {
  constexpr int P = G / 4;
  const uint32_t lane = threadIdx.x % 64;
  MfmaScreen<G> ms;
#pragma unroll
  for (int t = 0; t < P; ++t) ms.a[t] = s.m2[(lane % 16) * G + P * (lane / 16) + t];
#pragma unroll
  for (int r = 0; r < 4; ++r) ms.cn[r] = s.cn[4 * (lane / 16) + r];
  return ms;
}

// Swaps lanes 32..63 of a with lanes 0..31 of b (W = 32), or rows 1 and 3 of a
// with rows 0 and 2 of b (W = 16).
template <int W>
__device__ __forceinline__ void lane_swap(float& a, float& b) {
  const auto r = W == 32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b),
                                                            false, false)
                         : __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b),
                                                            false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

typedef float F2 __attribute__((ext_vector_type(2)));

// Loads of x for the matrix-core screen: non-temporal at groups 8 and 16
// (every value is read once; measured 46.5 against 49.0 us at g16 on 2^26
// values, no change at g8) and the default policy at group 32 (56 against
// 62 us).
template <int G, typename V>
__device__ __forceinline__ V x_load(const float* p) {
  if (G == 32) return *reinterpret_cast<const V*>(p);
  return __builtin_nontemporal_load(reinterpret_cast<const V*>(p));
}

// A wave's 64 whole vectors as the lane feeds them to the matrix core:
// components P (l / 16) .. + P - 1 of vector 16 g + l % 16, g = 0..3 (x: the
// wave's first vector, 16-byte aligned at G >= 16, 8-byte at G = 8).
template <int G>
struct MfmaTile {
  float v[4][G / 4];
};

template <int G>
__device__ __forceinline__ MfmaTile<G> mfma_tile_load(const float* x) {
  constexpr int P = G / 4;
  const uint32_t lane = threadIdx.x % 64;
  MfmaTile<G> t;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float* p = x + (16 * g + lane % 16) * G + P * (lane / 16);
    if (P == 2) {
      const F2 v = x_load<G, F2>(p);
      t.v[g][0] = v.x;
      t.v[g][P - 1] = v.y;
    } else {
#pragma unroll
      for (int q = 0; q < P; q += 4) {
        const F4 v = x_load<G, F4>(p + q);
        t.v[g][q] = v.x;
        t.v[g][q + 1] = v.y;
        t.v[g][q + 2] = v.z;
        t.v[g][q + 3] = v.w;
      }
    }
  }
  return t;
}

// The screened code of the lane's vector of a loaded tile, or kNoScreen.
template <int G>
__device__ __forceinline__ uint32_t argmin_screen_mfma(const MfmaTile<G>& tile,
                                                       const MfmaScreen<G>& ms, const Screen& s) {
  constexpr int P = G / 4;
  constexpr float k2 = float(16 * (G + 2)) * 0x1p-24f;
  const auto& xv = tile.v;
  F4 acc[4];
  float xp[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    acc[g] = F4{ms.cn[0], ms.cn[1], ms.cn[2], ms.cn[3]};
    float n = 0.0f;
#pragma unroll
    for (int t = 0; t < P; ++t) {
      acc[g] = __builtin_amdgcn_mfma_f32_16x16x4f32(ms.a[t], xv[g][t], acc[g], 0, 0, 0);
      n = fmaf(xv[g][t], xv[g][t], n);
    }
    xp[g] = n;
  }
  // lane row k holds codes 4 k .. 4 k + 3 of set g in ac[g]; afterwards lane
  // row g holds codes 4 b .. 4 b + 3 of set g in ac[b] (and xp[b]: the
  // squares of component block b)
  float ac[4][4];
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int r = 0; r < 4; ++r) ac[g][r] = acc[g][r];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    lane_swap<32>(ac[0][r], ac[2][r]);
    lane_swap<32>(ac[1][r], ac[3][r]);
  }
  lane_swap<32>(xp[0], xp[2]);
  lane_swap<32>(xp[1], xp[3]);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    lane_swap<16>(ac[0][r], ac[1][r]);
    lane_swap<16>(ac[2][r], ac[3][r]);
  }
  lane_swap<16>(xp[0], xp[1]);
  lane_swap<16>(xp[2], xp[3]);
  const float xn = ((xp[0] + xp[1]) + xp[2]) + xp[3];
  float b1 = ac[0][0], b2 = __int_as_float(0x7f800000);
  uint32_t i1 = 0;
#pragma unroll
  for (uint32_t code = 1; code < 16; ++code) {
    const float r = ac[code / 4][code % 4];
    const bool lt = r < b1;
    b2 = __builtin_amdgcn_fmed3f(b1, b2, r);
    b1 = lt ? r : b1;
    i1 = lt ? code : i1;
  }
  const bool proven = s.on && xn < 0x1p120f && (b2 - b1) > fmaf(k2, xn, s.base);
  return proven ? i1 : kNoScreen;
}

// OR the nibbles of 8 consecutive lanes into lane (v % 8 == 0)'s word.
__device__ __forceinline__ uint32_t gather_word(uint32_t part) {
  part |= __shfl_xor(part, 1);
  part |= __shfl_xor(part, 2);
  part |= __shfl_xor(part, 4);
  return part;
}

// F4 (above) also carries streaming (non-temporal) stores. They speed up op
// 3's three output streams (~7 % on config 5) and slow down decode's one.

// ---- op 0: encode -------------------------------------------------------
// Waves per SIMD (blocks of 4 waves per compute unit) that each group's
// encode keeps resident: the most whose registers, two tiles of x among them,
// fit without spilling.
template <int G>
constexpr uint32_t kEncodeWaves = G == 8 ? 8 : G == 16 ? 5 : 4;
template <int G>
__global__ __launch_bounds__(kThreads, kEncodeWaves<G>) void k_encode(Operands o, uint32_t m) {
  const uint32_t item = blockIdx.y;
  const float* x = item_ptr<float>(o.in[0], o.stride[0], item);
  const float* book = item_ptr<float>(o.in[1], o.stride[1], item);
  uint32_t* out = item_ptr_mut<uint32_t>(o.out, o.stride[4], item);
  __shared__ float sbook[16 * G];
  __shared__ float sm2[16 * G];
  __shared__ float scn[16];
  for (uint32_t i = threadIdx.x; i < 16 * G; i += kThreads) sbook[i] = book[i];
  if (blockIdx.x == 0) sweep_book(book, 16 * G, o.status);
  __syncthreads();
  screen_prepare<G>(sbook, sm2, scn, 1);
  __syncthreads();
  const Screen screen = screen_load<G>(sm2, scn);
  const MfmaScreen<G> ms = mfma_screen_load<G>(screen);

  const uint32_t vectors = m / G + (m % G != 0);
  const uint32_t words = vectors / 8 + (vectors % 8 != 0);
  const bool aligned = ((reinterpret_cast<uintptr_t>(x) & 15u) == 0);
  bool bad = false;
  // A wave whose 64 vectors are whole takes the matrix-core screen, with the
  // next step's tile loaded before this step's is ranked.
  const uint32_t stride = gridDim.x * kThreads, wlane0 = threadIdx.x & ~63u;
  auto mfma_step = [&](uint32_t base) { return aligned && base + wlane0 + 64 <= m / G; };
  MfmaTile<G> next{};
  if (mfma_step(blockIdx.x * kThreads))
    next = mfma_tile_load<G>(x + uint64_t(blockIdx.x * kThreads + wlane0) * G);
  for (uint32_t base = blockIdx.x * kThreads; base < words * 8; base += stride) {
    const uint32_t v = base + threadIdx.x;
    uint32_t code = 0;
    if (mfma_step(base)) {
      const MfmaTile<G> tile = next;
      if (mfma_step(base + stride))
        next = mfma_tile_load<G>(x + uint64_t(base + stride + wlane0) * G);
      code = argmin_screen_mfma<G>(tile, ms, screen);
      if (code == kNoScreen) {
        float xv[G];
#pragma unroll
        for (int j = 0; j < G; j += 4) {
          const float4 q = *reinterpret_cast<const float4*>(x + uint64_t(v) * G + j);
          xv[j] = q.x; xv[j + 1] = q.y; xv[j + 2] = q.z; xv[j + 3] = q.w;
        }
#pragma unroll
        for (int j = 0; j < G; ++j) bad |= !finite_f32(xv[j]);
        code = argmin32<G, true>(xv, G, sbook, bad);
      }
    } else if (v < vectors) {
      const uint32_t start = v * G;
      const uint32_t valid = (m - start) < G ? (m - start) : G;
      float xv[G];
      if (valid == G) {
        if (aligned) {
#pragma unroll
          for (int j = 0; j < G; j += 4) {
            const float4 q = *reinterpret_cast<const float4*>(x + start + j);
            xv[j] = q.x; xv[j + 1] = q.y; xv[j + 2] = q.z; xv[j + 3] = q.w;
          }
        } else {
#pragma unroll
          for (int j = 0; j < G; ++j) xv[j] = x[start + j];
        }
#pragma unroll
        for (int j = 0; j < G; ++j) bad |= !finite_f32(xv[j]);
        code = argmin_screen<G>(xv, screen);
        if (code == kNoScreen) code = argmin32<G, true>(xv, G, sbook, bad);
      } else {
#pragma unroll
        for (int j = 0; j < G; ++j) {
          xv[j] = uint32_t(j) < valid ? x[start + j] : 0.0f;
          bad |= uint32_t(j) < valid && !finite_f32(xv[j]);
        }
        code = argmin32<G, false>(xv, valid, sbook, bad);
      }
    }
    const uint32_t word = gather_word(code << (4u * (v & 7u)));
    if ((v & 7u) == 0 && (v >> 3) < words) out[v >> 3] = word;
  }
  if (__any(bad) && (threadIdx.x % warpSize) == 0) atomicOr(o.status, 1u);
}

// ---- op 1: decode -------------------------------------------------------
// out[i] = book[code(i / G)][i % G], a bit copy. Each lane writes one
// 16-byte quad (G is a multiple of 4, so a quad never straddles vectors).
template <int G>
__global__ __launch_bounds__(kThreads) void k_decode(Operands o, uint32_t m) {
  const uint32_t item = blockIdx.y;
  const uint32_t* codes = item_ptr<uint32_t>(o.in[0], o.stride[0], item);
  const uint32_t* book = item_ptr<uint32_t>(o.in[1], o.stride[1], item);
  uint32_t* out = item_ptr_mut<uint32_t>(o.out, o.stride[4], item);
  __shared__ __align__(16) uint32_t sbook[16 * G];
  for (uint32_t i = threadIdx.x; i < 16 * G; i += kThreads) sbook[i] = book[i];
  if (blockIdx.x == 0) sweep_book(reinterpret_cast<const float*>(book), 16 * G, o.status);
  __syncthreads();
  const uint32_t quads = m / 4;
  if ((reinterpret_cast<uintptr_t>(out) & 15u) == 0) {
    for (uint32_t q = blockIdx.x * kThreads + threadIdx.x; q < quads; q += gridDim.x * kThreads) {
      const uint32_t e = q * 4;
      const uint32_t code = nibble(codes, e / G);
      *reinterpret_cast<uint4*>(out + e) = *reinterpret_cast<const uint4*>(sbook + code * G + e % G);
    }
  } else {
    for (uint32_t e = blockIdx.x * kThreads + threadIdx.x; e < quads * 4; e += gridDim.x * kThreads)
      out[e] = sbook[nibble(codes, e / G) * G + e % G];
  }
  if (blockIdx.x == 0 && threadIdx.x < m % 4) {
    const uint32_t e = quads * 4 + threadIdx.x;
    out[e] = sbook[nibble(codes, e / G) * G + e % G];
  }
}

// ---- op 3: AdamW ---------------------------------------------------------
struct Coeffs {
  float lr, beta1, beta2, eps, decay, c1, c2;
  uint32_t fail;  // 0 ok, 1 nonfinite coefficient, 4 outside its domain
};

// vq4.comp:81-91: every coefficient finite, then the domains.
__device__ __forceinline__ Coeffs load_coeffs(const float* b2) {
  Coeffs c;
  c.lr = b2[0]; c.beta1 = b2[1]; c.beta2 = b2[2]; c.eps = b2[3];
  c.decay = b2[4]; c.c1 = b2[5]; c.c2 = b2[6];
  c.fail = 0;
  for (int j = 0; j < 7; ++j)
    if (!finite_f32(b2[j])) c.fail = 1;
  if (c.fail == 0 &&
      (c.lr < 0.0f || c.beta1 < 0.0f || c.beta1 >= 1.0f || c.beta2 < 0.0f || c.beta2 >= 1.0f ||
       c.eps <= 0.0f || c.decay < 0.0f || c.c1 <= 0.0f || c.c1 > 1.0f || c.c2 <= 0.0f ||
       c.c2 > 1.0f))
    c.fail = 4;
  return c;
}

struct AdamwOut {
  float w, m, v;
  uint32_t flags;  // status bits this element raises
  bool write;      // the shader writes the element (vq4.comp:92-115)
};

// The terms of vq4.comp:94-104 that depend on fewer than all four states, one
// expression each, so that adamw_value and the fused encode's per-block tables
// form the same bits (every operation rounded: -ffp-contract=off, IEEE
// division and square root).
__device__ __forceinline__ float adamw_next_m(float moment, float gradient, const Coeffs& c) {
  return c.beta1 * moment + (1.0f - c.beta1) * gradient;
}
__device__ __forceinline__ float adamw_next_v(float variance, float gradient, const Coeffs& c) {
  return c.beta2 * variance + (1.0f - c.beta2) * (gradient * gradient);
}
// lr * M'/c1 (M'/c1 returned through `corrected`)
__device__ __forceinline__ float adamw_scaled(float next_m, const Coeffs& c, float& corrected) {
  corrected = next_m / c.c1;
  return c.lr * corrected;
}
// sqrt(V'/c2) + eps (V'/c2 returned through `corrected`)
__device__ __forceinline__ float adamw_denominator(float next_v, const Coeffs& c, float& corrected) {
  corrected = next_v / c.c2;
  return sqrtf(corrected) + c.eps;
}
__device__ __forceinline__ float adamw_decayed(float weight, const Coeffs& c) {
  return weight * (1.0f - c.lr * c.decay);
}

// adamw_value (vq4.comp:80-116) for one element given its four decoded state
// values. Branch-free: the arithmetic always runs (a GPU raises no traps) and
// the shader's early returns become the flags and the write decision.
__device__ __forceinline__ AdamwOut adamw_value(float weight, float moment, float variance,
                                                float gradient, const Coeffs& c) {
  // bitwise, not short-circuit: the checks compile to flag arithmetic, not branches
  const bool inputs_finite =
      finite_f32(weight) & finite_f32(moment) & finite_f32(variance) & finite_f32(gradient);
  const float next_m = adamw_next_m(moment, gradient, c);
  const float next_v = adamw_next_v(variance, gradient, c);
  float corrected_m, corrected_v;
  const float scaled = adamw_scaled(next_m, c, corrected_m);
  const float denominator = adamw_denominator(next_v, c, corrected_v);
  const float decayed = adamw_decayed(weight, c);
  const float next_w = decayed - scaled / denominator;
  const bool results_finite = finite_f32(next_m) & finite_f32(next_v) &
                              finite_f32(corrected_m) & finite_f32(corrected_v) &
                              finite_f32(denominator) & finite_f32(decayed) & finite_f32(next_w);
  AdamwOut r;
  r.write = inputs_finite & !(variance < 0.0f);
  r.flags = !inputs_finite ? 1u : (variance < 0.0f ? 4u : (results_finite ? 0u : 1u));
  // An element the shader leaves unwritten reads as zero to the fused passes.
  r.w = r.write ? next_w : 0.0f;
  r.m = r.write ? next_m : 0.0f;
  r.v = r.write ? next_v : 0.0f;
  return r;
}

// adamw_value's M' and V' only (the same expressions, so the same bits): they
// need none of the divisions and the square root behind W'.
__device__ __forceinline__ void adamw_moments(float weight, float moment, float variance,
                                              float gradient, const Coeffs& c, float& m, float& v) {
  const bool inputs_finite =
      finite_f32(weight) & finite_f32(moment) & finite_f32(variance) & finite_f32(gradient);
  const float next_m = adamw_next_m(moment, gradient, c);
  const float next_v = adamw_next_v(variance, gradient, c);
  const bool write = inputs_finite & !(variance < 0.0f);
  m = write ? next_m : 0.0f;
  v = write ? next_v : 0.0f;
}

// unpack_state (vq4.comp:74-78) then adamw_value for element i.
template <int G>
__device__ __forceinline__ AdamwOut adamw_element(const uint32_t* codes4, const float* books4,
                                                  uint32_t words, uint32_t i, const Coeffs& c) {
  const uint32_t vector = i / G;
  const uint32_t t = i % G;
  float s[4];
#pragma unroll
  for (int st = 0; st < 4; ++st)
    s[st] = books4[st * 16 * G + nibble(codes4 + st * words, vector) * G + t];
  return adamw_value(s[0], s[1], s[2], s[3], c);
}

// Op 3. The four books sit in LDS; with m a multiple of 4 and an aligned
// output each lane takes four consecutive elements (one vector's quad: G is a
// multiple of 4), reads each state's code word once and stores 16-byte
// quads; otherwise one element per lane.
template <int G>
__global__ __launch_bounds__(kThreads) void k_adamw(Operands o, uint32_t m) {
  const uint32_t item = blockIdx.y;
  const uint32_t* codes4 = item_ptr<uint32_t>(o.in[0], o.stride[0], item);
  const float* books4 = item_ptr<float>(o.in[1], o.stride[1], item);
  const float* coeff = item_ptr<float>(o.in[2], o.stride[2], item);
  float* out = item_ptr_mut<float>(o.out, o.stride[4], item);
  __shared__ __align__(16) float sbook[4 * 16 * G];
  for (uint32_t i = threadIdx.x; i < 4 * 16 * G; i += kThreads) sbook[i] = books4[i];
  if (blockIdx.x == 0) sweep_book(books4, 64 * G, o.status);
  __syncthreads();
  const Coeffs c = load_coeffs(coeff);
  if (c.fail) {
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(o.status, c.fail);
    return;
  }
  const uint32_t words = words_for(m, G);
  uint32_t flags = 0;
  if (m % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0) {
    const uint32_t quads = m / 4;
    for (uint32_t q = blockIdx.x * kThreads + threadIdx.x; q < quads; q += gridDim.x * kThreads) {
      const uint32_t i = q * 4;
      const uint32_t vector = i / G;
      const uint32_t t = i % G;
      float4 s[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const uint32_t code = nibble(codes4 + st * words, vector);
        s[st] = *reinterpret_cast<const float4*>(sbook + (st * 16 + code) * G + t);
      }
      const AdamwOut r0 = adamw_value(s[0].x, s[1].x, s[2].x, s[3].x, c);
      const AdamwOut r1 = adamw_value(s[0].y, s[1].y, s[2].y, s[3].y, c);
      const AdamwOut r2 = adamw_value(s[0].z, s[1].z, s[2].z, s[3].z, c);
      const AdamwOut r3 = adamw_value(s[0].w, s[1].w, s[2].w, s[3].w, c);
      flags |= r0.flags | r1.flags | r2.flags | r3.flags;
      if (r0.write && r1.write && r2.write && r3.write) {
        // streaming stores: the 3m outputs are written once and not read back here
        __builtin_nontemporal_store(F4{r0.w, r1.w, r2.w, r3.w}, reinterpret_cast<F4*>(out + i));
        __builtin_nontemporal_store(F4{r0.m, r1.m, r2.m, r3.m}, reinterpret_cast<F4*>(out + m + i));
        __builtin_nontemporal_store(F4{r0.v, r1.v, r2.v, r3.v}, reinterpret_cast<F4*>(out + 2 * m + i));
      } else {
        const AdamwOut rs[4] = {r0, r1, r2, r3};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (!rs[u].write) continue;
          out[i + u] = rs[u].w;
          out[m + i + u] = rs[u].m;
          out[2 * m + i + u] = rs[u].v;
        }
      }
    }
  } else {
    for (uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < m; i += gridDim.x * kThreads) {
      const AdamwOut r = adamw_element<G>(codes4, sbook, words, i, c);
      flags |= r.flags;
      if (r.write) {
        out[i] = r.w;
        out[m + i] = r.m;
        out[2 * m + i] = r.v;
      }
    }
  }
  // Wave-reduce the bits before touching the status word.
  for (int off = 1; off < warpSize; off <<= 1) flags |= __shfl_xor(flags, off);
  if (flags && (threadIdx.x % warpSize) == 0) atomicOr(o.status, flags);
}

// ---- fused VQAdamW passes -------------------------------------------------
// AdamW at fit_codebook's strided sample: sample vector e is complete vector
// linspace(0, m/G - 1, count)[e] (vq.py:206-207).
template <int G>
__global__ __launch_bounds__(kThreads) void k_adamw_gather(AdamwInputs in, uint32_t count,
                                                           float* out, uint32_t* changed,
                                                           uint32_t* status, float* fit_book,
                                                           uint32_t* fit_flags) {
  if (blockIdx.x == 0 && threadIdx.x == 0) *changed = 0;  // the encode pass counts into it
  if (blockIdx.x == 0) {  // the three fits' set-up: each starts from its state's book
    bool bad = false;
    for (uint32_t i = threadIdx.x; i < 3 * 16 * G; i += kThreads) {
      const float v = in.books4[i];
      bad = bad || !finite_f32(v);
      fit_book[i] = v;
    }
    if (threadIdx.x < 12) fit_flags[threadIdx.x] = 0;
    if (__any(bad) && (threadIdx.x % warpSize) == 0) atomicOr(status, 1u);
  }
  const Coeffs c = load_coeffs(in.coeffs);
  if (c.fail) {
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(status, c.fail);
    return;
  }
  const uint32_t words = words_for(in.m, G);
  const uint32_t total = count * G;
  const uint64_t complete = in.m / G;
  uint32_t flags = 0;
  for (uint32_t e = blockIdx.x * kThreads + threadIdx.x; e < total; e += gridDim.x * kThreads) {
    const uint32_t i = fitdev::linspace_at(complete, count, e / G) * G + e % G;
    const AdamwOut r = adamw_element<G>(in.codes4, in.books4, words, i, c);
    flags |= r.flags;
    out[e] = r.w;
    out[total + e] = r.m;
    out[2 * total + e] = r.v;
  }
  for (int off = 1; off < warpSize; off <<= 1) flags |= __shfl_xor(flags, off);
  if (flags && (threadIdx.x % warpSize) == 0) atomicOr(status, flags);
}

// The keep decision for vector x of state st whose current code is `code`:
// the bit of its first float64 minimum under the new book when that minimum
// may be a candidate entry, else 0. Only the candidate entries' bits are
// read. The vector's current code e0 certifies most vectors at once: a
// candidate c with d_c > d_e0 is not the first minimum. ||c - e0|| >
// 2 ||x - e0|| proves it without d_c (triangle inequality; the 2e-6 margin
// dwarfs the float64 rounding of every distance involved); otherwise d_c is
// computed. Any other outcome (a tie, a closer candidate, a non-finite
// distance) takes the full argmin. sbook: the three books in rows of G + 1
// doubles; sgap: ||c - e|| within each book; bk: state st's book, global.
template <int G>
__device__ __forceinline__ uint32_t keep_bit(const double (&x)[G], uint32_t st, uint32_t code,
                                             uint32_t cand, const double* sbook,
                                             const double* sgap, const double* __restrict__ bk) {
  constexpr uint32_t RS = G + 1;
  // the current code, or, when it is a candidate itself (as for a state whose
  // codes were all zero), the nearest entry by the first two components: any
  // entry closer than c certifies it
  uint32_t e0 = code;
  if (cand & (1u << e0)) {
    float best = __int_as_float(0x7f800000);
    for (uint32_t e = 0; e < 16; ++e) {
      if (cand & (1u << e)) continue;  // wave-uniform
      const float t0 = float(x[0]) - float(sbook[(st * 16 + e) * RS]);
      const float t1 = float(x[1]) - float(sbook[(st * 16 + e) * RS + 1]);
      const float dd = t0 * t0 + t1 * t1;
      if (dd < best) { best = dd; e0 = e; }
    }
  }
  const double d0 = fitdev::dist64<G>(x, sbook + (st * 16 + e0) * RS);
  bool full = !(d0 <= 1.7976931348623157e308);  // NaN or infinite
  const double reach = 2.000002 * sqrt(d0);
  const double* gap_e0 = sgap + (st * 16) * 16 + e0;
  for (uint32_t bits = cand; bits != 0; bits &= bits - 1) {
    const uint32_t cidx = __builtin_ctz(bits);
    if (gap_e0[cidx * 16] > reach) continue;
    const double dc = fitdev::dist64<G>(x, bk + cidx * G);
    full |= !(dc > d0);
  }
  return full ? 1u << fitdev::nearest64_uniform<G>(x, bk) : 0u;
}

// The fit's keep pass over the recomputed states: for each state whose fit
// set its keep-pass switch, which of its candidate entries (empty in the
// sample, not duplicates; the only bits the update reads) its complete
// vectors select under the float64 rule. AdamW is evaluated once per element
// for all three.
//
// Pair tables (G <= 16), as in k_adamw_encode: when the shader writes every
// element, M' and with it the keep decision of a vector's M state depend only
// on its (M, G) code pair, and V' on its (V, G) pair, so each block decides
// the 256 pairs of each once and a vector ORs two table words; W', when its
// keep pass is on, costs G divisions from the pairs' lr M'/c1 and
// sqrt(V'/c2) + eps.
template <int G>
__global__ __launch_bounds__(kThreads) void k_adamw_keep(AdamwInputs in, FitArgs a) {
  constexpr bool TAB = G <= 16;
  constexpr uint32_t TG = TAB ? G : 1;
  __shared__ float sfit[3 * 16 * G];
  __shared__ uint32_t scand[3];
  fitdev::keep_candidates<G>(a.book, a.flags, 3, sfit, scand);
  const uint32_t cand[3] = {scand[0], scand[1], scand[2]};
  const uint32_t active = (cand[0] ? 1u : 0u) | (cand[1] ? 2u : 0u) | (cand[2] ? 4u : 0u);
  if (active == 0) return;
  const double* __restrict__ book64 = a.book64;  // written by the assign pass
  // rows padded to G + 1 doubles, so per-lane row gathers spread over the banks
  constexpr uint32_t RS = G + 1;
  __shared__ double sbook[3 * 16 * RS];
  __shared__ double sgap[3 * 16 * 16];  // ||c - e|| between the entries of each state's book
  __shared__ float sold[4 * 16 * G];
  __shared__ float sscaled[256 * TG];        // lr M'/c1 at [16 c_M + c_G]
  __shared__ float sden[256 * TG];           // sqrt(V'/c2) + eps at [16 c_V + c_G]
  __shared__ float sdec[16 * TG];            // W (1 - lr decay) at [c_W]
  __shared__ uint32_t spbits[TAB ? 512 : 1];  // keep bits of (M, G) pairs; (V, G) at 256 +
  __shared__ uint32_t bused[3];
  for (uint32_t i = threadIdx.x; i < 3 * 16 * G; i += kThreads) sbook[(i / G) * RS + i % G] = book64[i];
  for (uint32_t i = threadIdx.x; i < 4 * 16 * G; i += kThreads) sold[i] = in.books4[i];
  if (threadIdx.x < 3) bused[threadIdx.x] = 0;
  for (uint32_t i = threadIdx.x; i < 3 * 16 * 16; i += kThreads) {
    const double* b = book64 + (i / 256) * 16 * G;
    double d = 0.0;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const double t = b[((i / 16) % 16) * G + j] - b[(i % 16) * G + j];
      d = d + t * t;
    }
    sgap[i] = sqrt(d);
  }
  __syncthreads();
  const Coeffs c = load_coeffs(in.coeffs);
  if (c.fail) return;  // the gather and encode passes report coefficient failures
  bool tab = false;
  if constexpr (TAB) {
    bool ok = true;
    for (uint32_t i = threadIdx.x; i < 4 * 16 * G; i += kThreads)
      ok &= finite_f32(sold[i]) & !(i >= 32 * G && i < 48 * G && sold[i] < 0.0f);
    tab = __syncthreads_and(ok);
    if (tab) {
      // entry e < 256: (c_M, c_G) = (e / 16, e % 16); e >= 256: (c_V, c_G)
      for (uint32_t e = threadIdx.x; e < 512; e += kThreads) {
        const bool vm = e < 256;
        const uint32_t p = e % 256, a0 = p / 16, cg = p % 16, st = vm ? 1 : 2;
        double x[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const float gradient = sold[(48 + cg) * G + j];
          float corrected;
          if (vm) {
            const float next_m = adamw_next_m(sold[(16 + a0) * G + j], gradient, c);
            sscaled[p * G + j] = adamw_scaled(next_m, c, corrected);
            x[j] = double(next_m);
          } else {
            const float next_v = adamw_next_v(sold[(32 + a0) * G + j], gradient, c);
            sden[p * G + j] = adamw_denominator(next_v, c, corrected);
            x[j] = double(next_v);
          }
        }
        spbits[e] = (active & (1u << st))
                        ? keep_bit<G>(x, st, a0, cand[st], sbook, sgap, book64 + st * 16 * G)
                        : 0u;
      }
      for (uint32_t i = threadIdx.x; i < 16 * G; i += kThreads) sdec[i] = adamw_decayed(sold[i], c);
      __syncthreads();
    }
  }
  const uint32_t words = words_for(in.m, G);
  const uint32_t complete = in.m / G;
  uint32_t used[3] = {0, 0, 0};
  for (uint32_t v = blockIdx.x * kThreads + threadIdx.x; v < complete; v += gridDim.x * kThreads) {
    uint32_t code[4];
#pragma unroll
    for (int st = 0; st < 4; ++st) code[st] = nibble(in.codes4 + st * words, v);
    if constexpr (TAB) {
      if (tab) {
        const uint32_t em = 16 * code[1] + code[3], ev = 16 * code[2] + code[3];
        used[1] |= spbits[em];
        used[2] |= spbits[256 + ev];
        if (active & 1u) {
          double x0[G];
#pragma unroll
          for (int j = 0; j < G; ++j)
            x0[j] = double(sdec[code[0] * G + j] - sscaled[em * G + j] / sden[ev * G + j]);
          used[0] |= keep_bit<G>(x0, 0, code[0], cand[0], sbook, sgap, book64);
        }
        continue;
      }
    }
    double x[3][G];
    if (active & 1u) {
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const AdamwOut r = adamw_value(sold[code[0] * G + j], sold[(16 + code[1]) * G + j],
                                       sold[(32 + code[2]) * G + j], sold[(48 + code[3]) * G + j],
                                       c);
        x[0][j] = double(r.w);
        x[1][j] = double(r.m);
        x[2][j] = double(r.v);
      }
    } else {  // W's fit needs no pass: skip W' and its divisions
#pragma unroll
      for (int j = 0; j < G; ++j) {
        float m, v;
        adamw_moments(sold[code[0] * G + j], sold[(16 + code[1]) * G + j],
                      sold[(32 + code[2]) * G + j], sold[(48 + code[3]) * G + j], c, m, v);
        x[0][j] = 0.0;
        x[1][j] = double(m);
        x[2][j] = double(v);
      }
    }
#pragma unroll
    for (int st = 0; st < 3; ++st)
      if (active & (1u << st))
        used[st] |= keep_bit<G>(x[st], st, code[st], cand[st], sbook, sgap, book64 + st * 16 * G);
  }
  // One global atomic per block and state, and none when the bits are
  // already set: every block reports, so atomics on the three words would
  // otherwise serialise the whole pass.
#pragma unroll
  for (int st = 0; st < 3; ++st) {
    for (int off = 1; off < warpSize; off <<= 1) used[st] |= __shfl_xor(used[st], off);
    if (used[st] && (threadIdx.x % warpSize) == 0) atomicOr(&bused[st], used[st]);
  }
  __syncthreads();
  if (threadIdx.x < 3) {
    const uint32_t mine = bused[threadIdx.x];
    uint32_t* word = &a.flags[threadIdx.x * 4 + 1];
    const uint32_t seen = __hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (mine & ~seen) atomicOr(word, mine);
  }
}

// Recompute W', M', V' per vector and encode each against its new book with
// op 0's FP32 rule; count W values whose decoded value moved.
//
// Pair tables (G <= 16): a vector's M' depends only on its M and G codes and
// its V' only on its V and G codes, so when the shader writes every element
// (all four input books finite, no negative variance entry) each block first
// forms, for all 256 (M, G) and (V, G) code pairs, M' and its code, V' and its
// code, lr M'/c1 and sqrt(V'/c2) + eps, and W (1 - lr decay) for the 16 W
// codes. A whole vector then costs G divisions, G subtractions and the W'
// screen. The status bits are those of the element loop: a pair's nonfinite
// term or nonfinite encode distance is raised by every vector that uses it.
template <int G>
constexpr bool kPairTables = G <= 16;

template <int G>
__global__ __launch_bounds__(kThreads) void k_adamw_encode(AdamwInputs in, const float* books3,
                                                           uint32_t* out_codes, uint32_t* changed,
                                                           uint32_t* status) {
  constexpr bool TAB = kPairTables<G>;
  constexpr uint32_t TG = TAB ? G : 1;
  __shared__ float sbook[3 * 16 * G];
  __shared__ float sold[4 * 16 * G];  // the op-3 input books; W's is the old weight book
  __shared__ float sm2[3 * 16 * G];
  __shared__ float scn[3 * 16];
  __shared__ float sscaled[256 * TG];         // lr M'/c1 at [16 c_M + c_G]
  __shared__ float sden[256 * TG];            // sqrt(V'/c2) + eps at [16 c_V + c_G]
  __shared__ float sdec[16 * TG];             // W (1 - lr decay) at [c_W]
  __shared__ uint32_t spair[TAB ? 512 : 1];   // M' code | nonfinite << 4; V' at 256 +
  __shared__ uint32_t sdecbad[TAB ? 16 : 1];
  __shared__ uint32_t bflags, bmoved;
  for (uint32_t i = threadIdx.x; i < 3 * 16 * G; i += kThreads) sbook[i] = books3[i];
  for (uint32_t i = threadIdx.x; i < 4 * 16 * G; i += kThreads) sold[i] = in.books4[i];
  if (threadIdx.x == 0) bflags = bmoved = 0;
  if (blockIdx.x == 0) sweep_book(books3, 3 * 16 * G, status);
  __syncthreads();
  screen_prepare<G>(sbook, sm2, scn, 3);
  __syncthreads();
  Screen screen[3];
#pragma unroll
  for (int st = 0; st < 3; ++st) screen[st] = screen_load<G>(sm2 + st * 16 * G, scn + st * 16);
  const Coeffs c = load_coeffs(in.coeffs);
  if (c.fail) {
    if (blockIdx.x == 0 && threadIdx.x == 0) atomicOr(status, c.fail);
    return;
  }
  bool tab = false;
  if constexpr (TAB) {
    bool ok = true;
    for (uint32_t i = threadIdx.x; i < 4 * 16 * G; i += kThreads)
      ok &= finite_f32(sold[i]) & !(i >= 32 * G && i < 48 * G && sold[i] < 0.0f);
    tab = __syncthreads_and(ok);
    if (tab) {
      // entry e < 256: (c_M, c_G) = (e / 16, e % 16); e >= 256: (c_V, c_G)
      for (uint32_t e = threadIdx.x; e < 512; e += kThreads) {
        const bool vm = e < 256;
        const uint32_t p = e % 256, a = p / 16, cg = p % 16;
        float xv[G];
        bool nf = false;
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const float gradient = sold[(48 + cg) * G + j];
          float corrected;
          if (vm) {
            const float next_m = adamw_next_m(sold[(16 + a) * G + j], gradient, c);
            sscaled[p * G + j] = adamw_scaled(next_m, c, corrected);
            nf |= !finite_f32(next_m) | !finite_f32(corrected);
            xv[j] = next_m;
          } else {
            const float next_v = adamw_next_v(sold[(32 + a) * G + j], gradient, c);
            const float den = adamw_denominator(next_v, c, corrected);
            sden[p * G + j] = den;
            nf |= !finite_f32(next_v) | !finite_f32(corrected) | !finite_f32(den);
            xv[j] = next_v;
          }
        }
        uint32_t code = argmin_screen<G>(xv, vm ? screen[1] : screen[2]);
        if (code == kNoScreen) code = argmin32<G, true>(xv, G, sbook + (vm ? 16 : 32) * G, nf);
        spair[e] = code | (uint32_t(nf) << 4);
      }
      for (uint32_t i = threadIdx.x; i < 16 * G; i += kThreads) sdec[i] = adamw_decayed(sold[i], c);
      __syncthreads();
      if (threadIdx.x < 16) {
        bool nf = false;
#pragma unroll
        for (int j = 0; j < G; ++j) nf |= !finite_f32(sdec[threadIdx.x * G + j]);
        sdecbad[threadIdx.x] = nf;
      }
      __syncthreads();
    }
  }
  const uint32_t m = in.m;
  const uint32_t words = words_for(m, G);
  const uint32_t vectors = m / G + (m % G != 0);
  uint32_t flags = 0;
  uint32_t moved = 0;
  bool bad = false;
  for (uint32_t base = blockIdx.x * kThreads; base < words * 8; base += gridDim.x * kThreads) {
    const uint32_t v = base + threadIdx.x;
    uint32_t code[3] = {0, 0, 0};
    bool tabled = false;
    if constexpr (TAB) {
      if (tab && v < m / G) {  // a whole vector from the pair tables
        tabled = true;
        uint32_t in_code[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) in_code[st] = nibble(in.codes4 + st * words, v);
        const uint32_t em = 16 * in_code[1] + in_code[3], ev = 16 * in_code[2] + in_code[3];
        const uint32_t pm = spair[em], pv = spair[256 + ev];
        code[1] = pm & 15u;
        code[2] = pv & 15u;
        bool nf = ((pm | pv) >> 4) != 0 || sdecbad[in_code[0]] != 0;
        float xw[G];
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const float nw = sdec[in_code[0] * G + j] - sscaled[em * G + j] / sden[ev * G + j];
          xw[j] = nw;
          nf |= !finite_f32(nw);
        }
        flags |= nf ? 1u : 0u;
        code[0] = argmin_screen<G>(xw, screen[0]);
        if (code[0] == kNoScreen) code[0] = argmin32<G, true>(xw, G, sbook, bad);
#pragma unroll
        for (int j = 0; j < G; ++j) moved += sbook[code[0] * G + j] != sold[in_code[0] * G + j];
      }
    }
    if (!tabled && v < vectors) {
      const uint32_t start = v * G;
      const uint32_t valid = (m - start) < G ? (m - start) : G;
      uint32_t in_code[4];
#pragma unroll
      for (int st = 0; st < 4; ++st) in_code[st] = nibble(in.codes4 + st * words, v);
      float xs[3][G];
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const AdamwOut r = adamw_value(sold[in_code[0] * G + j], sold[(16 + in_code[1]) * G + j],
                                       sold[(32 + in_code[2]) * G + j],
                                       sold[(48 + in_code[3]) * G + j], c);
        // components past a tail vector's end are computed but neither
        // reported nor compared (the tail argmin reads only the valid ones)
        const bool live = uint32_t(j) < valid;
        flags |= live ? r.flags : 0u;
        xs[0][j] = r.w; xs[1][j] = r.m; xs[2][j] = r.v;
        bad |= live & (!finite_f32(r.w) | !finite_f32(r.m) | !finite_f32(r.v));
      }
      if (valid == G) {
#pragma unroll
        for (int st = 0; st < 3; ++st) {
          code[st] = argmin_screen<G>(xs[st], screen[st]);
          if (code[st] == kNoScreen) code[st] = argmin32<G, true>(xs[st], G, sbook + st * 16 * G, bad);
        }
      } else {
#pragma unroll
        for (int st = 0; st < 3; ++st)
          code[st] = argmin32<G, false>(xs[st], valid, sbook + st * 16 * G, bad);
      }
#pragma unroll
      for (int j = 0; j < G; ++j)
        moved += (uint32_t(j) < valid) & (sbook[code[0] * G + j] != sold[in_code[0] * G + j]);
    }
#pragma unroll
    for (int st = 0; st < 3; ++st) {
      const uint32_t word = gather_word(code[st] << (4u * (v & 7u)));
      if ((v & 7u) == 0 && (v >> 3) < words) out_codes[st * words + (v >> 3)] = word;
    }
  }
  if (bad) flags |= 1;
  for (int off = 1; off < warpSize; off <<= 1) {
    flags |= __shfl_xor(flags, off);
    moved += __shfl_xor(moved, off);
  }
  // one global atomic per block, not per wave (every block counts moves)
  if ((threadIdx.x % warpSize) == 0) {
    if (flags) atomicOr(&bflags, flags);
    if (moved) atomicAdd(&bmoved, moved);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    if (bflags) atomicOr(status, bflags);
    if (bmoved) atomicAdd(changed, bmoved);
  }
}

uint32_t grid_for(uint64_t items, uint32_t per_block) {
  uint64_t blocks = (items + per_block - 1) / per_block;
  if (blocks == 0) blocks = 1;
  return blocks > kMaxGridX ? kMaxGridX : uint32_t(blocks);
}

}  // namespace

#define ACKVQ_DISPATCH_GROUP(group, KERNEL, ...)                         \
  do {                                                                  \
    if ((group) == 8) { KERNEL<8><<<__VA_ARGS__>>>; }                   \
    else if ((group) == 16) { KERNEL<16><<<__VA_ARGS__>>>; }            \
    else { KERNEL<32><<<__VA_ARGS__>>>; }                               \
  } while (0)

// Encode's blocks stay resident and stream: one round of them on MI355X (256
// compute units, kEncodeWaves blocks of 4 waves each), so every wave loads its
// next tile while it ranks the current one.
constexpr uint32_t kComputeUnits = 256;

hipError_t launch_encode(hipStream_t s, const Operands& o, uint32_t m, uint32_t group) {
  const uint32_t vectors = m / group + (m % group != 0);
  const uint32_t words = vectors / 8 + (vectors % 8 != 0);
  const uint32_t cap = kComputeUnits * (group == 8    ? kEncodeWaves<8>
                                        : group == 16 ? kEncodeWaves<16>
                                                      : kEncodeWaves<32>);
  const uint32_t blocks = grid_for(uint64_t(words) * 8, kThreads);
  dim3 grid(blocks < cap ? blocks : cap, o.count);
  if (group == 8) k_encode<8><<<grid, kThreads, 0, s>>>(o, m);
  else if (group == 16) k_encode<16><<<grid, kThreads, 0, s>>>(o, m);
  else k_encode<32><<<grid, kThreads, 0, s>>>(o, m);
  return hipGetLastError();
}

hipError_t launch_decode(hipStream_t s, const Operands& o, uint32_t m, uint32_t group) {
  dim3 grid(grid_for((m + 3) / 4, kThreads), o.count);
  if (group == 8) k_decode<8><<<grid, kThreads, 0, s>>>(o, m);
  else if (group == 16) k_decode<16><<<grid, kThreads, 0, s>>>(o, m);
  else k_decode<32><<<grid, kThreads, 0, s>>>(o, m);
  return hipGetLastError();
}

hipError_t launch_adamw(hipStream_t s, const Operands& o, uint32_t m, uint32_t group) {
  dim3 grid(grid_for((m + 3) / 4, kThreads), o.count);
  if (group == 8) k_adamw<8><<<grid, kThreads, 0, s>>>(o, m);
  else if (group == 16) k_adamw<16><<<grid, kThreads, 0, s>>>(o, m);
  else k_adamw<32><<<grid, kThreads, 0, s>>>(o, m);
  return hipGetLastError();
}

hipError_t launch_adamw_gather(hipStream_t s, const AdamwInputs& in, uint32_t count, float* out,
                               uint32_t* changed, uint32_t* status, float* fit_book,
                               uint32_t* fit_flags) {
  dim3 grid(grid_for(uint64_t(count) * in.group, kThreads));
  if (in.group == 8)
    k_adamw_gather<8><<<grid, kThreads, 0, s>>>(in, count, out, changed, status, fit_book, fit_flags);
  else if (in.group == 16)
    k_adamw_gather<16><<<grid, kThreads, 0, s>>>(in, count, out, changed, status, fit_book, fit_flags);
  else
    k_adamw_gather<32><<<grid, kThreads, 0, s>>>(in, count, out, changed, status, fit_book, fit_flags);
  return hipGetLastError();
}

hipError_t launch_adamw_keep(hipStream_t s, const AdamwInputs& in, const FitArgs& a) {
  // one resident round (2 blocks per compute unit, 1 at group 32, as the
  // registers allow), each walking many vectors: the per-block set-up (books,
  // the entry-gap table, the pair tables) is paid once per block
  const uint32_t cap = kComputeUnits * (in.group == 32 ? 1 : 2);
  const uint32_t blocks = grid_for(in.m / in.group, kThreads);
  dim3 grid(blocks < cap ? blocks : cap);
  if (in.group == 8) k_adamw_keep<8><<<grid, kThreads, 0, s>>>(in, a);
  else if (in.group == 16) k_adamw_keep<16><<<grid, kThreads, 0, s>>>(in, a);
  else k_adamw_keep<32><<<grid, kThreads, 0, s>>>(in, a);
  return hipGetLastError();
}

// ---- sum of squares in float64 (the harness's gradient norm) -------------------
// Each square of an FP32 value is exact in float64. Thread t of the grid sums
// the squares of values t, t + T, t + 2T, ... (T = kSumBlocks x kThreads) in
// order, a wave sums its 64 lanes by a fixed butterfly, the block its waves in
// order; k_sumsq_final adds the block sums in block order. The order is fixed,
// so the result is deterministic, and every path from a square to the total
// has at most count / T + 15 additions: its error is within
// (count / T + 15) u64 of the sum.
constexpr uint32_t kSumBlocks = 256;

__global__ __launch_bounds__(kThreads) void k_sumsq_partial(const float* __restrict__ x,
                                                            uint64_t count,
                                                            double* __restrict__ partial) {
  __shared__ double wsum[kThreads / 64];
  const uint64_t stride = uint64_t(kSumBlocks) * kThreads;
  double acc = 0.0;
  for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < count; i += stride) {
    const double v = double(x[i]);
    acc += v * v;
  }
  for (int off = 32; off >= 1; off >>= 1) acc += __shfl_xor(acc, off);
  if (threadIdx.x % 64 == 0) wsum[threadIdx.x / 64] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double b = wsum[0];
    for (uint32_t w = 1; w < kThreads / 64; ++w) b += wsum[w];
    partial[blockIdx.x] = b;
  }
}

__global__ __launch_bounds__(64) void k_sumsq_final(const double* __restrict__ partial,
                                                    double* __restrict__ out) {
  if (threadIdx.x == 0) {
    double t = partial[0];
    for (uint32_t b = 1; b < kSumBlocks; ++b) t += partial[b];
    *out = t;
  }
}

// x[i] = x[i] * f, one rounded FP32 multiply per value (the harness's clip).
__global__ __launch_bounds__(kThreads) void k_scale_f32(float* __restrict__ x, uint64_t count,
                                                        float f) {
  const uint64_t stride = uint64_t(gridDim.x) * kThreads;
  for (uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x; i < count; i += stride)
    x[i] = x[i] * f;
}

hipError_t launch_scale(hipStream_t s, float* x, uint64_t count, float f) {
  const uint64_t want = (count + kThreads - 1) / kThreads;
  k_scale_f32<<<dim3(uint32_t(want < 4096 ? (want ? want : 1) : 4096)), kThreads, 0, s>>>(x, count, f);
  return hipGetLastError();
}

hipError_t launch_sum_squares(hipStream_t s, const float* x, uint64_t count, double* partial,
                              double* out) {
  k_sumsq_partial<<<kSumBlocks, kThreads, 0, s>>>(x, count, partial);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  k_sumsq_final<<<1, 64, 0, s>>>(partial, out);
  return hipGetLastError();
}

// The fused encode pass builds its pair tables once per block, so its grid is
// one resident round (blocks of 4 waves per compute unit: 3 at group 8, 2 at
// 16, 1 at 32, as its registers allow) and every block walks many vectors.
constexpr uint32_t kAdamwEncodeBlocks[3] = {kComputeUnits * 3, kComputeUnits * 2, kComputeUnits};

hipError_t launch_adamw_encode(hipStream_t s, const AdamwInputs& in, const float* books3,
                               uint32_t* out_codes, uint32_t* changed, uint32_t* status) {
  const uint32_t vectors = in.m / in.group + (in.m % in.group != 0);
  const uint32_t words = vectors / 8 + (vectors % 8 != 0);
  const uint32_t cap = kAdamwEncodeBlocks[in.group == 8 ? 0 : in.group == 16 ? 1 : 2];
  const uint32_t blocks = grid_for(uint64_t(words) * 8, kThreads);
  dim3 grid(blocks < cap ? blocks : cap);
  if (in.group == 8) k_adamw_encode<8><<<grid, kThreads, 0, s>>>(in, books3, out_codes, changed, status);
  else if (in.group == 16) k_adamw_encode<16><<<grid, kThreads, 0, s>>>(in, books3, out_codes, changed, status);
  else k_adamw_encode<32><<<grid, kThreads, 0, s>>>(in, books3, out_codes, changed, status);
  return hipGetLastError();
}

}  // namespace ackvq
