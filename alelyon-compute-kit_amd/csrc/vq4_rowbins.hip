// Large-m packed products on gfx950 without decoding the weight: "row bins".
//
// For C = A . B with B stored (k, n) and its groups along n (op 2, flags 0 of
// src/alelyon_compute_kit/_kit/kernels/vq4.comp:165-176), the output group j
// of row r is y[r][j*G+t] = sum_e C_B[e][t] * S[r][j][e] with
// S[r][j][e] = sum over rows kk of B whose code in group j is e of x[r][kk].
//
// Lanes are rows r of A, so the code of B's nibble (kk, j) is the same for all
// 64 lanes of a wave: it is read with scalar loads, and S[r][j][.] lives in 16
// consecutive VGPRs of each lane, addressed by that wave-uniform code through
// VGPR indexing (s_set_gpr_idx_on). One FP32 add per (row, nibble) -- G times
// fewer than decoding B and multiplying -- and no LDS traffic in the loop.
//
// Each wave owns one word column q of B (8 output groups, 128 bins) for 64
// rows and walks all of k; B's words are first transposed so a column is
// contiguous and each wave streams it with wide scalar loads. A is decoded
// per group of G activations: a row's G values at group u are one codebook
// row C_A[code(r, u)].
//
// The sum order differs from the shader's sequential one; results agree to
// FP32 rounding (bins of about k/16 terms each, then a 16-term product).
#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "kernels.hpp"

namespace ackvq {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ bool finite_f32(float x) { return fabsf(x) <= FLT_MAX; }

__device__ __forceinline__ uint32_t nibble(const uint32_t* codes, uint32_t vector) {
  return (codes[vector >> 3] >> ((vector & 7u) * 4u)) & 15u;
}

// ACC[e] += X for e = bits [SEL] of the wave-uniform WORD; ACC is pinned to
// the VGPRs REGS whose first register is BASE. VGPR indexing applies to the
// one v_add between s_set_gpr_idx_on and s_set_gpr_idx_off. s_bfe_u32 writes
// SCC, hence the clobber (a loop's compare-and-branch may straddle the asm);
// s_set_gpr_idx_on also writes M0, which nothing else in this file uses.
#define ROWBIN_ADD(ACC, REGS, BASE, WORD, SEL, X)                                   \
  do {                                                                              \
    uint32_t e_;                                                                    \
    asm volatile("s_bfe_u32 %1, %2, %3\n\t"                                        \
                 "s_set_gpr_idx_on %1, gpr_idx(SRC0,DST)\n\t"                      \
                 "v_add_f32 " BASE ", " BASE ", %4\n\t"                             \
                 "s_set_gpr_idx_off"                                                \
                 : "+{" REGS "}"(ACC), "=&s"(e_)                                    \
                 : "s"(WORD), "i"(SEL), "v"(X)                                      \
                 : "scc");                                                          \
  } while (0)

// The eight ROWBIN_ADDs of one code word in one indexing window: index
// mode stays on across them and s_set_gpr_idx_idx moves the index to the
// next nibble's code, so each add costs two scalar instructions, not three.
// Only the adds run inside the window (SRC0 and DST are indexed; X, their
// second source, is not).
#define ROWBIN_ADD8(B0, B1, B2, B3, B4, B5, B6, B7, WORD, X)                        \
  do {                                                                              \
    uint32_t e_;                                                                    \
    asm volatile("s_bfe_u32 %8, %9, 0x40000\n\t"                                  \
                 "s_set_gpr_idx_on %8, gpr_idx(SRC0,DST)\n\t"                     \
                 "v_add_f32 v0, v0, %10\n\t"                                       \
                 "s_bfe_u32 %8, %9, 0x40004\n\t"                                  \
                 "s_set_gpr_idx_idx %8\n\t"                                        \
                 "v_add_f32 v16, v16, %10\n\t"                                     \
                 "s_bfe_u32 %8, %9, 0x40008\n\t"                                  \
                 "s_set_gpr_idx_idx %8\n\t"                                        \
                 "v_add_f32 v32, v32, %10\n\t"                                     \
                 "s_bfe_u32 %8, %9, 0x4000c\n\t"                                  \
                 "s_set_gpr_idx_idx %8\n\t"                                        \
                 "v_add_f32 v48, v48, %10\n\t"                                     \
                 "s_bfe_u32 %8, %9, 0x40010\n\t"                                  \
                 "s_set_gpr_idx_idx %8\n\t"                                        \
                 "v_add_f32 v64, v64, %10\n\t"                                     \
                 "s_bfe_u32 %8, %9, 0x40014\n\t"                                  \
                 "s_set_gpr_idx_idx %8\n\t"                                        \
                 "v_add_f32 v80, v80, %10\n\t"                                     \
                 "s_bfe_u32 %8, %9, 0x40018\n\t"                                  \
                 "s_set_gpr_idx_idx %8\n\t"                                        \
                 "v_add_f32 v96, v96, %10\n\t"                                     \
                 "s_bfe_u32 %8, %9, 0x4001c\n\t"                                  \
                 "s_set_gpr_idx_idx %8\n\t"                                        \
                 "v_add_f32 v112, v112, %10\n\t"                                   \
                 "s_set_gpr_idx_off"                                                \
                 : "+{v[0:15]}"(B0), "+{v[16:31]}"(B1), "+{v[32:47]}"(B2),          \
                   "+{v[48:63]}"(B3), "+{v[64:79]}"(B4), "+{v[80:95]}"(B5),         \
                   "+{v[96:111]}"(B6), "+{v[112:127]}"(B7), "=&s"(e_)               \
                 : "s"(WORD), "v"(X)                                                \
                 : "scc");                                                          \
  } while (0)

constexpr int kRBWaves = 4;  // word columns per block

// Word column q of B's codes, contiguous: wt[q * k + kk] = codes[kk * rw + q].
__global__ __launch_bounds__(256) void k_transpose_words(const uint32_t* __restrict__ codes,
                                                         uint32_t* __restrict__ wt, uint32_t k,
                                                         uint32_t rw) {
  __shared__ uint32_t tile[32][33];
  const uint32_t q0 = blockIdx.x * 32, k0 = blockIdx.y * 32;
  const uint32_t tx = threadIdx.x % 32, ty = threadIdx.x / 32;
  for (uint32_t i = ty; i < 32; i += 8) {
    const uint32_t kk = k0 + i, q = q0 + tx;
    tile[i][tx] = (kk < k && q < rw) ? codes[uint64_t(kk) * rw + q] : 0u;
  }
  __syncthreads();
  for (uint32_t i = ty; i < 32; i += 8) {
    const uint32_t q = q0 + i, kk = k0 + tx;
    if (q < rw && kk < k) wt[uint64_t(q) * k + kk] = tile[tx][i];
  }
}

// One output group of one row: y[t] = sum_e sbt[t][e] * sb[e], written as
// float4s; returns whether any y is nonfinite.
template <int G>
__device__ __forceinline__ bool finish_group(const v16f sb, const float (*sbt)[16], float* orow,
                                             bool live) {
  bool bad = false;
#pragma unroll 1
  for (int t = 0; t < G; t += 4) {
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4* c = reinterpret_cast<const float4*>(&sbt[t + i][0]);
      const float4 c0 = c[0], c1 = c[1], c2 = c[2], c3 = c[3];
      float acc = 0.0f;
      acc = fmaf(c0.x, sb[0], acc);  acc = fmaf(c0.y, sb[1], acc);
      acc = fmaf(c0.z, sb[2], acc);  acc = fmaf(c0.w, sb[3], acc);
      acc = fmaf(c1.x, sb[4], acc);  acc = fmaf(c1.y, sb[5], acc);
      acc = fmaf(c1.z, sb[6], acc);  acc = fmaf(c1.w, sb[7], acc);
      acc = fmaf(c2.x, sb[8], acc);  acc = fmaf(c2.y, sb[9], acc);
      acc = fmaf(c2.z, sb[10], acc); acc = fmaf(c2.w, sb[11], acc);
      acc = fmaf(c3.x, sb[12], acc); acc = fmaf(c3.y, sb[13], acc);
      acc = fmaf(c3.z, sb[14], acc); acc = fmaf(c3.w, sb[15], acc);
      y[i] = acc;
      bad |= !finite_f32(acc);
    }
    if (live) *reinterpret_cast<float4*>(orow + t) = make_float4(y[0], y[1], y[2], y[3]);
  }
  return bad && live;
}

// AD: A is a dense FP32 m x k array in in[0] (the dense-activation product).
template <int G, bool AD>
__global__ __launch_bounds__(256) void k_rowbins(Operands o, uint32_t m, uint32_t n, uint32_t k,
                                                 const uint32_t* __restrict__ wt) {
  __shared__ __align__(16) float sbt[G][16];      // C_B transposed: sbt[t][e]
  const uint32_t* a_codes = static_cast<const uint32_t*>(o.in[0]);
  const float* a_book = static_cast<const float*>(o.in[1]);
  const float* b_book = static_cast<const float*>(o.in[3]);
  float* out = static_cast<float*>(o.out);
  const uint32_t lane = threadIdx.x % 64;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  const uint32_t rw = n / (8 * G);
  const uint32_t q = blockIdx.x * kRBWaves + wave;
  const uint32_t r = blockIdx.y * 64 + lane;
  const bool row_live = r < m;
  for (uint32_t i = threadIdx.x; i < 16 * G; i += blockDim.x) sbt[i % G][i / G] = b_book[i];
  if (blockIdx.x == 0 && blockIdx.y == 0) {
    bool bad = false;
    for (uint32_t i = threadIdx.x; i < 16 * G; i += blockDim.x)
      bad |= (!AD && !finite_f32(a_book[i])) || !finite_f32(b_book[i]);
    if (__any(bad) && lane == 0) atomicOr(o.status, 1u);
  }
  __syncthreads();
  if (q >= rw) return;

  v16f b0 = (v16f)0.0f, b1 = (v16f)0.0f, b2 = (v16f)0.0f, b3 = (v16f)0.0f;
  v16f b4 = (v16f)0.0f, b5 = (v16f)0.0f, b6 = (v16f)0.0f, b7 = (v16f)0.0f;
  const uint32_t groups = k / G;                       // A groups per row
  const uint32_t* col = wt + uint64_t(q) * k;
  // B words come in runs of 16 (one 64-byte scalar load), prefetched one run
  // ahead; x comes 16 values at a time from the A codebook row.
  constexpr int kRun = 16;
  const uint32_t runs = k / kRun;
  uint32_t wn[kRun];
#pragma unroll
  for (int i = 0; i < kRun; ++i) wn[i] = col[i];
  // x comes from the A codebook in global memory (L1-resident, 16 x G
  // floats): reading it through LDS would share lgkmcnt with the scalar
  // prefetch and wait for it.
  uint32_t a = (!AD && row_live) ? nibble(a_codes, r * groups) : 0u;
  uint32_t a_next = (!AD && row_live && groups > 1) ? nibble(a_codes, r * groups + 1) : 0u;
  const float* x_row = static_cast<const float*>(o.in[0]) + uint64_t(row_live ? r : 0) * k;
  for (uint32_t run = 0; run < runs; ++run) {
    uint32_t w[kRun];
#pragma unroll
    for (int i = 0; i < kRun; ++i) w[i] = wn[i];
    if (run + 1 < runs) {
#pragma unroll
      for (int i = 0; i < kRun; ++i) wn[i] = col[(run + 1) * kRun + i];
    }
    const uint32_t kk0 = run * kRun;
    const uint32_t u = kk0 / G, s0 = kk0 % G;
    if (!AD && s0 == 0 && u > 0) {
      a = a_next;
      if (row_live && u + 1 < groups) a_next = nibble(a_codes, r * groups + u + 1);
    }
    float x[kRun];
    const float4* xrow = AD ? reinterpret_cast<const float4*>(x_row + kk0)
                            : reinterpret_cast<const float4*>(a_book + a * G + s0);
#pragma unroll
    for (int s = 0; s < kRun; s += 4) {
      const float4 v = xrow[s / 4];
      x[s] = row_live ? v.x : 0.0f;
      x[s + 1] = row_live ? v.y : 0.0f;
      x[s + 2] = row_live ? v.z : 0.0f;
      x[s + 3] = row_live ? v.w : 0.0f;
    }
#pragma unroll
    for (int s = 0; s < kRun; ++s) {
      const uint32_t ww = w[s];
      const float xv = x[s];
      ROWBIN_ADD8(b0, b1, b2, b3, b4, b5, b6, b7, ww, xv);
    }
  }

  // y[r][(8q + g8) * G + t] = sum_e C_B[e][t] * bins[g8][e]
  float* orow = out + uint64_t(r) * n + uint64_t(q) * 8 * G;
  bool bad = false;
  bad |= finish_group<G>(b0, sbt, orow + 0 * G, row_live);
  bad |= finish_group<G>(b1, sbt, orow + 1 * G, row_live);
  bad |= finish_group<G>(b2, sbt, orow + 2 * G, row_live);
  bad |= finish_group<G>(b3, sbt, orow + 3 * G, row_live);
  bad |= finish_group<G>(b4, sbt, orow + 4 * G, row_live);
  bad |= finish_group<G>(b5, sbt, orow + 5 * G, row_live);
  bad |= finish_group<G>(b6, sbt, orow + 6 * G, row_live);
  bad |= finish_group<G>(b7, sbt, orow + 7 * G, row_live);
  if (__any(bad) && lane == 0) atomicOr(o.status, 1u);
}

}  // namespace

// Dense A has no groups to straddle: any group, k a multiple of 16 (runs).
bool rowbins_applies_dense(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags) {
  return flags == 0 && m >= 64 && n % (8 * group) == 0 && k % 16 == 0;
}

bool rowbins_applies(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags) {
  // runs of 16 rows of B never straddle an A group: k % 16 == 0 and g >= 16
  // divides them, g = 8 takes two groups per run (handled: s0 + s < 16 < 2g).
  return flags == 0 && m >= 64 && n % (8 * group) == 0 && k % group == 0 && k % 16 == 0 &&
         group >= 16;
}

size_t rowbins_workspace_bytes(uint32_t n, uint32_t k, uint32_t group) {
  return size_t(n / (8 * group)) * k * 4;
}

namespace {

template <bool AD>
hipError_t rowbins_launch(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                          uint32_t group, void* workspace) {
  const uint32_t rw = n / (8 * group);
  uint32_t* wt = static_cast<uint32_t*>(workspace);
  dim3 tgrid((rw + 31) / 32, (k + 31) / 32);
  k_transpose_words<<<tgrid, 256, 0, s>>>(static_cast<const uint32_t*>(o.in[2]), wt, k, rw);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  dim3 grid((rw + kRBWaves - 1) / kRBWaves, (m + 63) / 64);
  if (group == 8) k_rowbins<8, AD><<<grid, 64 * kRBWaves, 0, s>>>(o, m, n, k, wt);
  else if (group == 16) k_rowbins<16, AD><<<grid, 64 * kRBWaves, 0, s>>>(o, m, n, k, wt);
  else k_rowbins<32, AD><<<grid, 64 * kRBWaves, 0, s>>>(o, m, n, k, wt);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_rowbins(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                          uint32_t group, void* workspace) {
  return rowbins_launch<false>(s, o, m, n, k, group, workspace);
}

hipError_t launch_rowbins_dense(hipStream_t s, const Operands& o, uint32_t m, uint32_t n,
                                uint32_t k, uint32_t group, void* workspace) {
  return rowbins_launch<true>(s, o, m, n, k, group, workspace);
}

}  // namespace ackvq
