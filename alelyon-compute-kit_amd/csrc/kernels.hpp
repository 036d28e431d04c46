// Launch interface between the C ABI (abi.cpp) and the gfx950 kernels.
//
// Every launcher enqueues on the caller's stream and returns the launch
// status; none allocates or synchronises. Pointers are device addresses of
// the first instance; `stride` gives the byte distance between consecutive
// batch instances of each slot (ack_vq_batch), zero for a single instance.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace ackvq {

struct Operands {
  const void* in[4] = {nullptr, nullptr, nullptr, nullptr};
  void* out = nullptr;
  uint32_t* status = nullptr;
  uint64_t stride[5] = {0, 0, 0, 0, 0};  // slots 0..3, then out
  uint32_t count = 1;
  // gemv-direct's arrival counters: kDirectCounters words, zero between
  // launches, one array per device handle (its launches share one stream)
  uint32_t* arrivals = nullptr;
};

constexpr uint32_t kDirectCounters = 1u << 16;

// Which implementation serves an op-2 product.
enum class MatmulPath : int {
  General = 0,    // tiled, sequential FP32 per output: bit-identical to vq4.comp
  GemvRows = 1,   // 2 <= m <= 8, B groups along n: nibble bins, two rows per 64-bit atomic
  GemvTable = 2,  // B groups along k (B stored (n,k)): dot-product table, small m
  GramMfma = 3,   // both operands grouped along k: one-hot x Gram table on fp16 MFMA
  // 4 is retired: row bins, an FP32 add per (row, nibble) through VGPR index
  // mode, served dense activations of large m before onehot-mfma took them
  GemvPairs = 5,  // m = 1, B groups along n: one atomic per byte into 256-way pair bins
  GemvRowPairs = 6,  // 2 <= m <= 8 (row-major A, batches that fill the chip): each row of A
                     // a GemvPairs instance, the rows of one product on one XCD
  GemvDirect = 7,    // m <= 8, few weights (kDirectMaxWeights): decode and FMA per output,
                     // split k reduced by the last block of each tile, one launch
  OneHotMfma = 8,    // m >= kOneHotMinRows, packed A along k, B along n: A's book rows x
                     // one-hot of B's codes on bf16 MFMA, then the 16-term codebook product
};

const char* matmul_path_name(MatmulPath p);

// Chooses the path for a product; `policy` 1 forces General, 2 takes a
// factorised path wherever its shape applies, whatever the size (tests; it
// never takes gemv-direct, and onehot-mfma only from kOneHotMinRows rows,
// where no bin kernel applies, so the bin kernels stay covered at the same
// shapes).
MatmulPath choose_matmul_path(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                              uint32_t count, uint32_t policy);

bool gram_applies(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                  bool any_size);
// Float64 sum of squares of count float32 values: 256 block partials into
// `partial`, then their ordered total into *out.
hipError_t launch_sum_squares(hipStream_t s, const float* x, uint64_t count, double* partial,
                              double* out);
// x[i] *= f in FP32, in place.
hipError_t launch_scale(hipStream_t s, float* x, uint64_t count, float f);
hipError_t launch_gram(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                       uint32_t group);

// gemv-direct (vq4_direct.hip): the automatic choice for products of at most
// kDirectMaxRows rows of A and at most kDirectMaxWeights weights in all
// (n k count); above them the bin kernels are faster.
constexpr uint32_t kDirectMaxRows = 8;
constexpr uint64_t kDirectMaxWeights = uint64_t(1) << 25;
bool direct_applies(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                    uint32_t count);
size_t direct_workspace_bytes(uint32_t m, uint32_t n, uint32_t k, uint32_t group,
                              uint32_t count);
hipError_t launch_direct(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                         uint32_t group, uint32_t flags, bool dense, void* workspace);

// onehot-mfma (vq4_onehot.hip): the automatic choice for products of at least
// kOneHotMinRows rows with B grouped along n: packed A grouped along k (g 16
// or 32), or dense activations (any group).
constexpr uint32_t kOneHotMinRows = 64;
constexpr uint32_t kOneHotMinRowsSmall = 8;   // from here when B holds >= 2^20 values
constexpr uint32_t kOneHotMinRowsDense = 9;   // the same for dense activations
bool onehot_applies(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                    uint32_t count);
bool onehot_applies_dense(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                          uint32_t count);
size_t onehot_workspace_bytes(uint32_t m, uint32_t n, uint32_t k, uint32_t group);
// dense activations: the nibble columns and, on large grids, x's bf16 planes
size_t onehot_dense_workspace_bytes(uint32_t m, uint32_t n, uint32_t k, uint32_t group);
hipError_t launch_onehot(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                         uint32_t group, bool dense, void* workspace);

// Bytes of device workspace a path needs (split-k partials, counters).
size_t matmul_workspace_bytes(MatmulPath p, uint32_t m, uint32_t n, uint32_t k, uint32_t group,
                              uint32_t flags, uint32_t count);

hipError_t launch_encode(hipStream_t s, const Operands& o, uint32_t m, uint32_t group);

hipError_t launch_decode(hipStream_t s, const Operands& o, uint32_t m, uint32_t group);
hipError_t launch_adamw(hipStream_t s, const Operands& o, uint32_t m, uint32_t group);
hipError_t launch_matmul(hipStream_t s, const Operands& o, uint32_t m, uint32_t n, uint32_t k,
                         uint32_t group, uint32_t flags, MatmulPath path, void* workspace,
                         size_t workspace_bytes);

// The dense-activation product: op 2's geometry and flags with A a dense FP32
// array in in[0] (in[1] unused). Paths: onehot-mfma (m >= 9 with B of at least
// 2^20 values, every m >= 64), the GEMV paths (m <= 8, and up to 64 rows in
// chunks of 8 where the one-hot path does not apply, such as A stored k x m;
// each window's fixed-point scale comes from x itself), else General.
MatmulPath choose_dense_path(uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                             uint32_t count, uint32_t policy);
size_t dense_workspace_bytes(MatmulPath p, uint32_t m, uint32_t n, uint32_t k, uint32_t group,
                             uint32_t flags, uint32_t count);
hipError_t launch_matmul_dense(hipStream_t s, const Operands& o, uint32_t m, uint32_t n,
                               uint32_t k, uint32_t group, uint32_t flags, MatmulPath path,
                               void* workspace, size_t workspace_bytes);

// Fused VQAdamW passes (ack_vq_adamw_step). codes4/books4/coeffs are the
// op-3 inputs.
struct AdamwInputs {
  const uint32_t* codes4;
  const float* books4;
  const float* coeffs;
  uint32_t m;
  uint32_t group;
};

// Device codebook calibration (fit_codebook, vq.py:182-257) for `problems`
// independent fits that share one geometry. Per problem p the buffers are
// laid out back to back: sample [count][G] FP32 (the strided sample of
// complete vectors), idx [count] entry indices, book [16][G] (the working
// and final book), flags [4] (used mask, kept mask, keep-pass switch, spare),
// gaps [17][count] float64 (the reseeds' per-row gaps over updated entries and
// their suffix minima over untouched ones).
struct FitArgs {
  const float* sample = nullptr;
  uint8_t* idx = nullptr;
  float* book = nullptr;
  uint32_t* flags = nullptr;
  double* gaps = nullptr;
  double* book64 = nullptr;   // float64 copy of the books for the keep pass (problems x 16 x group)
  uint32_t count = 0;         // sample vectors per problem
  uint64_t complete = 0;      // complete vectors of the tensor being fitted
  uint32_t* status = nullptr;
};

// What the warm-start keep rule re-encodes when it needs the whole tensor.
struct FitWhole {
  const float* values = nullptr;   // dense tensor (one problem), or
  const AdamwInputs* adamw = nullptr;  // the three AdamW states (problems 0..2)
};

// Samples rows linspace(0, complete-1, count) of a dense tensor into
// a.sample, and sets up a one-problem fit: book = init or the sample's rows
// linspace(0, count-1, 16), flags cleared. A nonfinite sampled or init value
// sets status bit 1.
hipError_t launch_fit_sample_dense(hipStream_t s, const float* values, uint32_t group,
                                   const FitArgs& a, const float* init);
// The Lloyd iterations: book = init (problem p at init + p * 16 * group) or
// sample rows linspace(0, count-1, 16) (unless `book_ready`: set up already,
// as launch_fit_sample_dense does), then `iterations` rounds of assign,
// optional keep pass over `whole`, and update. Enqueue only; allocates
// nothing.
hipError_t launch_fit(hipStream_t s, const FitArgs& a, uint32_t group, uint32_t problems,
                      uint32_t iterations, const float* init, const FitWhole& whole,
                      bool book_ready = false);

// AdamW at fit_codebook's strided sample of whole vectors (rows
// linspace(0, m/group - 1, count)): out = [3][count][group]. Also clears
// *changed, which the encode pass counts into, and sets up the three state
// fits as launch_fit would: fit_book = the W, M, V books (a nonfinite entry
// sets status bit 1), the fits' 12 flag words cleared.
hipError_t launch_adamw_gather(hipStream_t s, const AdamwInputs& in, uint32_t count, float* out,
                               uint32_t* changed, uint32_t* status, float* fit_book,
                               uint32_t* fit_flags);
// Keep pass of the fit over the three recomputed states (FitArgs problems
// 0..2): entries selected by complete vectors under the float64 rule, OR-ed
// into each problem's kept mask when its keep-pass switch is set.
hipError_t launch_adamw_keep(hipStream_t s, const AdamwInputs& in, const FitArgs& a);
// Recompute and encode all three states against books3; count changed W.
hipError_t launch_adamw_encode(hipStream_t s, const AdamwInputs& in, const float* books3,
                               uint32_t* out_codes, uint32_t* changed, uint32_t* status);

}  // namespace ackvq
