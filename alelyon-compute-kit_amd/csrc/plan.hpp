// vq4/v1 admission: a closed 32-byte plan block [op,m,n,k,group,16,flags,0]
// is turned into per-slot byte requirements, a work-item count and the
// reference's two-dimensional 64-wide grid, or refused by name.
//
// Restates the reference's pure admission module
// (src/alelyon_compute_kit/_kit/src/vq4_ops.rs:13-243): the same check order
// (from_words :111-183), the same byte formulas, the same alias rules
// (validate_buffers :188-209) and the same refusal names (:66-84). One bound is
// this library's own: the reference caps one dispatch at 2^28 multiply-adds
// because its shader is a scalar loop (vq4_ops.rs:21-23); the kernels here are
// tiled and admit up to 2^38 (kMaxMatmulMacs). The reference bound stays
// available as Bounds::Reference so its known-answer tests still run.
//
// Header-only and free of any GPU dependency so the host can be tested on a
// machine without a device.
#pragma once

#include <array>
#include <cstdint>
#include <string>

namespace ackvq {

constexpr uint32_t kSchema = 1;
constexpr int kOperands = 6;
constexpr size_t kPushBytes = 32;
constexpr uint32_t kEntries = 16;
constexpr uint32_t kIndicesPerWord = 8;
constexpr uint32_t kWorkgroupSize = 64;
constexpr uint32_t kMaxValues = 1u << 28;
constexpr uint32_t kMaxDim = 65536;
// The reference's scalar-shader bound (vq4_ops.rs:23).
constexpr uint64_t kReferenceMaxMatmulMacs = 1ull << 28;
// This library's bound: the largest single product it admits. It covers the
// 2048 x 14336 x 4096 prefill product (2^36.8 multiply-adds) in one call.
constexpr uint64_t kMaxMatmulMacs = 1ull << 38;
constexpr uint32_t kGridX = 65535;

enum class Op : uint32_t { Encode = 0, Decode = 1, Matmul = 2, AdamW = 3 };

enum class Bounds : uint32_t { Library = 0, Reference = 1 };

enum class PlanError : int {
  None = 0,
  Operation,
  Group,
  Entries,
  Flags,
  Reserved,
  Geometry,
  AddressLimit,
  WorkLimit,
  Capacity,
  NullIdentity,
  OutputAlias,
  StatusAlias,
  Dispatch,
};

// Names match the reference's Display strings (vq4_ops.rs:66-84).
inline std::string plan_error_name(PlanError e, int slot = 0) {
  switch (e) {
    case PlanError::None: return "ok";
    case PlanError::Operation: return "vq-operation-out-of-range";
    case PlanError::Group: return "vq-unsupported-group";
    case PlanError::Entries: return "vq-codebook-entries-not-16";
    case PlanError::Flags: return "vq-unsupported-flags";
    case PlanError::Reserved: return "vq-nonzero-reserved-word";
    case PlanError::Geometry: return "vq-invalid-geometry";
    case PlanError::AddressLimit: return "vq-address-limit-exceeded";
    case PlanError::WorkLimit: return "vq-matmul-work-limit";
    case PlanError::Capacity: return "vq-binding-" + std::to_string(slot) + "-too-small";
    case PlanError::NullIdentity: return "vq-null-allocation-identity";
    case PlanError::OutputAlias: return "vq-output-aliases-input";
    case PlanError::StatusAlias: return "vq-status-aliases-operand";
    case PlanError::Dispatch: return "vq-dispatch-grid-unsupported";
  }
  return "vq-unknown";
}

inline uint32_t div_up(uint32_t x, uint32_t d) { return x / d + (x % d != 0); }

// Packed u32 words for `values` logical values at `group` (vq4.comp words_for).
inline uint32_t packed_words(uint32_t values, uint32_t group) {
  return div_up(div_up(values, group), kIndicesPerWord);
}

inline uint64_t packed_bytes(uint32_t values, uint32_t group) {
  return uint64_t(packed_words(values, group)) * 4;
}

struct Plan {
  std::array<uint32_t, 8> words{};
  Op op = Op::Encode;
  std::array<uint64_t, kOperands> required_bytes{};
  uint32_t work_items = 0;
  std::array<uint32_t, 3> dispatch{};

  uint32_t m() const { return words[1]; }
  uint32_t n() const { return words[2]; }
  uint32_t k() const { return words[3]; }
  uint32_t group() const { return words[4]; }
  uint32_t flags() const { return words[6]; }
};

namespace detail {
inline PlanError product(uint32_t a, uint32_t b, uint32_t* out) {
  uint64_t v = uint64_t(a) * uint64_t(b);
  if (v > kMaxValues) return PlanError::AddressLimit;
  *out = uint32_t(v);
  return PlanError::None;
}
}  // namespace detail

// VqPlan::from_words (vq4_ops.rs:111-183), check for check.
inline PlanError plan_from_words(const std::array<uint32_t, 8>& words, Bounds bounds, Plan* plan) {
  const uint32_t op_word = words[0], m = words[1], n = words[2], k = words[3];
  const uint32_t group = words[4], entries = words[5], flags = words[6], reserved = words[7];
  if (op_word > 3) return PlanError::Operation;
  const Op op = Op(op_word);
  if (!(group == 8 || group == 16 || group == 32)) return PlanError::Group;
  if (entries != kEntries) return PlanError::Entries;
  if (reserved != 0) return PlanError::Reserved;
  if ((op == Op::Matmul && flags > 3) || (op != Op::Matmul && flags != 0)) return PlanError::Flags;
  if (m == 0 || n == 0 || k == 0) return PlanError::Geometry;
  const uint64_t book = uint64_t(kEntries * group) * 4;
  std::array<uint64_t, kOperands> req{};
  uint32_t work = 0;
  if (op != Op::Matmul) {
    if (n != 1 || k != 1) return PlanError::Geometry;
    if (m > kMaxValues) return PlanError::AddressLimit;
    const uint64_t packed = packed_bytes(m, group);
    const uint64_t dense = uint64_t(m) * 4;
    if (op == Op::Encode) {
      req = {dense, book, 0, 0, packed, 4};
      work = uint32_t(packed / 4);
    } else if (op == Op::Decode) {
      req = {packed, book, 0, 0, dense, 4};
      work = m;
    } else {
      uint32_t unused;
      if (PlanError e = detail::product(m, 3, &unused); e != PlanError::None) return e;
      req = {4 * packed, 4 * book, 7 * 4, 0, 3 * dense, 4};
      work = m;
    }
  } else {
    if (m > kMaxDim || n > kMaxDim || k > kMaxDim) return PlanError::Geometry;
    uint32_t a, b, c;
    if (PlanError e = detail::product(m, k, &a); e != PlanError::None) return e;
    if (PlanError e = detail::product(k, n, &b); e != PlanError::None) return e;
    if (PlanError e = detail::product(m, n, &c); e != PlanError::None) return e;
    const uint64_t limit = bounds == Bounds::Reference ? kReferenceMaxMatmulMacs : kMaxMatmulMacs;
    if (uint64_t(c) * uint64_t(k) > limit) return PlanError::WorkLimit;
    req = {packed_bytes(a, group), book, packed_bytes(b, group), book, uint64_t(c) * 4, 4};
    work = c;
  }
  const uint32_t groups = div_up(work, kWorkgroupSize);
  const uint32_t x = groups < kGridX ? groups : kGridX;
  plan->words = words;
  plan->op = op;
  plan->required_bytes = req;
  plan->work_items = work;
  plan->dispatch = {x, div_up(groups, x), 1};
  return PlanError::None;
}

// VqPlan::validate_buffers (vq4_ops.rs:188-209). Read slots may share an
// allocation; the output and the status word must differ from every read
// slot, including slots the operation does not read.
inline PlanError validate_buffers(const Plan& plan, const uint64_t capacities[kOperands],
                                  const uint64_t ids[kOperands], int* slot_out) {
  for (int i = 0; i < kOperands; ++i)
    if (ids[i] == 0) return PlanError::NullIdentity;
  for (int i = 0; i < kOperands; ++i) {
    if (capacities[i] < plan.required_bytes[i]) {
      if (slot_out) *slot_out = i;
      return PlanError::Capacity;
    }
  }
  for (int i = 0; i < 4; ++i)
    if (ids[i] == ids[4]) return PlanError::OutputAlias;
  for (int i = 0; i < 5; ++i)
    if (ids[i] == ids[5]) return PlanError::StatusAlias;
  return PlanError::None;
}

// VqPlan::validate_dispatch (vq4_ops.rs:211-222).
inline PlanError validate_dispatch(const Plan& plan, const uint32_t limits[3]) {
  for (int i = 0; i < 3; ++i)
    if (plan.dispatch[i] == 0 || plan.dispatch[i] > limits[i]) return PlanError::Dispatch;
  return PlanError::None;
}

}  // namespace ackvq
