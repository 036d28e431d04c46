// Host-side vq4 calibration: the CPU float64 encode and fit_codebook of
// src/alelyon_compute_kit/_kit/python/vq.py, restated in C++ so the
// optimizer step does not leave native code.
#pragma once

#include <cstdint>

namespace ackvq {

// floor(numpy.linspace(0, n - 1, num)) as int64 (numpy 2.x semantics: i *
// ((n - 1) / (num - 1)) in float64, last element exactly n - 1).
void linspace_index(uint64_t n, uint32_t num, uint32_t* out);

// vq.py:154-179: nearest entry by float64 squared distance summed over j in
// order, lowest index on ties; the final partial vector uses its valid
// values only. codes_out receives the packed words (unused nibbles zero).
void host_encode64(const float* values, uint64_t m, const float* book, uint32_t group,
                   uint32_t* codes_out);

// vq.py:182-229 on a dense tensor of m values.
void host_fit_codebook(const float* values, uint64_t m, uint32_t group, uint32_t iterations,
                       uint32_t sample_vectors, const float* init, float* book_out);

// The same fit given its strided sample (count x group values drawn by
// linspace_index from `complete` complete vectors). When the warm-start keep
// pass is due (vq.py:219-222), used_mask(ctx, book, &mask) must report which
// entries the whole tensor selects under `book`; it returns nonzero on
// failure, which ends the fit early.
using UsedMaskFn = int32_t (*)(void* ctx, const float* book, uint32_t* mask);
void host_fit_sample(const float* sample, uint32_t count, uint64_t complete, uint32_t group,
                     uint32_t iterations, const float* init, UsedMaskFn used_mask, void* ctx,
                     float* book_out);

}  // namespace ackvq
