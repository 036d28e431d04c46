/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle for the vq4/v1 kernels.
 *
 * A literal, scalar restatement of the reference shader
 * src/alelyon_compute_kit/_kit/kernels/vq4.comp, one function per op, in
 * IEEE single precision with every operation rounded (built with
 * -ffp-contract=off on x86-64 SSE: no fused multiply-add, no excess
 * precision). Division and square root are correctly rounded here; the
 * shader's are driver-precision (Vulkan allows 2.5 and 3 ULP), so only the
 * AdamW results carry that caveat. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, as the checker.
 *
 * Every function returns the status bits the shader would OR into its
 * status word (1 nonfinite, 2 layout, 4 optimizer domain), including the
 * codebook sweep of vq4.comp:149-158.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static int finite_value(float x) { return !isnan(x) && !isinf(x); }

static uint32_t div_up(uint32_t x, uint32_t d) { return x / d + (x % d != 0); }

/* words_for (vq4.comp:31) */
static uint32_t words_for(uint32_t values, uint32_t group) {
  return div_up(div_up(values, group), 8u);
}

/* The codebook sweep of vq4.comp:153-158 over `values` entries. */
static uint32_t sweep(const float* book, uint32_t values) {
  for (uint32_t j = 0; j < values; ++j)
    if (!finite_value(book[j])) return 1u;
  return 0u;
}

/* unpack_a / unpack_b (vq4.comp:64-73) */
static float unpack(const uint32_t* codes, const float* book, uint32_t logical, uint32_t group) {
  uint32_t vector = logical / group;
  uint32_t code = (codes[vector / 8u] >> (4u * (vector % 8u))) & 15u;
  return book[code * group + logical % group];
}

/* op 0: encode_word for every word (vq4.comp:118-144, :159-160). */
uint32_t oracle_encode(const float* x, uint32_t m, const float* book, uint32_t group,
                       uint32_t* out) {
  uint32_t status = sweep(book, 16u * group);
  uint32_t vectors = div_up(m, group);
  uint32_t words = words_for(m, group);
  for (uint32_t word = 0; word < words; ++word) {
    uint32_t packed = 0u;
    for (uint32_t nibble = 0; nibble < 8u; ++nibble) {
      uint32_t vector = word * 8u + nibble;
      if (vector >= vectors) break;
      uint32_t start = vector * group;
      uint32_t valid = group < m - start ? group : m - start;
      float best = INFINITY;
      uint32_t selected = 0u;
      for (uint32_t code = 0; code < 16u; ++code) {
        float distance = 0.0f;
        for (uint32_t j = 0; j < valid; ++j) {
          float value = x[start + j];
          float b = book[code * group + j];
          float delta = value - b;
          float squared = delta * delta;
          distance = distance + squared;
          if (!finite_value(value) || !finite_value(b) || !finite_value(distance)) status |= 1u;
        }
        if (distance < best) {
          best = distance;
          selected = code;
        }
      }
      packed |= selected << (4u * nibble);
    }
    out[word] = packed;
  }
  return status;
}

/* op 1 (vq4.comp:161-162): a bit copy through memcpy, so NaN payloads survive. */
uint32_t oracle_decode(const uint32_t* codes, const float* book, uint32_t m, uint32_t group,
                       float* out) {
  uint32_t status = sweep(book, 16u * group);
  for (uint32_t i = 0; i < m; ++i) {
    uint32_t vector = i / group;
    uint32_t code = (codes[vector / 8u] >> (4u * (vector % 8u))) & 15u;
    memcpy(&out[i], &book[code * group + i % group], sizeof(float));
  }
  return status;
}

/* op 2 (vq4.comp:165-176): sequential FP32 sum over inner, product and total
 * each rounded. flags bit0: A stored (k, m); bit1: B stored (n, k). */
uint32_t oracle_matmul(const uint32_t* a_codes, const float* a_book, const uint32_t* b_codes,
                       const float* b_book, uint32_t m, uint32_t n, uint32_t k, uint32_t group,
                       uint32_t flags, float* out) {
  uint32_t status = sweep(a_book, 16u * group) | sweep(b_book, 16u * group);
  for (uint32_t row = 0; row < m; ++row) {
    for (uint32_t col = 0; col < n; ++col) {
      float total = 0.0f;
      for (uint32_t inner = 0; inner < k; ++inner) {
        uint32_t ai = (flags & 1u) ? inner * m + row : row * k + inner;
        uint32_t bi = (flags & 2u) ? col * k + inner : inner * n + col;
        float product = unpack(a_codes, a_book, ai, group) * unpack(b_codes, b_book, bi, group);
        total = total + product;
        if (!finite_value(product) || !finite_value(total)) status |= 1u;
      }
      out[(size_t)row * n + col] = total;
    }
  }
  return status;
}

/* The dense-activation product (libackvq's ack_vq_matmul_dense, an extension
 * with no reference counterpart): op 2's loop (vq4.comp:165-176) with A read
 * from a dense FP32 array at the flat index the packed A would be decoded at.
 * Pinned by the op-2 oracle: with x = decode(A) it must equal oracle_matmul
 * bit for bit (tests/test_oracle.py). */
uint32_t oracle_matmul_dense(const float* x, const uint32_t* b_codes, const float* b_book,
                             uint32_t m, uint32_t n, uint32_t k, uint32_t group, uint32_t flags,
                             float* out) {
  uint32_t status = sweep(b_book, 16u * group);
  for (uint32_t row = 0; row < m; ++row) {
    for (uint32_t col = 0; col < n; ++col) {
      float total = 0.0f;
      for (uint32_t inner = 0; inner < k; ++inner) {
        uint32_t ai = (flags & 1u) ? inner * m + row : row * k + inner;
        uint32_t bi = (flags & 2u) ? col * k + inner : inner * n + col;
        float product = x[ai] * unpack(b_codes, b_book, bi, group);
        total = total + product;
        if (!finite_value(product) || !finite_value(total)) status |= 1u;
      }
      out[(size_t)row * n + col] = total;
    }
  }
  return status;
}

/* op 3 (vq4.comp:80-116, :163-164). Elements the shader returns from early
 * are left unwritten in out (3m floats). */
uint32_t oracle_adamw(const uint32_t* codes4, const float* books4, const float* b2, uint32_t m,
                      uint32_t group, float* out) {
  uint32_t status = sweep(books4, 64u * group);
  uint32_t words = words_for(m, group);
  float lr = b2[0], beta1 = b2[1], beta2 = b2[2], eps = b2[3];
  float decay = b2[4], correction1 = b2[5], correction2 = b2[6];
  for (uint32_t i = 0; i < m; ++i) {
    int bad_coeff = 0;
    for (uint32_t j = 0; j < 7u; ++j)
      if (!finite_value(b2[j])) bad_coeff = 1;
    if (bad_coeff) {
      status |= 1u;
      continue;
    }
    if (lr < 0.0f || beta1 < 0.0f || beta1 >= 1.0f || beta2 < 0.0f || beta2 >= 1.0f ||
        eps <= 0.0f || decay < 0.0f || correction1 <= 0.0f || correction1 > 1.0f ||
        correction2 <= 0.0f || correction2 > 1.0f) {
      status |= 4u;
      continue;
    }
    float s[4];
    for (uint32_t state = 0; state < 4u; ++state) {
      uint32_t vector = i / group;
      uint32_t code = (codes4[state * words + vector / 8u] >> (4u * (vector % 8u))) & 15u;
      s[state] = books4[state * 16u * group + code * group + i % group];
    }
    float weight = s[0], moment = s[1], variance = s[2], gradient = s[3];
    if (!finite_value(weight) || !finite_value(moment) || !finite_value(variance) ||
        !finite_value(gradient)) {
      status |= 1u;
      continue;
    }
    if (variance < 0.0f) {
      status |= 4u;
      continue;
    }
    float t1 = beta1 * moment;
    float t2 = (1.0f - beta1) * gradient;
    float next_m = t1 + t2;
    float u1 = beta2 * variance;
    float gg = gradient * gradient;
    float u2 = (1.0f - beta2) * gg;
    float next_v = u1 + u2;
    float corrected_m = next_m / correction1;
    float corrected_v = next_v / correction2;
    float denominator = sqrtf(corrected_v) + eps;
    float decayed = weight * (1.0f - lr * decay);
    float step = lr * corrected_m / denominator;
    float next_w = decayed - step;
    if (!finite_value(next_m) || !finite_value(next_v) || !finite_value(corrected_m) ||
        !finite_value(corrected_v) || !finite_value(denominator) || !finite_value(decayed) ||
        !finite_value(next_w))
      status |= 1u;
    out[i] = next_w;
    out[m + i] = next_m;
    out[2u * m + i] = next_v;
  }
  return status;
}
