// CPU float64 encode and codebook calibration (vq.py:154-257), native.
//
// Every floating-point step is ordered as numpy orders it for the reference's
// expressions, so results are bit-identical to the Python on the same input:
// distances accumulate d = d + delta*delta over j (an explicit Python loop
// over j, vq.py:169-173); the cluster mean is a sequential float64 sum over
// the selected rows divided by their count (numpy's axis-0 reduction), then
// rounded to float32; the reseed gap sums the g squared differences in
// numpy's pairwise order for contiguous reductions (eight interleaved
// partial sums combined as ((r0+r1)+(r2+r3))+((r4+r5)+(r6+r7)), vq.py:255-256).
// Built with -ffp-contract=off: no fused multiply-adds.
#include "host_fit.hpp"

#include <cmath>
#include <cstring>
#include <vector>

namespace ackvq {
namespace {

constexpr int kEntries = 16;

// argmin over the 16 entries of the float64 distance of one vector, with
// np.argmin's rule: the first minimum, or the first NaN if there is one.
uint32_t nearest64(const float* x, uint32_t valid, const float* book, uint32_t g) {
  double best = 0.0;
  uint32_t sel = 0;
  for (uint32_t e = 0; e < kEntries; ++e) {
    double d = 0.0;
    for (uint32_t j = 0; j < valid; ++j) {
      const double delta = double(x[j]) - double(book[e * g + j]);
      d = d + delta * delta;
    }
    if (e == 0 || std::isnan(d) || d < best) {
      best = d;
      sel = e;
      if (std::isnan(d)) break;
    }
  }
  return sel;
}

double pairwise_sum(const double* v, uint32_t n) {
  if (n < 8) {
    double s = 0.0;
    for (uint32_t i = 0; i < n; ++i) s = s + v[i];
    return s;
  }
  double r[8];
  for (int j = 0; j < 8; ++j) r[j] = v[j];
  uint32_t i = 8;
  for (; i + 8 <= n; i += 8)
    for (int j = 0; j < 8; ++j) r[j] = r[j] + v[i + j];
  double res = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
  for (; i < n; ++i) res = res + v[i];
  return res;
}

// vq.py:232-257: the sample row with the largest distance to its nearest
// entry. min over entries propagates NaN; argmax takes the first maximum or
// the first NaN.
uint32_t reseed_row(const float* sample, uint32_t count, const float* book, uint32_t g) {
  std::vector<double> sq(g);
  double best_gap = 0.0;
  uint32_t best = 0;
  for (uint32_t i = 0; i < count; ++i) {
    double gap = 0.0;
    for (uint32_t e = 0; e < kEntries; ++e) {
      for (uint32_t j = 0; j < g; ++j) {
        const double d = double(sample[size_t(i) * g + j]) - double(book[e * g + j]);
        sq[j] = d * d;
      }
      const double s = pairwise_sum(sq.data(), g);
      if (e == 0 || std::isnan(s) || s < gap) gap = s;
      if (std::isnan(gap)) break;
    }
    if (i == 0 || std::isnan(gap) || gap > best_gap) {
      best_gap = gap;
      best = i;
      if (std::isnan(gap)) break;
    }
  }
  return best;
}

bool rows_equal(const float* a, const float* b, uint32_t g) {
  for (uint32_t j = 0; j < g; ++j)
    if (!(a[j] == b[j])) return false;
  return true;
}

struct DenseCtx {
  const float* values;
  uint64_t complete;
  uint32_t group;
};

int32_t dense_used(void* p, const float* book, uint32_t* mask) {
  const DenseCtx& c = *static_cast<const DenseCtx*>(p);
  uint32_t used = 0;
  for (uint64_t v = 0; v < c.complete; ++v)
    used |= 1u << nearest64(c.values + v * c.group, c.group, book, c.group);
  *mask = used;
  return 0;
}

}  // namespace

void linspace_index(uint64_t n, uint32_t num, uint32_t* out) {
  if (num == 0) return;
  if (num == 1) {
    out[0] = 0;
    return;
  }
  const double delta = double(n - 1);
  const double div = double(num - 1);
  const double step = delta / div;
  for (uint32_t i = 0; i < num; ++i) {
    double y;
    if (step == 0.0) {
      y = (double(i) / div) * delta;
    } else {
      y = double(i) * step;
    }
    y = y + 0.0;
    if (i == num - 1) y = delta;
    out[i] = uint32_t(std::floor(y));
  }
}

void host_encode64(const float* values, uint64_t m, const float* book, uint32_t group,
                   uint32_t* codes_out) {
  const uint64_t vectors = (m + group - 1) / group;
  const uint64_t words = (vectors + 7) / 8;
  std::memset(codes_out, 0, words * 4);
  for (uint64_t v = 0; v < vectors; ++v) {
    const uint64_t start = v * group;
    const uint32_t valid = uint32_t(m - start < group ? m - start : group);
    const uint32_t code = nearest64(values + start, valid, book, group);
    codes_out[v / 8] |= code << (4 * (v % 8));
  }
}

void host_fit_sample(const float* sample, uint32_t count, uint64_t complete, uint32_t g,
                     uint32_t iterations, const float* init, UsedMaskFn used_mask, void* ctx,
                     float* book) {
  if (init != nullptr) {
    std::memcpy(book, init, size_t(kEntries) * g * sizeof(float));
  } else {
    uint32_t rows[kEntries];
    linspace_index(count, kEntries, rows);
    for (int e = 0; e < kEntries; ++e)
      std::memcpy(book + e * g, sample + size_t(rows[e]) * g, g * sizeof(float));
  }
  std::vector<uint32_t> idx(count);
  std::vector<double> sum(g);
  for (uint32_t it = 0; it < iterations; ++it) {
    uint32_t used = 0;
    for (uint32_t i = 0; i < count; ++i) {
      idx[i] = nearest64(sample + size_t(i) * g, g, book, g);
      used |= 1u << idx[i];
    }
    bool reachable = false;
    for (uint32_t e = 0; e < kEntries && !reachable; ++e) {
      if (used & (1u << e)) continue;
      bool duplicate = false;
      for (uint32_t j = 0; j < e && !duplicate; ++j) duplicate = rows_equal(book + e * g, book + j * g, g);
      reachable = !duplicate;
    }
    uint32_t kept = 0;
    if (init != nullptr && count < complete && reachable) {
      if (used_mask(ctx, book, &kept) != 0) return;
    }
    for (uint32_t e = 0; e < kEntries; ++e) {
      uint64_t n = 0;
      for (uint32_t j = 0; j < g; ++j) sum[j] = 0.0;
      for (uint32_t i = 0; i < count; ++i) {
        if (idx[i] != e) continue;
        ++n;
        for (uint32_t j = 0; j < g; ++j) sum[j] = sum[j] + double(sample[size_t(i) * g + j]);
      }
      if (n) {
        for (uint32_t j = 0; j < g; ++j) book[e * g + j] = float(sum[j] / double(n));
      } else if (!(kept & (1u << e))) {
        const uint32_t row = reseed_row(sample, count, book, g);
        std::memcpy(book + e * g, sample + size_t(row) * g, g * sizeof(float));
      }
    }
  }
}

void host_fit_codebook(const float* values, uint64_t m, uint32_t g, uint32_t iterations,
                       uint32_t sample_vectors, const float* init, float* book_out) {
  const uint64_t complete = m / g;
  const uint32_t count = uint32_t(complete < sample_vectors ? complete : sample_vectors);
  std::vector<uint32_t> rows(count);
  linspace_index(complete, count, rows.data());
  std::vector<float> sample(size_t(count) * g);
  for (uint32_t i = 0; i < count; ++i)
    std::memcpy(sample.data() + size_t(i) * g, values + size_t(rows[i]) * g, g * sizeof(float));
  DenseCtx ctx{values, complete, g};
  host_fit_sample(sample.data(), count, complete, g, iterations, init, dense_used, &ctx, book_out);
}

}  // namespace ackvq
