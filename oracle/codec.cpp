// TurboQuant codec restated from lumen-core (test infrastructure only).
//
// Floating-point order follows the Rust exactly: every sum is sequential from
// index 0, products and sums round separately (no FMA; the file is built with
// -ffp-contract=off), normalisation is x * (1/sigma), and Lloyd-Max decisions
// compare in f64. Rust's f32 `Sum` folds from -0.0; only an all-zero product
// list can tell the seed apart, and the sign of that zero never reaches a
// code, scale or sign bit.
#include <cmath>
#include <cstring>

#include "oracle.h"

namespace oracle {
namespace {

constexpr double kPi = 3.14159265358979323846;
constexpr double kFrac1Sqrt2 = 0.70710678118654752440;

// lloyd_max.rs:35-38
double phi(double x) { return std::exp(-0.5 * x * x) / std::sqrt(2.0 * kPi); }

// lloyd_max.rs:47-55, Abramowitz & Stegun 7.1.26.
double erf_as(double x) {
  double sign = std::copysign(1.0, x);
  double ax = std::fabs(x);
  double t = 1.0 / (1.0 + 0.3275911 * ax);
  double poly =
      t * (0.254829592 +
           t * (-0.284496736 + t * (1.421413741 + t * (-1.453152027 + t * 1.061405429))));
  return sign * (1.0 - poly * std::exp(-ax * ax));
}

// lloyd_max.rs:41-44
double capital_phi(double x) { return 0.5 * (1.0 + erf_as(x * kFrac1Sqrt2)); }

// lloyd_max.rs:61-68
double conditional_expectation(double a, double b) {
  double prob = capital_phi(b) - capital_phi(a);
  if (prob < 1e-15) return 0.5 * (a + b);
  return (phi(a) - phi(b)) / prob;
}

// This build's N(0,1) stream for R and Phi: SplitMix64 -> two 53-bit
// uniforms -> Box-Muller in f64 (both outputs used).
struct NormalStream {
  SplitMix64 rng;
  bool have = false;
  double spare = 0.0;
  explicit NormalStream(uint64_t seed) : rng(seed) {}
  double next() {
    if (have) {
      have = false;
      return spare;
    }
    double u1 = double((rng.next() >> 11) + 1) * 0x1.0p-53;  // (0, 1]
    double u2 = double(rng.next() >> 11) * 0x1.0p-53;        // [0, 1)
    double r = std::sqrt(-2.0 * std::log(u1));
    double a = 2.0 * kPi * u2;
    spare = r * std::sin(a);
    have = true;
    return r * std::cos(a);
  }
};

}  // namespace

bool codebook_compute(uint32_t bits, size_t n_iter, Codebook* out) {
  if (bits == 0 || bits > 8) return false;
  const int n = 1 << bits;
  std::vector<double> c(n), b(n + 1, 0.0);
  for (int i = 0; i < n; ++i) c[i] = -3.0 + 6.0 * (double(i) + 0.5) / double(n);
  for (size_t it = 0; it < n_iter; ++it) {
    b[0] = -INFINITY;
    b[n] = INFINITY;
    for (int i = 1; i < n; ++i) b[i] = 0.5 * (c[i - 1] + c[i]);
    for (int i = 0; i < n; ++i) c[i] = conditional_expectation(b[i], b[i + 1]);
  }
  const int half = n / 2;
  for (int i = 0; i < half; ++i) {
    double avg = 0.5 * (std::fabs(c[i]) + std::fabs(c[n - 1 - i]));
    c[i] = -avg;
    c[n - 1 - i] = avg;
  }
  b[0] = -INFINITY;
  b[n] = INFINITY;
  for (int i = 1; i < n; ++i) b[i] = 0.5 * (c[i - 1] + c[i]);
  out->bits = bits;
  out->boundaries = b;
  out->centroids = c;
  return true;
}

// lloyd_max.rs:132-144 (linear scan)
uint8_t Codebook::quantize(double x) const {
  const int n = n_levels();
  for (int i = 1; i < n; ++i)
    if (x < boundaries[i]) return uint8_t(i - 1);
  return uint8_t(n - 1);
}

// lloyd_max.rs:165-187
double Codebook::mse() const {
  double total = 0.0;
  for (int i = 0; i < n_levels(); ++i) {
    double a = boundaries[i], b = boundaries[i + 1];
    double prob = capital_phi(b) - capital_phi(a);
    if (prob < 1e-15) continue;
    double cc = centroids[i];
    double ex = (phi(a) - phi(b)) / prob;
    double a_phi = std::isfinite(a) ? a * phi(a) : 0.0;
    double b_phi = std::isfinite(b) ? b * phi(b) : 0.0;
    double ex2 = 1.0 + (a_phi - b_phi) / prob;
    total += prob * (ex2 - 2.0 * cc * ex + cc * cc);
  }
  return total;
}

// rotation.rs:35-89
std::vector<float> rotation_random(int dim, uint64_t seed) {
  NormalStream ns(seed);
  std::vector<std::vector<double>> cols(dim, std::vector<double>(dim));
  for (int j = 0; j < dim; ++j)
    for (int i = 0; i < dim; ++i) cols[j][i] = ns.next();
  std::vector<double> rdiag(dim);
  for (int j = 0; j < dim; ++j) {
    for (int k = 0; k < j; ++k) {
      double dot = -0.0;
      for (int i = 0; i < dim; ++i) dot += cols[k][i] * cols[j][i];
      for (int i = 0; i < dim; ++i) cols[j][i] -= dot * cols[k][i];
    }
    double ss = -0.0;
    for (int i = 0; i < dim; ++i) ss += cols[j][i] * cols[j][i];
    double norm = std::sqrt(ss);
    rdiag[j] = norm;
    double inv = 1.0 / norm;
    for (int i = 0; i < dim; ++i) cols[j][i] *= inv;
  }
  for (int j = 0; j < dim; ++j) {
    double sg = std::isnan(rdiag[j]) ? rdiag[j] : std::copysign(1.0, rdiag[j]);
    for (int i = 0; i < dim; ++i) cols[j][i] *= sg;
  }
  std::vector<float> m(size_t(dim) * dim);
  for (int i = 0; i < dim; ++i)
    for (int j = 0; j < dim; ++j) m[size_t(i) * dim + j] = float(cols[j][i]);
  return m;
}

// rotation.rs:91-99
void rotation_apply(const float* R, int dim, const float* x, float* y) {
  for (int i = 0; i < dim; ++i) {
    const float* row = R + size_t(i) * dim;
    float acc = -0.0f;
    for (int j = 0; j < dim; ++j) acc += row[j] * x[j];
    y[i] = acc;
  }
}

// rotation.rs:102-113
void rotation_apply_inverse(const float* R, int dim, const float* y, float* x) {
  for (int i = 0; i < dim; ++i) x[i] = 0.0f;
  for (int j = 0; j < dim; ++j) {
    const float yj = y[j];
    const float* row = R + size_t(j) * dim;
    for (int i = 0; i < dim; ++i) x[i] += row[i] * yj;
  }
}

// bitpack.rs:11-14
size_t packed_words(size_t n, uint32_t bits) {
  size_t per = 64 / bits;
  return (n + per - 1) / per;
}

// bitpack.rs:17-31
std::vector<uint64_t> pack_codes(const uint8_t* codes, size_t n, uint32_t bits) {
  size_t per = 64 / bits;
  std::vector<uint64_t> out(packed_words(n, bits), 0);
  for (size_t i = 0; i < n; ++i) out[i / per] |= uint64_t(codes[i]) << ((i % per) * bits);
  return out;
}

// bitpack.rs:34-46
std::vector<uint8_t> unpack_codes(const uint64_t* packed, size_t n, uint32_t bits) {
  size_t per = 64 / bits;
  uint64_t mask = (uint64_t(1) << bits) - 1;
  std::vector<uint8_t> out(n);
  for (size_t i = 0; i < n; ++i) out[i] = uint8_t((packed[i / per] >> ((i % per) * bits)) & mask);
  return out;
}

// qjl.rs:40-51
std::vector<float> qjl_random(int dim, int m, uint64_t seed) {
  NormalStream ns(seed);
  float scale = 1.0f / std::sqrt(float(m));
  std::vector<float> phi(size_t(m) * dim);
  for (size_t i = 0; i < phi.size(); ++i) phi[i] = float(ns.next()) * scale;
  return phi;
}

// qjl.rs:33-36
size_t qjl_packed_len(size_t m) { return (m + 63) / 64; }

// qjl.rs:57-74
std::vector<uint64_t> qjl_project_and_pack(const float* phi, int m, int dim, const float* r) {
  std::vector<uint64_t> out(qjl_packed_len(size_t(m)), 0);
  for (int row = 0; row < m; ++row) {
    const float* p = phi + size_t(row) * dim;
    float dot = -0.0f;
    for (int j = 0; j < dim; ++j) dot += p[j] * r[j];
    if (dot >= 0.0f) out[row / 64] |= uint64_t(1) << (row % 64);
  }
  return out;
}

// qjl.rs:76-84
std::vector<float> qjl_project_query(const float* phi, int m, int dim, const float* q) {
  std::vector<float> out(m);
  for (int row = 0; row < m; ++row) {
    const float* p = phi + size_t(row) * dim;
    float dot = -0.0f;
    for (int j = 0; j < dim; ++j) dot += p[j] * q[j];
    out[row] = dot;
  }
  return out;
}

// qjl.rs:86-118
float qjl_correction_from_projection(const float* pq, int m, const uint64_t* packed, float rnorm) {
  if (rnorm < 1e-10f) return 0.0f;
  float sum = 0.0f;
  for (int row = 0; row < m; ++row) {
    float s = ((packed[row / 64] >> (row % 64)) & 1) ? 1.0f : -1.0f;
    sum += s * pq[row];
  }
  const float frac_pi_2 = 1.57079632679489661923f;
  float scale = rnorm * std::sqrt(frac_pi_2) / std::sqrt(float(m));
  return scale * sum;
}

// compressor.rs:61-107
Compressed Compressor::compress_one(const float* x) const {
  std::vector<float> y(dim), deq(dim), recon(dim), resid(dim);
  rotation_apply(R.data(), dim, x, y.data());
  float norm_sq = -0.0f;
  for (int i = 0; i < dim; ++i) norm_sq += y[i] * y[i];
  float scale = std::sqrt(norm_sq / float(dim));
  std::vector<uint8_t> codes(dim, 0);
  if (!(scale < 1e-10f)) {
    float inv = 1.0f / scale;
    for (int i = 0; i < dim; ++i) codes[i] = cb.quantize(double(y[i] * inv));
  }
  for (int i = 0; i < dim; ++i) deq[i] = float(cb.centroids[codes[i]]) * scale;
  rotation_apply_inverse(R.data(), dim, deq.data(), recon.data());
  float rn = 0.0f;
  for (int i = 0; i < dim; ++i) {
    resid[i] = x[i] - recon[i];
    rn += resid[i] * resid[i];
  }
  Compressed c;
  c.residual_norm = std::sqrt(rn);
  c.stage2 = qjl_project_and_pack(phi.data(), m, dim, resid.data());
  c.stage1 = pack_codes(codes.data(), size_t(dim), bits);
  c.scale = scale;
  return c;
}

// compressor.rs:165-184
std::vector<float> Compressor::scores_stage1(const float* q,
                                             const std::vector<Compressed>& cs) const {
  std::vector<float> rq(dim);
  rotation_apply(R.data(), dim, q, rq.data());
  std::vector<float> out(cs.size());
  for (size_t t = 0; t < cs.size(); ++t) {
    std::vector<uint8_t> codes = unpack_codes(cs[t].stage1.data(), size_t(dim), bits);
    float dot = -0.0f;
    for (int i = 0; i < dim; ++i) dot += rq[i] * float(cb.centroids[codes[i]]);
    out[t] = dot * cs[t].scale;
  }
  return out;
}

// compressor.rs:122-159
std::vector<float> Compressor::scores_two_stage(const float* q,
                                                const std::vector<Compressed>& cs) const {
  std::vector<float> s1 = scores_stage1(q, cs);
  std::vector<float> pq = qjl_project_query(phi.data(), m, dim, q);
  for (size_t t = 0; t < cs.size(); ++t)
    s1[t] = s1[t] + qjl_correction_from_projection(pq.data(), m, cs[t].stage2.data(),
                                                   cs[t].residual_norm);
  return s1;
}

// simple.rs:40-62 (accumulate_weighted_value) and :105-118 (attend_values)
std::vector<float> Compressor::attend_values(const float* w,
                                             const std::vector<Compressed>& cs) const {
  std::vector<float> out(dim, 0.0f);
  for (size_t t = 0; t < cs.size(); ++t) {
    if (std::fabs(w[t]) < 1e-10f) continue;
    std::vector<uint8_t> codes = unpack_codes(cs[t].stage1.data(), size_t(dim), bits);
    float sc = cs[t].scale * w[t];
    for (int j = 0; j < dim; ++j) {
      float yj = float(cb.centroids[codes[j]]) * sc;
      const float* row = R.data() + size_t(j) * dim;
      for (int i = 0; i < dim; ++i) out[i] += row[i] * yj;
    }
  }
  return out;
}

}  // namespace oracle
