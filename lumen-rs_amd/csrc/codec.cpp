// Host-side tables of the TurboQuant codebook format: the Lloyd-Max
// quantizer for N(0,1), the seeded Haar rotation and the QJL projection.
// Built once per cache (the reference caches them in OnceLock tables,
// turboquant.rs:214-331) and uploaded to the device.
//
// Lloyd-Max follows crates/lumen-core/src/lloyd_max.rs:35-122 step for step
// (f64 EM from a uniform start on [-3, 3], Abramowitz & Stegun 7.1.26 erf,
// symmetrization, midpoint boundaries), so its tables are bit-identical to
// the reference's. The rotation is a Haar orthogonal matrix by modified
// Gram-Schmidt QR with Mezzadri's sign fix (rotation.rs:35-89), drawn from
// this library's own N(0,1) stream (SplitMix64 uniforms, Box-Muller): the
// reference draws from rand's ChaCha12, which is not available here, so a
// caller that needs the reference's exact R passes it in (its TQRM file,
// rotation.rs:133-151). The QJL matrix is N(0,1)/sqrt(m) entries from the
// same stream at seed + 1 (qjl.rs:40-55, compressor.rs:24).
#include <cmath>
#include <cstring>
#include <vector>

#include "common.hpp"

namespace tqkv {
namespace {

constexpr double kPi = 3.14159265358979323846;

double erf_as(double x) {
  const double sign = std::copysign(1.0, x);  // Rust f64::signum: +1 at +0.0
  x = std::fabs(x);
  const double t = 1.0 / (1.0 + 0.3275911 * x);
  const double poly =
      t * (0.254829592 + t * (-0.284496736 + t * (1.421413741 + t * (-1.453152027 + t * 1.061405429))));
  return sign * (1.0 - poly * std::exp(-x * x));
}
double pdf(double x) { return std::exp(-0.5 * x * x) / std::sqrt(2.0 * kPi); }
double cdf(double x) { return 0.5 * (1.0 + erf_as(x * 0.70710678118654752440)); }
double cond_mean(double a, double b) {
  const double prob = cdf(b) - cdf(a);
  if (prob < 1e-15) return 0.5 * (a + b);
  return (pdf(a) - pdf(b)) / prob;
}

// N(0,1) draws: SplitMix64 uniforms through Box-Muller, both outputs used.
struct Normals {
  uint64_t s;
  bool have = false;
  double spare = 0.0;
  explicit Normals(uint64_t seed) : s(seed) {}
  uint64_t next_u64() {
    s += 0x9e3779b97f4a7c15ull;
    uint64_t z = s;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  }
  double next() {
    if (have) {
      have = false;
      return spare;
    }
    const double u1 = double((next_u64() >> 11) + 1) * 0x1.0p-53;  // (0, 1]
    const double u2 = double(next_u64() >> 11) * 0x1.0p-53;        // [0, 1)
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double a = 2.0 * kPi * u2;
    spare = r * std::sin(a);
    have = true;
    return r * std::cos(a);
  }
};

}  // namespace
}  // namespace tqkv

using namespace tqkv;

extern "C" {

int32_t tqkv_lloyd_max(uint32_t bits, size_t n_iter, double* boundaries, double* centroids) {
  if (bits == 0 || bits > 8) return fail(TQKV_EUNSUPPORTED, "codebook bits=%u not in 1..8", bits);
  if (!boundaries || !centroids) return fail(TQKV_EINVAL_ARG, "null pointer");
  const int n = 1 << bits;
  std::vector<double> c(static_cast<size_t>(n)), b(static_cast<size_t>(n) + 1, 0.0);
  for (int i = 0; i < n; ++i) c[i] = -3.0 + 6.0 * (double(i) + 0.5) / double(n);
  for (size_t it = 0; it < n_iter; ++it) {
    b[0] = -INFINITY;
    b[n] = INFINITY;
    for (int i = 1; i < n; ++i) b[i] = 0.5 * (c[i - 1] + c[i]);
    for (int i = 0; i < n; ++i) c[i] = cond_mean(b[i], b[i + 1]);
  }
  for (int i = 0; i < n / 2; ++i) {
    const double avg = 0.5 * (std::fabs(c[i]) + std::fabs(c[n - 1 - i]));
    c[i] = -avg;
    c[n - 1 - i] = avg;
  }
  b[0] = -INFINITY;
  b[n] = INFINITY;
  for (int i = 1; i < n; ++i) b[i] = 0.5 * (c[i - 1] + c[i]);
  std::memcpy(boundaries, b.data(), b.size() * sizeof(double));
  std::memcpy(centroids, c.data(), c.size() * sizeof(double));
  return ok();
}

int32_t tqkv_rotation_matrix(int32_t dim, uint64_t seed, float* out) {
  if (dim <= 0 || dim > 4096) return fail(TQKV_EINVAL_SHAPE, "dim=%d", dim);
  if (!out) return fail(TQKV_EINVAL_ARG, "null pointer");
  Normals ns(seed);
  const size_t d = size_t(dim);
  std::vector<double> cols(d * d);  // column j at [j * d, (j + 1) * d)
  for (size_t i = 0; i < d * d; ++i) cols[i] = ns.next();
  std::vector<double> rdiag(d);
  for (size_t j = 0; j < d; ++j) {
    double* cj = &cols[j * d];
    for (size_t k = 0; k < j; ++k) {
      const double* ck = &cols[k * d];
      double dot = -0.0;
      for (size_t i = 0; i < d; ++i) dot += ck[i] * cj[i];
      for (size_t i = 0; i < d; ++i) cj[i] -= dot * ck[i];
    }
    double ss = -0.0;
    for (size_t i = 0; i < d; ++i) ss += cj[i] * cj[i];
    const double norm = std::sqrt(ss);
    rdiag[j] = norm;
    const double inv = 1.0 / norm;
    for (size_t i = 0; i < d; ++i) cj[i] *= inv;
  }
  for (size_t j = 0; j < d; ++j) {
    const double sg = std::isnan(rdiag[j]) ? rdiag[j] : std::copysign(1.0, rdiag[j]);
    for (size_t i = 0; i < d; ++i) cols[j * d + i] *= sg;
  }
  for (size_t i = 0; i < d; ++i)
    for (size_t j = 0; j < d; ++j) out[i * d + j] = float(cols[j * d + i]);
  return ok();
}

int32_t tqkv_qjl_matrix(int32_t dim, int32_t m, uint64_t seed, float* out) {
  if (dim <= 0 || m <= 0) return fail(TQKV_EINVAL_SHAPE, "dim=%d m=%d", dim, m);
  if (!out) return fail(TQKV_EINVAL_ARG, "null pointer");
  Normals ns(seed);
  const float scale = 1.0f / std::sqrt(float(m));
  for (size_t i = 0; i < size_t(m) * size_t(dim); ++i) out[i] = float(ns.next()) * scale;
  return ok();
}

}  // extern "C"
