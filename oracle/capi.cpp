// extern "C" surface of the CPU oracle, loaded by tests/ through ctypes
// (test infrastructure only; see oracle.h).
#include <cmath>
#include <cstring>
#include <vector>

#include "oracle.h"

using namespace oracle;

extern "C" {

uint64_t oracle_golden_digest(const char* kind, const char* plan, int prealloc, int round_mode,
                              int wmax0, int clip_low) {
  AffineOpts ao;
  ao.round = round_mode ? RoundMode::HalfEven : RoundMode::HalfAway;
  ao.wmax_starts_at_zero = wmax0 != 0;
  ao.clip_low = clip_low != 0;
  return golden_digest(kind, plan, prealloc != 0, ao);
}

// Golden-plan input tape: returns the number of events (or -1 if the
// buffers are too small); events as (op, n, at) triples of int64.
int64_t oracle_golden_tape(const char* kind, const char* plan, int64_t* events,
                           int64_t max_events, uint8_t* data, int64_t data_cap,
                           int64_t* data_len, int64_t* max_size, int64_t* keep) {
  GoldenTape t = golden_tape(kind, plan);
  *data_len = int64_t(t.data.size());
  *max_size = t.max_size;
  *keep = t.keep;
  if (int64_t(t.events.size()) > max_events || int64_t(t.data.size()) > data_cap) return -1;
  for (size_t i = 0; i < t.events.size(); ++i) {
    events[3 * i] = t.events[i].op;
    events[3 * i + 1] = t.events[i].n;
    events[3 * i + 2] = t.events[i].at;
  }
  std::memcpy(data, t.data.data(), t.data.size());
  return int64_t(t.events.size());
}

// FNV-1a digest steps of golden_tests.rs:73-155: a number, raw bytes, and a
// [1, h, s, last] array of dtype 1 = u8, 2 = u32, 3 = f32, 4 = bf16.
uint64_t oracle_fnv_num(uint64_t h, uint64_t n) {
  Digest d;
  d.h = h;
  d.num(n);
  return d.h;
}
uint64_t oracle_fnv_array(uint64_t h, int dtype, int hh, int s, int last, const void* data) {
  Digest d;
  d.h = h;
  Arr a(DType(dtype), hh, s, last);
  if (!a.data.empty()) std::memcpy(a.data.data(), data, a.data.size());
  digest_array(d, a);
  return d.h;
}

// ---- numerics
void oracle_f32_to_bf16(const float* x, size_t n, uint16_t* out) {
  for (size_t i = 0; i < n; ++i) out[i] = f32_to_bf16(x[i]);
}

// ---- Lloyd-Max
int oracle_codebook(uint32_t bits, size_t n_iter, double* boundaries, double* centroids,
                    double* mse) {
  Codebook cb;
  if (!codebook_compute(bits, n_iter, &cb)) return -1;
  std::memcpy(boundaries, cb.boundaries.data(), cb.boundaries.size() * 8);
  std::memcpy(centroids, cb.centroids.data(), cb.centroids.size() * 8);
  *mse = cb.mse();
  return 0;
}

int oracle_codebook_quantize(uint32_t bits, const double* xs, size_t n, uint8_t* out) {
  Codebook cb;
  if (!codebook_compute(bits, 1000, &cb)) return -1;
  for (size_t i = 0; i < n; ++i) out[i] = cb.quantize(xs[i]);
  return 0;
}

// ---- rotation / QJL / bitpack
void oracle_rotation_random(int dim, uint64_t seed, float* out) {
  std::vector<float> r = rotation_random(dim, seed);
  std::memcpy(out, r.data(), r.size() * 4);
}
void oracle_rotation_apply(const float* R, int dim, const float* x, float* y) {
  rotation_apply(R, dim, x, y);
}
void oracle_rotation_apply_inverse(const float* R, int dim, const float* y, float* x) {
  rotation_apply_inverse(R, dim, y, x);
}
void oracle_qjl_random(int dim, int m, uint64_t seed, float* out) {
  std::vector<float> p = qjl_random(dim, m, seed);
  std::memcpy(out, p.data(), p.size() * 4);
}
size_t oracle_packed_words(size_t n, uint32_t bits) { return packed_words(n, bits); }
void oracle_pack_codes(const uint8_t* codes, size_t n, uint32_t bits, uint64_t* out) {
  std::vector<uint64_t> p = pack_codes(codes, n, bits);
  std::memcpy(out, p.data(), p.size() * 8);
}
void oracle_unpack_codes(const uint64_t* packed, size_t n, uint32_t bits, uint8_t* out) {
  std::vector<uint8_t> c = unpack_codes(packed, n, bits);
  std::memcpy(out, c.data(), n);
}
size_t oracle_qjl_packed_len(size_t m) { return qjl_packed_len(m); }
void oracle_qjl_project_and_pack(const float* phi, int m, int dim, const float* r,
                                 uint64_t* out) {
  std::vector<uint64_t> p = qjl_project_and_pack(phi, m, dim, r);
  std::memcpy(out, p.data(), p.size() * 8);
}
float oracle_qjl_estimate(const float* phi, int m, int dim, const float* q,
                          const uint64_t* packed, float rnorm) {
  std::vector<float> pq = qjl_project_query(phi, m, dim, q);
  return qjl_correction_from_projection(pq.data(), m, packed, rnorm);
}

// ---- TurboQuant compressor and SimpleCache-style attend.
// Compressed vectors are passed flat: stage1 [n, w1] u64, stage2 [n, w2] u64,
// rnorm [n] f32, scale [n] f32.
struct OracleCompressor {
  Compressor c;
};
void* oracle_compressor_new(int dim, uint32_t bits, int m, const float* R, const float* phi) {
  auto* oc = new OracleCompressor;
  oc->c.dim = dim;
  oc->c.bits = bits;
  oc->c.m = m;
  oc->c.R.assign(R, R + size_t(dim) * dim);
  oc->c.phi.assign(phi, phi + size_t(m) * dim);
  if (!codebook_compute(bits, 1000, &oc->c.cb)) {
    delete oc;
    return nullptr;
  }
  return oc;
}
void oracle_compressor_free(void* p) { delete static_cast<OracleCompressor*>(p); }

static void unflatten(const OracleCompressor* oc, size_t n, const uint64_t* s1,
                      const uint64_t* s2, const float* rn, const float* sc,
                      std::vector<Compressed>* out) {
  const size_t w1 = packed_words(size_t(oc->c.dim), oc->c.bits);
  const size_t w2 = qjl_packed_len(size_t(oc->c.m));
  out->resize(n);
  for (size_t t = 0; t < n; ++t) {
    (*out)[t].stage1.assign(s1 + t * w1, s1 + (t + 1) * w1);
    (*out)[t].stage2.assign(s2 + t * w2, s2 + (t + 1) * w2);
    (*out)[t].residual_norm = rn[t];
    (*out)[t].scale = sc[t];
  }
}

void oracle_compress(const void* p, const float* x, size_t n, uint64_t* s1, uint64_t* s2,
                     float* rn, float* sc) {
  const auto* oc = static_cast<const OracleCompressor*>(p);
  const size_t w1 = packed_words(size_t(oc->c.dim), oc->c.bits);
  const size_t w2 = qjl_packed_len(size_t(oc->c.m));
  for (size_t t = 0; t < n; ++t) {
    Compressed c = oc->c.compress_one(x + t * oc->c.dim);
    std::memcpy(s1 + t * w1, c.stage1.data(), w1 * 8);
    std::memcpy(s2 + t * w2, c.stage2.data(), w2 * 8);
    rn[t] = c.residual_norm;
    sc[t] = c.scale;
  }
}

void oracle_scores(const void* p, const float* q, size_t n, const uint64_t* s1,
                   const uint64_t* s2, const float* rn, const float* sc, int two_stage,
                   float* out) {
  const auto* oc = static_cast<const OracleCompressor*>(p);
  std::vector<Compressed> cs;
  unflatten(oc, n, s1, s2, rn, sc, &cs);
  std::vector<float> r = two_stage ? oc->c.scores_two_stage(q, cs) : oc->c.scores_stage1(q, cs);
  std::memcpy(out, r.data(), n * 4);
}

void oracle_attend_values(const void* p, const float* w, size_t n, const uint64_t* s1,
                          const uint64_t* s2, const float* rn, const float* sc, float* out) {
  const auto* oc = static_cast<const OracleCompressor*>(p);
  std::vector<Compressed> cs;
  unflatten(oc, n, s1, s2, rn, sc, &cs);
  std::vector<float> r = oc->c.attend_values(w, cs);
  std::memcpy(out, r.data(), size_t(oc->c.dim) * 4);
}

// ---- MLX affine
void oracle_affine_quantize(const uint16_t* w, size_t rows, int dim, int gs, int bits,
                            uint32_t* packed, uint16_t* scales, uint16_t* biases, int round_mode,
                            int wmax0, int clip_low) {
  AffineOpts ao;
  ao.round = round_mode ? RoundMode::HalfEven : RoundMode::HalfAway;
  ao.wmax_starts_at_zero = wmax0 != 0;
  ao.clip_low = clip_low != 0;
  affine_quantize_rows(w, rows, dim, gs, bits, packed, scales, biases, ao);
}
void oracle_affine_dequantize(const uint32_t* packed, const uint16_t* scales,
                              const uint16_t* biases, size_t rows, int dim, int gs, int bits,
                              uint16_t* out) {
  affine_dequantize_rows(packed, scales, biases, rows, dim, gs, bits, out);
}
void oracle_affine_dequantize_two_roundings(const uint32_t* packed, const uint16_t* scales,
                                            const uint16_t* biases, size_t rows, int dim, int gs,
                                            int bits, uint16_t* out) {
  affine_dequantize_rows(packed, scales, biases, rows, dim, gs, bits, out, true);
}
void oracle_affine_quantize_f32(const float* w, size_t rows, int dim, int gs, int bits,
                                uint32_t* packed, float* scales, float* biases, int round_mode,
                                int wmax0, int clip_low) {
  AffineOpts ao;
  ao.round = round_mode ? RoundMode::HalfEven : RoundMode::HalfAway;
  ao.wmax_starts_at_zero = wmax0 != 0;
  ao.clip_low = clip_low != 0;
  affine_quantize_rows_f32(w, rows, dim, gs, bits, packed, scales, biases, ao);
}
void oracle_affine_dequantize_f32(const uint32_t* packed, const float* scales,
                                  const float* biases, size_t rows, int dim, int gs, int bits,
                                  float* out) {
  affine_dequantize_rows_f32(packed, scales, biases, rows, dim, gs, bits, out);
}
void oracle_write_code(uint32_t* words, size_t i, int bits, uint32_t code) {
  write_code(words, i, bits, code);
}
uint32_t oracle_read_code(const uint32_t* words, size_t i, int bits) {
  return read_code(words, i, bits);
}

// ---- masks
int oracle_mask_allowed(size_t q_abs, size_t k_abs, long window) {
  return mask_allowed(q_abs, k_abs, window) ? 1 : 0;
}

}  // extern "C"
