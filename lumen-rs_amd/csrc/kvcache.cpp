// The reference's CPU cache API, turboquant_cache::KVCache
// (crates/turboquant-cache/src/traits.rs:9-36) as SimpleCache implements it
// (simple.rs:13-149), with the compressed vectors kept on the device and the
// compression and estimators run by the kernels of turboquant.hip. Host
// pointers in and out, synchronous, like the trait's borrowed slices and
// owned Vecs. Storage per (layer, head), keys and values alike: the codes in
// CompressedVector::stage1_packed's layout (u64 words, 64 / bits codes a
// word, LSB first, none straddling: bitpack.rs:11-52), scale f32, QJL signs
// u32 [ceil(m/32)] and residual norm f32 per token, in arrays that double
// when full. The encode writes one byte per code into staging and packs it
// on the device; the estimators read the packed words directly.
#include <cstring>
#include <new>
#include <vector>

#include "common.hpp"

extern "C" {
int32_t tqkv_lloyd_max(uint32_t bits, size_t n_iter, double* boundaries, double* centroids);
int32_t tqkv_rotation_matrix(int32_t dim, uint64_t seed, float* out);
int32_t tqkv_qjl_matrix(int32_t dim, int32_t m, uint64_t seed, float* out);
int32_t tqkv_tq_encode(const void* x, int32_t x_is_bf16, int64_t n_slabs, int64_t s, int32_t dim,
                       const float* rotation, const double* boundaries, const float* centroids_f32,
                       int32_t bits, const float* qjl, int32_t qjl_m, uint8_t* codes, float* sigma,
                       uint32_t* signs, float* rnorm, int64_t dst_cap, int64_t dst_start,
                       tqkv_stream stream);
int32_t tqkv_tq_rotate_query(const float* rotation, const float* q, int32_t dim, float* rq,
                             tqkv_stream stream);
int64_t tqkv_packed_words(int32_t dim, int32_t bits);
int32_t tqkv_pack_codes(const uint8_t* codes, int64_t n, int32_t dim, int32_t bits,
                        uint64_t* words, tqkv_stream stream);
int32_t tqkv_unpack_codes(const uint64_t* words, int64_t n, int32_t dim, int32_t bits,
                          uint8_t* codes, tqkv_stream stream);
int32_t tqkv_tq_scores_packed(const float* rq, const uint64_t* words, const float* sigma,
                              const float* centroids_f32, int32_t bits, int32_t dim, int64_t n,
                              float* scores, tqkv_stream stream);
int32_t tqkv_tq_values_packed(const float* rotation, const uint64_t* words, const float* sigma,
                              const float* centroids_f32, const float* weights, int32_t bits,
                              int32_t dim, int64_t n, float* out, tqkv_stream stream);
}

namespace tqkv {
namespace {

template <typename T>
int32_t dalloc(T** p, size_t n) {
  void* v = nullptr;
  if (hipMalloc(&v, n * sizeof(T) + 1) != hipSuccess)
    return fail(TQKV_ENOMEM, "hipMalloc of %zu bytes failed", n * sizeof(T));
  *p = static_cast<T*>(v);
  return TQKV_OK;
}

// The compressed vectors of one (layer, head, keys|values) on the device.
struct Stream {
  uint64_t* words = nullptr;  // packed codes [cap, words a vector]
  float* sigma = nullptr;
  uint32_t* signs = nullptr;
  float* rnorm = nullptr;
  int64_t n = 0, cap = 0;
};

}  // namespace
}  // namespace tqkv

using namespace tqkv;

struct tqkv_kvcache {
  tqkv_tq_config cfg{};
  int n_layers = 0, n_heads = 0;
  int words = 0;  // QJL u32 words per vector
  int pw = 0;     // packed code u64 words per vector
  float* R = nullptr;
  float* phi = nullptr;
  double* bnd = nullptr;
  float* cent = nullptr;
  float* scratch = nullptr;  // staging for inputs, queries, weights and outputs
  size_t scratch_floats = 0;
  std::vector<Stream> keys, values;  // [layer * n_heads + head]
};

namespace {

void free_stream(Stream& s) {
  (void)hipFree(s.words);
  (void)hipFree(s.sigma);
  (void)hipFree(s.signs);
  (void)hipFree(s.rnorm);
  s = Stream{};
}

int32_t reserve(const tqkv_kvcache* c, Stream& s, int64_t need) {
  if (need <= s.cap) return TQKV_OK;
  int64_t cap = s.cap ? s.cap : 64;
  while (cap < need) cap *= 2;
  const int PW = c->pw, W = c->words;
  Stream ns;
  ns.n = s.n;
  ns.cap = cap;
  int32_t rc = dalloc(&ns.words, size_t(cap) * PW);
  if (!rc) rc = dalloc(&ns.sigma, size_t(cap));
  if (!rc) rc = dalloc(&ns.signs, size_t(cap) * (W ? W : 1));
  if (!rc) rc = dalloc(&ns.rnorm, size_t(cap));
  if (rc) {
    free_stream(ns);
    return rc;
  }
  if (s.n > 0) {
    TQKV_HIP(hipMemcpy(ns.words, s.words, size_t(s.n) * PW * 8, hipMemcpyDeviceToDevice));
    TQKV_HIP(hipMemcpy(ns.sigma, s.sigma, size_t(s.n) * 4, hipMemcpyDeviceToDevice));
    if (W) TQKV_HIP(hipMemcpy(ns.signs, s.signs, size_t(s.n) * W * 4, hipMemcpyDeviceToDevice));
    TQKV_HIP(hipMemcpy(ns.rnorm, s.rnorm, size_t(s.n) * 4, hipMemcpyDeviceToDevice));
  }
  free_stream(s);
  s = ns;
  return TQKV_OK;
}

int32_t staging(tqkv_kvcache* c, size_t floats, float** out) {
  if (c->scratch_floats < floats) {
    (void)hipFree(c->scratch);
    c->scratch = nullptr;
    c->scratch_floats = 0;
    if (int32_t rc = dalloc(&c->scratch, floats)) return rc;
    c->scratch_floats = floats;
  }
  *out = c->scratch;
  return TQKV_OK;
}

int32_t check_lh(const tqkv_kvcache* c, int32_t layer, int32_t head) {
  if (!c) return fail(TQKV_EINVAL_ARG, "null cache");
  if (layer < 0 || layer >= c->n_layers || head < 0 || head >= c->n_heads)
    return fail(TQKV_EINVAL_ARG, "layer %d / head %d out of range (%d x %d)", layer, head,
                c->n_layers, c->n_heads);
  return TQKV_OK;
}

int32_t encode_into(tqkv_kvcache* c, Stream& s, const float* host, int64_t n) {
  const int D = c->cfg.head_dim, W = c->words;
  if (int32_t rc = reserve(c, s, s.n + n)) return rc;
  // Staging: x f32 [n, D], sigma [n], residual norms [n], signs u32
  // [n, max(W, 1)], then the encode's codes u8 [n, D]. The encode writes
  // them all at rows [0, n); the codes are packed into the stream and the
  // rest copied to rows [s.n, s.n + n) of it.
  // (codes start on a 16-byte boundary, as the encode's 16-byte stores want).
  const size_t nd = size_t(n) * D, ws = size_t(W ? W : 1);
  const size_t codes_at = (nd + 2 * size_t(n) + size_t(n) * ws + 3) / 4 * 4;
  float* x = nullptr;
  if (int32_t rc = staging(c, codes_at + (nd + 3) / 4, &x)) return rc;
  float* sigma = x + nd;
  float* rnorm = sigma + n;
  uint32_t* signs = reinterpret_cast<uint32_t*>(rnorm + n);
  uint8_t* codes = reinterpret_cast<uint8_t*>(x + codes_at);
  TQKV_HIP(hipMemcpy(x, host, nd * 4, hipMemcpyHostToDevice));
  if (int32_t rc = tqkv_tq_encode(x, 0, 1, n, D, c->R, c->bnd, c->cent, c->cfg.bits, c->phi,
                                  c->cfg.qjl_m, codes, sigma, signs, rnorm, n, 0, nullptr))
    return rc;
  const int64_t at = s.n;
  if (int32_t rc = tqkv_pack_codes(codes, n, D, c->cfg.bits, s.words + at * c->pw, nullptr))
    return rc;
  TQKV_HIP(hipMemcpy(s.sigma + at, sigma, size_t(n) * 4, hipMemcpyDeviceToDevice));
  if (W) {
    TQKV_HIP(hipMemcpy(s.signs + at * W, signs, size_t(n) * W * 4, hipMemcpyDeviceToDevice));
    TQKV_HIP(hipMemcpy(s.rnorm + at, rnorm, size_t(n) * 4, hipMemcpyDeviceToDevice));
  }
  TQKV_HIP(hipDeviceSynchronize());
  s.n += n;
  return TQKV_OK;
}

}  // namespace

extern "C" {

int32_t tqkv_kvcache_create(const tqkv_tq_config* cfg, const float* rotation, const float* qjl,
                            int32_t n_layers, int32_t n_kv_heads, tqkv_kvcache** out) {
  if (!cfg || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  *out = nullptr;
  const int D = cfg->head_dim, m = cfg->qjl_m;
  if (n_layers <= 0 || n_kv_heads <= 0) return fail(TQKV_EINVAL_SHAPE, "%d layers, %d heads", n_layers, n_kv_heads);
  if (!(D == 64 || D == 128 || D == 256 || D == 512))
    return fail(TQKV_EUNSUPPORTED, "head_dim=%d not in {64,128,256,512}", D);
  if (cfg->bits < 1 || cfg->bits > 8 || m < 0) return fail(TQKV_EUNSUPPORTED, "bits=%d qjl_m=%d", cfg->bits, m);
  tqkv_kvcache* c = new (std::nothrow) tqkv_kvcache();
  if (!c) return fail(TQKV_ENOMEM, "cache object");
  c->cfg = *cfg;
  c->n_layers = n_layers;
  c->n_heads = n_kv_heads;
  c->words = (m + 31) / 32;
  c->pw = int(tqkv_packed_words(D, cfg->bits));
  c->keys.resize(size_t(n_layers) * n_kv_heads);
  c->values.resize(size_t(n_layers) * n_kv_heads);
  const int n = 1 << cfg->bits;
  std::vector<double> b(n + 1), ce(n);
  std::vector<float> cf(n), R(size_t(D) * D), P(size_t(m > 0 ? m : 1) * D);
  const size_t iters = cfg->lloyd_max_iter > 0 ? size_t(cfg->lloyd_max_iter) : 1000;
  int32_t rc = tqkv_lloyd_max(uint32_t(cfg->bits), iters, b.data(), ce.data());
  for (int i = 0; i < n; ++i) cf[i] = float(ce[i]);
  if (!rc) {
    if (rotation) std::memcpy(R.data(), rotation, R.size() * 4);
    else rc = tqkv_rotation_matrix(D, cfg->seed, R.data());
  }
  if (!rc && m > 0) {
    if (qjl) std::memcpy(P.data(), qjl, size_t(m) * D * 4);
    else rc = tqkv_qjl_matrix(D, m, cfg->seed + 1, P.data());
  }
  if (!rc) rc = dalloc(&c->R, R.size());
  if (!rc) rc = dalloc(&c->phi, P.size());
  if (!rc) rc = dalloc(&c->bnd, b.size());
  if (!rc) rc = dalloc(&c->cent, cf.size());
  if (!rc && hipMemcpy(c->R, R.data(), R.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
    rc = fail(TQKV_EDEVICE, "upload of R failed");
  if (!rc && hipMemcpy(c->phi, P.data(), P.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
    rc = fail(TQKV_EDEVICE, "upload of Phi failed");
  if (!rc && hipMemcpy(c->bnd, b.data(), b.size() * 8, hipMemcpyHostToDevice) != hipSuccess)
    rc = fail(TQKV_EDEVICE, "upload of the boundaries failed");
  if (!rc && hipMemcpy(c->cent, cf.data(), cf.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
    rc = fail(TQKV_EDEVICE, "upload of the centroids failed");
  if (rc) {
    tqkv_kvcache_destroy(c);
    return rc;
  }
  *out = c;
  return ok();
}

int32_t tqkv_kvcache_destroy(tqkv_kvcache* c) {
  if (!c) return ok();
  (void)hipDeviceSynchronize();
  for (Stream& s : c->keys) free_stream(s);
  for (Stream& s : c->values) free_stream(s);
  (void)hipFree(c->R);
  (void)hipFree(c->phi);
  (void)hipFree(c->bnd);
  (void)hipFree(c->cent);
  (void)hipFree(c->scratch);
  delete c;
  return ok();
}

int32_t tqkv_kvcache_store(tqkv_kvcache* c, int32_t layer, int32_t head, const float* keys,
                           const float* values, int64_t n_tokens) {
  if (int32_t rc = check_lh(c, layer, head)) return rc;
  if (n_tokens < 0) return fail(TQKV_EINVAL_SHAPE, "n_tokens=%lld", (long long)n_tokens);
  if (n_tokens == 0) return ok();
  if (!keys || !values) return fail(TQKV_EINVAL_ARG, "null pointer");
  const size_t at = size_t(layer) * c->n_heads + head;
  if (int32_t rc = encode_into(c, c->keys[at], keys, n_tokens)) return rc;
  if (int32_t rc = encode_into(c, c->values[at], values, n_tokens)) return rc;
  return ok();
}

int64_t tqkv_kvcache_seq_len(const tqkv_kvcache* c, int32_t layer, int32_t head) {
  if (check_lh(c, layer, head)) return -1;
  return c->keys[size_t(layer) * c->n_heads + head].n;
}

int32_t tqkv_kvcache_attend_keys(tqkv_kvcache* c, int32_t layer, int32_t head,
                                 const float* query, float* scores) {
  if (int32_t rc = check_lh(c, layer, head)) return rc;
  if (!query || !scores) return fail(TQKV_EINVAL_ARG, "null pointer");
  const Stream& s = c->keys[size_t(layer) * c->n_heads + head];
  const int D = c->cfg.head_dim;
  float* buf = nullptr;
  if (int32_t rc = staging(c, size_t(2) * D + size_t(s.n), &buf)) return rc;
  float *q = buf, *rq = buf + D, *out = buf + 2 * D;
  TQKV_HIP(hipMemcpy(q, query, size_t(D) * 4, hipMemcpyHostToDevice));
  if (int32_t rc = tqkv_tq_rotate_query(c->R, q, D, rq, nullptr)) return rc;
  if (int32_t rc = tqkv_tq_scores_packed(rq, s.words, s.sigma, c->cent, c->cfg.bits, D, s.n, out,
                                         nullptr))
    return rc;
  TQKV_HIP(hipMemcpy(scores, out, size_t(s.n) * 4, hipMemcpyDeviceToHost));
  return ok();
}

int32_t tqkv_kvcache_attend_values(tqkv_kvcache* c, int32_t layer, int32_t head,
                                   const float* weights, float* out) {
  if (int32_t rc = check_lh(c, layer, head)) return rc;
  if (!out || (!weights && c->values[size_t(layer) * c->n_heads + head].n > 0))
    return fail(TQKV_EINVAL_ARG, "null pointer");
  const Stream& s = c->values[size_t(layer) * c->n_heads + head];
  const int D = c->cfg.head_dim;
  float* buf = nullptr;
  if (int32_t rc = staging(c, size_t(s.n) + size_t(D), &buf)) return rc;
  float *w = buf, *o = buf + s.n;
  if (s.n > 0) TQKV_HIP(hipMemcpy(w, weights, size_t(s.n) * 4, hipMemcpyHostToDevice));
  if (int32_t rc = tqkv_tq_values_packed(c->R, s.words, s.sigma, c->cent, w, c->cfg.bits, D, s.n,
                                         o, nullptr))
    return rc;
  TQKV_HIP(hipMemcpy(out, o, size_t(D) * 4, hipMemcpyDeviceToHost));
  return ok();
}

int32_t tqkv_kvcache_clear(tqkv_kvcache* c) {
  if (!c) return fail(TQKV_EINVAL_ARG, "null cache");
  for (Stream& s : c->keys) s.n = 0;
  for (Stream& s : c->values) s.n = 0;
  return ok();
}

int32_t tqkv_kvcache_truncate(tqkv_kvcache* c, int32_t layer, int64_t n_keep) {
  if (int32_t rc = check_lh(c, layer, 0)) return rc;
  if (n_keep < 0) return fail(TQKV_EINVAL_TARGET, "n_keep=%lld", (long long)n_keep);
  for (int h = 0; h < c->n_heads; ++h) {
    Stream& k = c->keys[size_t(layer) * c->n_heads + h];
    Stream& v = c->values[size_t(layer) * c->n_heads + h];
    if (k.n > n_keep) k.n = n_keep;
    if (v.n > n_keep) v.n = n_keep;
  }
  return ok();
}

int64_t tqkv_kvcache_memory_bytes(const tqkv_kvcache* c) {
  if (!c) return 0;
  // CompressedVector::size_bytes (config.rs:50-55) per stored vector: packed
  // codes, QJL bits in u64 words, residual norm and scale, dim and bits.
  const int64_t m = c->cfg.qjl_m;
  const int64_t per = int64_t(c->pw) * 8 + ((m + 63) / 64) * 8 + 4 + 4 + 8 + 4;
  int64_t n = 0;
  for (const Stream& s : c->keys) n += s.n;
  for (const Stream& s : c->values) n += s.n;
  return n * per;
}

int32_t tqkv_kvcache_device_bytes(const tqkv_kvcache* c, int64_t* held, int64_t* reserved) {
  if (!c) return fail(TQKV_EINVAL_ARG, "null cache");
  const int64_t D = c->cfg.head_dim, W = c->words, PW = c->pw;
  // Per stored vector: packed codes, scale, and with QJL its sign words and
  // residual norm.
  const int64_t per_held = PW * 8 + 4 + (W ? W * 4 + 4 : 0);
  const int64_t per_slot = PW * 8 + 4 + (W ? W : 1) * 4 + 4;
  int64_t n = 0, slots = 0;
  for (const std::vector<Stream>* v : {&c->keys, &c->values})
    for (const Stream& s : *v) {
      n += s.n;
      slots += s.cap;
    }
  const int64_t n_levels = int64_t(1) << c->cfg.bits;
  const int64_t tables = D * D * 4 + (W ? int64_t(c->cfg.qjl_m) : 1) * D * 4 +
                         (n_levels + 1) * 8 + n_levels * 4;
  if (held) *held = n * per_held;
  if (reserved) *reserved = slots * per_slot + tables + int64_t(c->scratch_floats) * 4;
  return ok();
}

int32_t tqkv_kvcache_read(tqkv_kvcache* c, int32_t layer, int32_t head, int32_t which_values,
                          int64_t first, int64_t n, uint8_t* codes, float* scale,
                          uint32_t* signs, float* residual_norm) {
  if (int32_t rc = check_lh(c, layer, head)) return rc;
  const Stream& s = (which_values ? c->values : c->keys)[size_t(layer) * c->n_heads + head];
  if (first < 0 || n < 0 || first + n > s.n)
    return fail(TQKV_EINVAL_TARGET, "vectors [%lld, %lld) of %lld", (long long)first,
                (long long)(first + n), (long long)s.n);
  if (n == 0) return ok();
  const int D = c->cfg.head_dim, W = c->words;
  if (codes) {
    float* buf = nullptr;
    if (int32_t rc = staging(c, (size_t(n) * D + 3) / 4, &buf)) return rc;
    uint8_t* u8 = reinterpret_cast<uint8_t*>(buf);
    if (int32_t rc = tqkv_unpack_codes(s.words + first * c->pw, n, D, c->cfg.bits, u8, nullptr))
      return rc;
    TQKV_HIP(hipMemcpy(codes, u8, size_t(n) * D, hipMemcpyDeviceToHost));
  }
  if (scale) TQKV_HIP(hipMemcpy(scale, s.sigma + first, size_t(n) * 4, hipMemcpyDeviceToHost));
  if (signs && W)
    TQKV_HIP(hipMemcpy(signs, s.signs + first * W, size_t(n) * W * 4, hipMemcpyDeviceToHost));
  if (residual_norm && W)
    TQKV_HIP(hipMemcpy(residual_norm, s.rnorm + first, size_t(n) * 4, hipMemcpyDeviceToHost));
  return ok();
}

}  // extern "C"
