// Dequantize-then-attend: the oracle for every attention kernel (test
// infrastructure only).
//
// Quantized K/V are dequantized, then scaled-dot-product attention runs over
// them (native_attention.rs:78-110 sdpa, :545-622 mask). Affine caches
// dequantize either exactly in f32 (scale * code + bias, what the reference's
// decode paths compute: native_quant_attention.rs:131-132 and
// quantized_matmul) or to bf16 the way mlx::dequantize does for its prefill
// path (gemma4_moe.rs:2394-2399); codebook caches dequantize to
// bf16(centroid[c] * sigma) (turboquant.rs:428-439). Scores, softmax and the
// weighted sum are computed in f64 here; the result is returned both exactly
// (f32) and rounded to bf16, the dtype the reference returns. GQA maps query
// head h to KV head h / (H / H_kv) (native_attention.rs:124-132).
#include <cmath>
#include <cstring>
#include <vector>

#include "oracle.h"

using namespace oracle;

namespace {

inline double load(uint16_t b) { return double(bf16_to_f32(b)); }
inline double load(float f) { return double(f); }

// One (b, h, query row): softmax(scale * q.K^T masked) . V over n keys.
template <typename T>
void attend_row(const uint16_t* q, const T* K, const T* V, size_t n, int d,
                float scale, bool causal, size_t q_abs, size_t first_held, long window,
                float* out_f32, uint16_t* out_bf16, float* lse) {
  std::vector<double> s(n);
  std::vector<double> qf(d);
  for (int i = 0; i < d; ++i) qf[i] = double(bf16_to_f32(q[i]));
  double mx = -INFINITY;
  for (size_t k = 0; k < n; ++k) {
    if (causal && !mask_allowed(q_abs, first_held + k, window)) {
      s[k] = -INFINITY;
      continue;
    }
    const T* kr = K + k * size_t(d);
    double acc = 0.0;
    for (int i = 0; i < d; ++i) acc += qf[i] * load(kr[i]);
    s[k] = double(scale) * acc;
    if (s[k] > mx) mx = s[k];
  }
  std::vector<double> o(d, 0.0);
  double l = 0.0;
  if (mx != -INFINITY) {
    for (size_t k = 0; k < n; ++k) {
      if (s[k] == -INFINITY) continue;
      double p = std::exp(s[k] - mx);
      l += p;
      const T* vr = V + k * size_t(d);
      for (int i = 0; i < d; ++i) o[i] += p * load(vr[i]);
    }
  }
  for (int i = 0; i < d; ++i) {
    double v = l > 0.0 ? o[i] / l : 0.0;
    out_f32[i] = float(v);
    out_bf16[i] = f32_to_bf16(float(v));
  }
  if (lse) *lse = l > 0.0 ? float(mx + std::log(l)) : -INFINITY;
}

template <typename T>
void attend(const uint16_t* q, const T* K, const T* V, int B, int H, int H_kv, int L, size_t N,
            int D, float scale, int causal, size_t q_start, size_t first_held, long window,
            float* out_f32, uint16_t* out_bf16, float* lse) {
  const int G = H / H_kv;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const int kvh = h / G;
      const T* Kb = K + (size_t(b) * H_kv + kvh) * N * D;
      const T* Vb = V + (size_t(b) * H_kv + kvh) * N * D;
      for (int l = 0; l < L; ++l) {
        const size_t row = (size_t(b) * H + h) * L + l;
        attend_row(q + row * D, Kb, Vb, N, D, scale, causal != 0, q_start + size_t(l),
                   first_held, window, out_f32 + row * D, out_bf16 + row * D,
                   lse ? lse + row : nullptr);
      }
    }
}

// Exact affine dequantization, scale * code + bias from the stored bf16 scale
// and bias, in f32: what the reference's decode paths compute in registers
// (native_quant_attention.rs:131-132, 157-165; quantized_matmul).
void dequantize_f32(const uint32_t* packed, const uint16_t* scales, const uint16_t* biases,
                    size_t rows, int dim, int gs, int bits, float* out) {
  const int groups = dim / gs;
  const size_t words = size_t(dim) * bits / 32;
  for (size_t r = 0; r < rows; ++r)
    for (int i = 0; i < dim; ++i) {
      const float s = bf16_to_f32(scales[r * groups + i / gs]);
      const float b = bf16_to_f32(biases[r * groups + i / gs]);
      out[r * dim + i] = s * float(read_code(packed + r * words, size_t(i), bits)) + b;
    }
}

}  // namespace

extern "C" {

// q [B, H, L, D] bf16; K, V [B, H_kv, N, D] bf16 (already dequantized);
// out_f32 / out_bf16 [B, H, L, D]; lse [B, H, L] (may be null).
// causal: apply the absolute-position mask with query row l at q_start + l and
// key k at first_held + k (window < 0: no window).
void oracle_attend_bf16(const uint16_t* q, const uint16_t* K, const uint16_t* V, int B, int H,
                        int H_kv, int L, size_t N, int D, float scale, int causal,
                        size_t q_start, size_t first_held, long window, float* out_f32,
                        uint16_t* out_bf16, float* lse) {
  attend(q, K, V, B, H, H_kv, L, N, D, scale, causal, q_start, first_held, window, out_f32,
         out_bf16, lse);
}

// Affine-quantized K/V triples [B, H_kv, N, .] dequantized, then attended.
// dequant_f32 = 0: mlx::dequantize to bf16 (the reference's prefill path,
// gemma4_moe.rs:2394-2399), one rounding of the fused f32 multiply-add; 1:
// exact f32 scale * code + bias (its decode paths); 2: mlx::dequantize read
// as two bf16 roundings (the secondary reading). K and V may use different
// bit widths.
void oracle_attend_affine(const uint16_t* q, const uint32_t* kw, const uint16_t* ks,
                          const uint16_t* kb, const uint32_t* vw, const uint16_t* vs,
                          const uint16_t* vb, int B, int H, int H_kv, int L, size_t N, int D,
                          int gs, int bits_k, int bits_v, float scale, int causal,
                          size_t q_start, size_t first_held, long window, float* out_f32,
                          uint16_t* out_bf16, float* lse, int dequant_f32) {
  const size_t rows = size_t(B) * H_kv * N;
  if (dequant_f32) {
    std::vector<float> K(rows * D), V(rows * D);
    dequantize_f32(kw, ks, kb, rows, D, gs, bits_k, K.data());
    dequantize_f32(vw, vs, vb, rows, D, gs, bits_v, V.data());
    attend(q, K.data(), V.data(), B, H, H_kv, L, N, D, scale, causal, q_start, first_held,
           window, out_f32, out_bf16, lse);
    return;
  }
  std::vector<uint16_t> K(rows * D), V(rows * D);
  affine_dequantize_rows(kw, ks, kb, rows, D, gs, bits_k, K.data(), dequant_f32 == 2);
  affine_dequantize_rows(vw, vs, vb, rows, D, gs, bits_v, V.data(), dequant_f32 == 2);
  attend(q, K.data(), V.data(), B, H, H_kv, L, N, D, scale, causal, q_start, first_held, window,
         out_f32, out_bf16, lse);
}

// Codebook (TurboQuant stage-1) K/V: u8 codes [B, H_kv, N, D] and sigma
// [B, H_kv, N] dequantized as bf16(float(centroid[c]) * sigma)
// (turboquant.rs:368-373, 428-439), then oracle_attend_bf16. The keys are in
// the rotated basis, so q must already be rotated by the caller.
void oracle_attend_codebook(const uint16_t* q, const uint8_t* kc, const float* ksig,
                            const uint8_t* vc, const float* vsig, const float* centroids_k,
                            const float* centroids_v, int B, int H, int H_kv, int L, size_t N,
                            int D, float scale, int causal, size_t q_start, size_t first_held,
                            long window, float* out_f32, uint16_t* out_bf16, float* lse) {
  const size_t rows = size_t(B) * H_kv * N;
  std::vector<uint16_t> K(rows * D), V(rows * D);
  for (size_t r = 0; r < rows; ++r)
    for (int i = 0; i < D; ++i) {
      K[r * D + i] = f32_to_bf16(centroids_k[kc[r * D + i]] * ksig[r]);
      V[r * D + i] = f32_to_bf16(centroids_v[vc[r * D + i]] * vsig[r]);
    }
  attend(q, K.data(), V.data(), B, H, H_kv, L, N, D, scale, causal, q_start, first_held, window,
         out_f32, out_bf16, lse);
}

}  // extern "C"

// ---- CPU baseline: the reference's attention semantics in f32 (bench only)
//
// Attention over an affine cache the way a CPU port of the reference would
// compute it, not the f64 oracle above: K/V dequantized exactly in f32
// (scale * code + bias, the decode paths, native_quant_attention.rs:131-166)
// or as mlx::dequantize's bf16 (dequant_bf16 = 1, the prefill path,
// gemma4_moe.rs:2394-2399); f32 scores, softmax (expf) and weighted sum;
// bf16 out. Each key and value row is dequantized once per (batch row, KV
// head) and shared by the group's query heads and rows. OpenMP over (batch
// row, KV head) with `threads` threads. q [B, H, L, D]; triples
// [B, H_kv, cap, .] holding n rows; causal: the absolute-position mask with
// query row l at q_start + l and key t at first_held + t (window < 0: none);
// out bf16 [B, H, L, D].
extern "C" void oracle_attend_affine_f32(const uint16_t* q, const uint32_t* kw,
                                         const uint16_t* ks, const uint16_t* kb,
                                         const uint32_t* vw, const uint16_t* vs,
                                         const uint16_t* vb, int B, int H, int H_kv, int L,
                                         size_t cap, size_t n, int D, int gs, int bits_k,
                                         int bits_v, float scale, int causal, size_t q_start,
                                         size_t first_held, long window, int dequant_bf16,
                                         int threads, uint16_t* out) {
  const int G = H / H_kv;
  const int groups = D / gs;
  const size_t rows_q = size_t(G) * L;
  const size_t kwords = size_t(D) * bits_k / 32, vwords = size_t(D) * bits_v / 32;
  auto deq = [&](const uint32_t* w, const uint16_t* sc, const uint16_t* bi, size_t r,
                 size_t words, int bits, float* row) {
    if (dequant_bf16) {
      uint16_t tmp[1024];
      affine_dequantize_rows(w + r * words, sc + r * groups, bi + r * groups, 1, D, gs, bits,
                             tmp);
      for (int i = 0; i < D; ++i) row[i] = bf16_to_f32(tmp[i]);
      return;
    }
    for (int i = 0; i < D; ++i)
      row[i] = bf16_to_f32(sc[r * groups + i / gs]) * float(read_code(w + r * words, size_t(i), bits)) +
               bf16_to_f32(bi[r * groups + i / gs]);
  };
#pragma omp parallel for collapse(2) schedule(dynamic) num_threads(threads)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H_kv; ++h) {
      const size_t slab = (size_t(b) * H_kv + h) * cap;
      // Query rows j = g * L + l of the group.
      std::vector<float> qf(rows_q * D), row(D), s(rows_q * n), o(rows_q * D, 0.0f);
      for (int g = 0; g < G; ++g)
        for (int l = 0; l < L; ++l)
          for (int i = 0; i < D; ++i)
            qf[(size_t(g) * L + l) * D + i] =
                bf16_to_f32(q[((size_t(b) * H + h * G + g) * L + l) * D + i]);
      std::vector<float> mx(rows_q, -INFINITY), lsum(rows_q, 0.0f);
      for (size_t t = 0; t < n; ++t) {
        deq(kw, ks, kb, slab + t, kwords, bits_k, row.data());
        for (size_t j = 0; j < rows_q; ++j) {
          const int l = int(j % size_t(L));
          if (causal && !mask_allowed(q_start + size_t(l), first_held + t, window)) {
            s[j * n + t] = -INFINITY;
            continue;
          }
          float acc = 0.0f;
          for (int i = 0; i < D; ++i) acc += qf[j * D + i] * row[i];
          const float sc = acc * scale;
          s[j * n + t] = sc;
          if (sc > mx[j]) mx[j] = sc;
        }
      }
      for (size_t j = 0; j < rows_q; ++j)
        for (size_t t = 0; t < n; ++t) {
          const float x = s[j * n + t];
          const float p = x == -INFINITY ? 0.0f : std::exp(x - mx[j]);
          s[j * n + t] = p;
          lsum[j] += p;
        }
      for (size_t t = 0; t < n; ++t) {
        deq(vw, vs, vb, slab + t, vwords, bits_v, row.data());
        for (size_t j = 0; j < rows_q; ++j) {
          const float p = s[j * n + t];
          if (p == 0.0f) continue;
          for (int i = 0; i < D; ++i) o[j * D + i] += p * row[i];
        }
      }
      for (int g = 0; g < G; ++g)
        for (int l = 0; l < L; ++l) {
          const size_t j = size_t(g) * L + l;
          for (int i = 0; i < D; ++i)
            out[((size_t(b) * H + h * G + g) * L + l) * D + i] =
                f32_to_bf16(lsum[j] > 0.0f ? o[j * D + i] / lsum[j] : 0.0f);
        }
    }
}
