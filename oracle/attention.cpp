// Dequantize-then-attend: the oracle for every attention kernel (test
// infrastructure only).
//
// Restates the reference's fallback chain: quantized K/V are dequantized to
// bf16 (mlx::dequantize for the affine format, gemma4_moe.rs:2394-2399;
// centroid[c] * sigma -> bf16 for the codebook format, turboquant.rs:428-439),
// then scaled-dot-product attention runs over them
// (native_attention.rs:78-110 sdpa, :545-622 mask). Scores, softmax and the
// weighted sum are computed in f64 here; the result is returned both exactly
// (f32) and rounded to bf16, the dtype the reference returns. GQA maps query
// head h to KV head h / (H / H_kv) (native_attention.rs:124-132).
#include <cmath>
#include <cstring>
#include <vector>

#include "oracle.h"

using namespace oracle;

namespace {

// One (b, h, query row): softmax(scale * q.K^T masked) . V over n keys.
void attend_row(const uint16_t* q, const uint16_t* K, const uint16_t* V, size_t n, int d,
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
    const uint16_t* kr = K + k * size_t(d);
    double acc = 0.0;
    for (int i = 0; i < d; ++i) acc += qf[i] * double(bf16_to_f32(kr[i]));
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
      const uint16_t* vr = V + k * size_t(d);
      for (int i = 0; i < d; ++i) o[i] += p * double(bf16_to_f32(vr[i]));
    }
  }
  for (int i = 0; i < d; ++i) {
    double v = l > 0.0 ? o[i] / l : 0.0;
    out_f32[i] = float(v);
    out_bf16[i] = f32_to_bf16(float(v));
  }
  if (lse) *lse = l > 0.0 ? float(mx + std::log(l)) : -INFINITY;
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
  const int G = H / H_kv;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const int kvh = h / G;
      const uint16_t* Kb = K + (size_t(b) * H_kv + kvh) * N * D;
      const uint16_t* Vb = V + (size_t(b) * H_kv + kvh) * N * D;
      for (int l = 0; l < L; ++l) {
        const size_t row = (size_t(b) * H + h) * L + l;
        attend_row(q + row * D, Kb, Vb, N, D, scale, causal != 0, q_start + size_t(l),
                   first_held, window, out_f32 + row * D, out_bf16 + row * D,
                   lse ? lse + row : nullptr);
      }
    }
}

// Affine-quantized K/V triples [B, H_kv, N, .] dequantized to bf16 (MLX
// dequantize), then oracle_attend_bf16. K and V may use different bit widths.
void oracle_attend_affine(const uint16_t* q, const uint32_t* kw, const uint16_t* ks,
                          const uint16_t* kb, const uint32_t* vw, const uint16_t* vs,
                          const uint16_t* vb, int B, int H, int H_kv, int L, size_t N, int D,
                          int gs, int bits_k, int bits_v, float scale, int causal,
                          size_t q_start, size_t first_held, long window, float* out_f32,
                          uint16_t* out_bf16, float* lse) {
  const size_t rows = size_t(B) * H_kv * N;
  std::vector<uint16_t> K(rows * D), V(rows * D);
  affine_dequantize_rows(kw, ks, kb, rows, D, gs, bits_k, K.data());
  affine_dequantize_rows(vw, vs, vb, rows, D, gs, bits_v, V.data());
  oracle_attend_bf16(q, K.data(), V.data(), B, H, H_kv, L, N, D, scale, causal, q_start,
                     first_held, window, out_f32, out_bf16, lse);
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
  oracle_attend_bf16(q, K.data(), V.data(), B, H, H_kv, L, N, D, scale, causal, q_start,
                     first_held, window, out_f32, out_bf16, lse);
}

}  // extern "C"
