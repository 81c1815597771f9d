// QJL stage 2 as the reference's GPU TurboQuant path computes it, and
// attention over a codebook cache with the QJL score correction (test
// infrastructure only; see oracle.h).
//
// qjl_encode_stage2_packed (turboquant.rs:592-622): residual = f32(K_rot) -
// f32(K_dq); r_norm = sqrt(sum r^2); r_proj = residual @ Phi^T; sign bit =
// r_proj >= 0, LSB-first in u32 words.
// qjl_apply_correction_packed / _to_k_dq (turboquant.rs:624-691):
// K_eff = bf16(K_dq + bf16((signs(+-1) @ Phi) * (r_norm * sqrt(pi/2) / sqrt(m)))).
// MLX leaves the summation order of its sums and matmuls open; these run
// sequentially from index 0 (from +0.0), the order the device kernels use.
//
// Codebook attention with the correction: the score of key t is the
// two-stage estimate of compressor.rs:122-159 (rotated-space stage 1 on the
// stored codes, plus ||r|| sqrt(pi/2)/sqrt(m) * sum_i sign_i (Phi q)_i on
// the original-space residual signs of compress_one), times the softmax
// scale; values are bf16(centroid * sigma) in the rotated basis and the
// output returns through R^T (turboquant.rs:763-923 with stage 2).
#include <cmath>
#include <cstdint>
#include <vector>

#include "oracle.h"

using namespace oracle;

namespace {
float qjl_scale(int m) {
  const float frac_pi_2 = 1.57079632679489661923f;
  return std::sqrt(frac_pi_2) / std::sqrt(float(m));
}
}  // namespace

extern "C" {

void oracle_qjl_encode_stage2(const uint16_t* k_rot, const uint16_t* k_dq, const float* phi,
                              size_t rows, int D, int m, uint32_t* signs, float* rnorm) {
  const int words = (m + 31) / 32;
  std::vector<float> r(static_cast<size_t>(D));
  for (size_t t = 0; t < rows; ++t) {
    float ss = 0.0f;
    for (int d = 0; d < D; ++d) {
      r[size_t(d)] = bf16_to_f32(k_rot[t * D + d]) - bf16_to_f32(k_dq[t * D + d]);
      ss += r[size_t(d)] * r[size_t(d)];
    }
    rnorm[t] = std::sqrt(ss);
    for (int w = 0; w < words; ++w) signs[t * words + w] = 0u;
    for (int i = 0; i < m; ++i) {
      float acc = 0.0f;
      for (int d = 0; d < D; ++d) acc += r[size_t(d)] * phi[size_t(i) * D + d];
      if (acc >= 0.0f) signs[t * words + i / 32] |= 1u << (i % 32);
    }
  }
}

void oracle_qjl_apply_correction(const uint16_t* k_dq, const uint32_t* signs, const float* rnorm,
                                 const float* phi, size_t rows, int D, int m, uint16_t* k_eff) {
  const int words = (m + 31) / 32;
  const float sc = qjl_scale(m);
  for (size_t t = 0; t < rows; ++t) {
    const float scaled = rnorm[t] * sc;
    for (int d = 0; d < D; ++d) {
      float acc = 0.0f;
      for (int i = 0; i < m; ++i) {
        const float s = ((signs[t * words + i / 32] >> (i % 32)) & 1u) ? 1.0f : -1.0f;
        acc += s * phi[size_t(i) * D + d];
      }
      const float corr = bf16_to_f32(f32_to_bf16(acc * scaled));
      k_eff[t * D + d] = f32_to_bf16(bf16_to_f32(k_dq[t * D + d]) + corr);
    }
  }
}

// q bf16 [B, H, D] (original basis); caches [B, H_kv, N, .]: codes u8 [D],
// sigma f32, signs u32 [ceil(m/32)], r_norm f32; R f32 [D, D] (y = R x);
// Phi f32 [m, D]. out f32 [B, H, D] (original basis), in f64 internally.
void oracle_attend_codebook_qjl(const uint16_t* q, const uint8_t* kc, const float* ksig,
                                const uint32_t* ksg, const float* krn, const uint8_t* vc,
                                const float* vsig, const float* cent_k, const float* cent_v,
                                const float* R, const float* phi, int B, int H, int H_kv,
                                size_t N, int D, int m, float scale, float* out) {
  const int G = H / H_kv, words = (m + 31) / 32;
  const double qs = std::sqrt(1.57079632679489661923) / std::sqrt(double(m));
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      const size_t slab = size_t(b) * H_kv + size_t(h / G);
      std::vector<double> qf(size_t(D), 0.0), rq(size_t(D), 0.0), pq(size_t(m), 0.0);
      for (int d = 0; d < D; ++d) qf[size_t(d)] = bf16_to_f32(q[(size_t(b) * H + h) * D + d]);
      for (int i = 0; i < D; ++i)
        for (int j = 0; j < D; ++j) rq[size_t(i)] += double(R[size_t(i) * D + j]) * qf[size_t(j)];
      for (int i = 0; i < m; ++i)
        for (int j = 0; j < D; ++j) pq[size_t(i)] += double(phi[size_t(i) * D + j]) * qf[size_t(j)];
      std::vector<double> s(N);
      double mx = -INFINITY;
      for (size_t t = 0; t < N; ++t) {
        const size_t r = slab * N + t;
        double s1 = 0.0;
        for (int d = 0; d < D; ++d)
          s1 += rq[size_t(d)] * double(cent_k[kc[r * D + d]]) * double(ksig[r]);
        double s2 = 0.0;
        if (krn[r] >= 1e-10f) {
          for (int i = 0; i < m; ++i)
            s2 += (((ksg[r * words + i / 32] >> (i % 32)) & 1u) ? 1.0 : -1.0) * pq[size_t(i)];
          s2 *= double(krn[r]) * qs;
        }
        s[t] = (s1 + s2) * double(scale);
        mx = std::max(mx, s[t]);
      }
      double l = 0.0;
      std::vector<double> o(size_t(D), 0.0);
      for (size_t t = 0; t < N; ++t) {
        const size_t r = slab * N + t;
        const double p = std::exp(s[t] - mx);
        l += p;
        for (int d = 0; d < D; ++d)
          o[size_t(d)] += p * double(bf16_to_f32(f32_to_bf16(cent_v[vc[r * D + d]] * vsig[r])));
      }
      for (int i = 0; i < D; ++i) {
        double acc = 0.0;  // o = R^T o_rot
        for (int j = 0; j < D; ++j) acc += double(R[size_t(j) * D + i]) * o[size_t(j)] / l;
        out[(size_t(b) * H + h) * D + i] = float(acc);
      }
    }
}

}  // extern "C"

// The GPU TurboQuant encode (lloyd_max_quantize_stage1, turboquant.rs:
// 398-423, and its rotate variants :720-745; test infrastructure only): y =
// x (mode 0), bf16(x M) (mode 1) or x M in f32 (mode 2), M = R or R^T;
// y_i = fma chain over j from 0.0; sigma = sqrt(sum y^2 / D) with the sum
// over channels l + 64 k first along k (per lane l), then across the 64
// lane partials by an xor butterfly of offsets 32, 16, ..., 1 (the order the
// device kernel fixes; MLX's reduction order is not in the reference);
// code = the number of inner boundaries b with b <= bf16(y / sigma).
extern "C" void oracle_tq_encode_gpu_path(const uint16_t* x, size_t rows, int D, const float* R,
                                          int mode, int transpose, const float* inner,
                                          int n_inner, uint8_t* codes, float* sigma) {
  const int lanes = 64, per = D / lanes;
  std::vector<float> xs(static_cast<size_t>(D)), y(static_cast<size_t>(D));
  for (size_t r = 0; r < rows; ++r) {
    for (int i = 0; i < D; ++i) xs[i] = bf16_to_f32(x[r * D + i]);
    for (int i = 0; i < D; ++i) {
      if (mode == 0) {
        y[i] = xs[i];
        continue;
      }
      float acc = 0.0f;
      for (int j = 0; j < D; ++j)
        acc = std::fma(xs[j], transpose ? R[size_t(i) * D + j] : R[size_t(j) * D + i], acc);
      y[i] = mode == 1 ? bf16_to_f32(f32_to_bf16(acc)) : acc;
    }
    float p[64];
    for (int l = 0; l < lanes; ++l) {
      float a = 0.0f;
      for (int k = 0; k < per; ++k) {
        const float v = y[l + k * lanes];
        const float sq = v * v;
        a = a + sq;
      }
      p[l] = a;
    }
    for (int off = lanes / 2; off >= 1; off >>= 1) {
      float q[64];
      for (int l = 0; l < lanes; ++l) q[l] = p[l] + p[l ^ off];
      for (int l = 0; l < lanes; ++l) p[l] = q[l];
    }
    const float sg = std::sqrt(p[0] / float(D));
    sigma[r] = sg;
    for (int i = 0; i < D; ++i) {
      const float xn = bf16_to_f32(f32_to_bf16(y[i] / sg));
      int c = 0;
      while (c < n_inner && inner[c] <= xn) ++c;
      codes[r * D + i] = uint8_t(c);
    }
  }
}
