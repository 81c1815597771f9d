// MLX affine (scale + zero-point) quantization restated (test infrastructure).
//
// The reference quantizes its KV cache with mlx::quantize (native_cache.rs:
// 968-971, 1445-1448), whose arithmetic lives in third-party MLX (v0.32.3 via
// the rabbitson87/mlx fork, Cargo.lock:3031-3060), not in the reference tree.
// This is MLX's published per-group algorithm as its Metal kernel
// (quantized.h, affine_quantize) computes it:
//
//   w_min = min(group) (starting from the dtype's max), w_max = max(group)
//   (starting from 0 in the Metal kernel; the CPU fallback starts from -inf)
//   scale = max((w_max - w_min) / n_bins, 1e-7), negated unless |w_min| > |w_max|
//   edge  = the larger-magnitude extreme; q0 = round(edge / scale)
//   q0 != 0: scale = edge / q0, bias = edge;  q0 == 0: bias = 0
//   code  = min(round((w - bias) / scale), n_bins)    (CPU fallback also clips at 0)
//   scale and bias are stored in the input dtype (bf16, round to nearest even),
//   codes are computed from the unrounded f32 scale and bias.
//
// `round` is the Metal kernel's round-half-away-from-zero; the CPU fallback
// uses rint (half to even). Which one the reference ran is decided by its
// recorded golden digests (golden_tests.rs:425-463), which pin 4-bit gs64.
#include <cfloat>
#include <cmath>

#include "oracle.h"

namespace oracle {

uint32_t read_code(const uint32_t* words, size_t i, int bits) {
  size_t bit = i * size_t(bits);
  size_t w = bit / 32, off = bit % 32;
  uint64_t v = words[w] >> off;
  if (off + size_t(bits) > 32) v |= uint64_t(words[w + 1]) << (32 - off);
  return uint32_t(v & ((1u << bits) - 1));
}

void write_code(uint32_t* words, size_t i, int bits, uint32_t code) {
  size_t bit = i * size_t(bits);
  size_t w = bit / 32, off = bit % 32;
  words[w] |= code << off;
  if (off + size_t(bits) > 32) words[w + 1] |= code >> (32 - off);
}

static float round_with(float x, RoundMode m) {
  return m == RoundMode::HalfAway ? std::round(x) : std::rint(x);
}

void affine_quantize_rows(const uint16_t* w, size_t rows, int dim, int gs, int bits,
                          uint32_t* packed, uint16_t* scales, uint16_t* biases,
                          const AffineOpts& o) {
  const float n_bins = float((1 << bits) - 1);
  const float eps = 1e-7f;
  const int groups = dim / gs;
  const size_t words_per_row = size_t(dim) * bits / 32;
  const float bf16_max = bf16_to_f32(0x7f7f);
  for (size_t r = 0; r < rows; ++r) {
    uint32_t* pw = packed + r * words_per_row;
    for (size_t k = 0; k < words_per_row; ++k) pw[k] = 0;
    for (int g = 0; g < groups; ++g) {
      const uint16_t* x = w + r * dim + size_t(g) * gs;
      float w_min = o.wmax_starts_at_zero ? bf16_max : INFINITY;
      float w_max = o.wmax_starts_at_zero ? 0.0f : -INFINITY;
      for (int i = 0; i < gs; ++i) {
        float v = bf16_to_f32(x[i]);
        w_min = std::fmin(w_min, v);
        w_max = std::fmax(w_max, v);
      }
      float scale = std::fmax((w_max - w_min) / n_bins, eps);
      bool side = std::fabs(w_min) > std::fabs(w_max);
      scale = side ? scale : -scale;
      float edge = side ? w_min : w_max;
      float q0 = round_with(edge / scale, o.round);
      bool at_zero = q0 == 0.0f;
      scale = at_zero ? scale : edge / q0;
      float bias = at_zero ? 0.0f : edge;
      scales[r * groups + g] = f32_to_bf16(scale);
      biases[r * groups + g] = f32_to_bf16(bias);
      for (int i = 0; i < gs; ++i) {
        float q = round_with((bf16_to_f32(x[i]) - bias) / scale, o.round);
        q = std::fmin(q, n_bins);
        if (o.clip_low) q = std::fmax(q, 0.0f);
        uint32_t code = q <= 0.0f ? 0u : uint32_t(q);  // -0.0 and clipped negatives -> 0
        write_code(pw, size_t(g) * gs + i, bits, code);
      }
    }
  }
}

// mlx dequantize for bf16 scales: out = scale * code + bias in bf16
// arithmetic (each operation rounds to bf16); one_rounding: the product and
// sum in f32 (the product is exact: 8 by at most 8 significant bits), then
// one rounding to bf16.
void affine_dequantize_rows(const uint32_t* packed, const uint16_t* scales,
                            const uint16_t* biases, size_t rows, int dim, int gs,
                            int bits, uint16_t* out, bool one_rounding) {
  const int groups = dim / gs;
  const size_t words_per_row = size_t(dim) * bits / 32;
  for (size_t r = 0; r < rows; ++r) {
    const uint32_t* pw = packed + r * words_per_row;
    for (int i = 0; i < dim; ++i) {
      float s = bf16_to_f32(scales[r * groups + i / gs]);
      float b = bf16_to_f32(biases[r * groups + i / gs]);
      float c = float(read_code(pw, size_t(i), bits));
      if (one_rounding) {
        out[r * dim + i] = f32_to_bf16(s * c + b);
        continue;
      }
      float sc = bf16_to_f32(f32_to_bf16(s * c));
      out[r * dim + i] = f32_to_bf16(sc + b);
    }
  }
}

}  // namespace oracle
