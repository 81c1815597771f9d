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
// recorded golden digests (golden_tests.rs:425-463), which pin 4-bit gs64
// over bf16 inputs. Real MLX output in the reference's qwen4exp_tiny fixture
// (model.safetensors, f32 scales: 4-bit gs32 and 8-bit gs64, README.md:17-19)
// pins the f32 path at those widths: every full-range group there is a fixed
// point of dequantize-then-requantize (tests/test_oracle_mlx_fixture.py).
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

// One group of `gs` values through the per-group algorithm above. load(i)
// returns value i as f32; the scale and bias are returned unrounded (the
// caller stores them in the input dtype).
template <typename Load>
static void quantize_group(Load load, int gs, int bits, float dtype_max, const AffineOpts& o,
                           uint32_t* pw, size_t first_code, float* scale_out, float* bias_out) {
  const float n_bins = float((1 << bits) - 1);
  const float eps = 1e-7f;
  float w_min = o.wmax_starts_at_zero ? dtype_max : INFINITY;
  float w_max = o.wmax_starts_at_zero ? 0.0f : -INFINITY;
  for (int i = 0; i < gs; ++i) {
    const float v = load(i);
    w_min = std::fmin(w_min, v);
    w_max = std::fmax(w_max, v);
  }
  float scale = std::fmax((w_max - w_min) / n_bins, eps);
  const bool side = std::fabs(w_min) > std::fabs(w_max);
  scale = side ? scale : -scale;
  const float edge = side ? w_min : w_max;
  const float q0 = round_with(edge / scale, o.round);
  const bool at_zero = q0 == 0.0f;
  scale = at_zero ? scale : edge / q0;
  const float bias = at_zero ? 0.0f : edge;
  *scale_out = scale;
  *bias_out = bias;
  for (int i = 0; i < gs; ++i) {
    float q = round_with((load(i) - bias) / scale, o.round);
    q = std::fmin(q, n_bins);
    if (o.clip_low) q = std::fmax(q, 0.0f);
    const uint32_t code = q <= 0.0f ? 0u : uint32_t(q);  // -0.0 and clipped negatives -> 0
    write_code(pw, first_code + size_t(i), bits, code);
  }
}

void affine_quantize_rows(const uint16_t* w, size_t rows, int dim, int gs, int bits,
                          uint32_t* packed, uint16_t* scales, uint16_t* biases,
                          const AffineOpts& o) {
  const int groups = dim / gs;
  const size_t words_per_row = size_t(dim) * bits / 32;
  const float bf16_max = bf16_to_f32(0x7f7f);
  for (size_t r = 0; r < rows; ++r) {
    uint32_t* pw = packed + r * words_per_row;
    for (size_t k = 0; k < words_per_row; ++k) pw[k] = 0;
    for (int g = 0; g < groups; ++g) {
      const uint16_t* x = w + r * dim + size_t(g) * gs;
      float scale, bias;
      quantize_group([x](int i) { return bf16_to_f32(x[i]); }, gs, bits, bf16_max, o, pw,
                     size_t(g) * gs, &scale, &bias);
      scales[r * groups + g] = f32_to_bf16(scale);
      biases[r * groups + g] = f32_to_bf16(bias);
    }
  }
}

void affine_quantize_rows_f32(const float* w, size_t rows, int dim, int gs, int bits,
                              uint32_t* packed, float* scales, float* biases,
                              const AffineOpts& o) {
  const int groups = dim / gs;
  const size_t words_per_row = size_t(dim) * bits / 32;
  for (size_t r = 0; r < rows; ++r) {
    uint32_t* pw = packed + r * words_per_row;
    for (size_t k = 0; k < words_per_row; ++k) pw[k] = 0;
    for (int g = 0; g < groups; ++g) {
      const float* x = w + r * dim + size_t(g) * gs;
      quantize_group([x](int i) { return x[i]; }, gs, bits, FLT_MAX, o, pw, size_t(g) * gs,
                     &scales[r * groups + g], &biases[r * groups + g]);
    }
  }
}

// mlx::dequantize: out = scale * code + bias, computed as one fused
// multiply-add in f32 and rounded once to the output dtype. The reference's
// own record settles the rounding: its qwen4exp_tiny fixture stores MLX's
// dequantize of an f32-scaled 4-bit gs32 table (reference/mtp_outputs.
// safetensors mtp_embedded, produced by qwen4exp_tiny_fixture.py:318 from
// model.safetensors' embed_tokens), and every element equals fmaf(scale,
// code, bias) while the product-then-sum form misses half of them
// (tests/test_oracle_mlx_fixture.py). For bf16 scales the product is exact in
// f32 (at most 8 by 8 significant bits), so this is bf16(f32(s * c + b)).
// two_roundings: the other reading, each operation rounding to bf16
// (bf16(bf16(s * c) + b)), kept as the secondary check.
void affine_dequantize_rows(const uint32_t* packed, const uint16_t* scales,
                            const uint16_t* biases, size_t rows, int dim, int gs, int bits,
                            uint16_t* out, bool two_roundings) {
  const int groups = dim / gs;
  const size_t words_per_row = size_t(dim) * bits / 32;
  for (size_t r = 0; r < rows; ++r) {
    const uint32_t* pw = packed + r * words_per_row;
    for (int i = 0; i < dim; ++i) {
      const float s = bf16_to_f32(scales[r * groups + i / gs]);
      const float b = bf16_to_f32(biases[r * groups + i / gs]);
      const float c = float(read_code(pw, size_t(i), bits));
      if (!two_roundings) {
        out[r * dim + i] = f32_to_bf16(std::fma(s, c, b));
        continue;
      }
      const float sc = bf16_to_f32(f32_to_bf16(s * c));
      out[r * dim + i] = f32_to_bf16(sc + b);
    }
  }
}

void affine_dequantize_rows_f32(const uint32_t* packed, const float* scales, const float* biases,
                                size_t rows, int dim, int gs, int bits, float* out) {
  const int groups = dim / gs;
  const size_t words_per_row = size_t(dim) * bits / 32;
  for (size_t r = 0; r < rows; ++r) {
    const uint32_t* pw = packed + r * words_per_row;
    for (int i = 0; i < dim; ++i)
      out[r * dim + i] = std::fma(scales[r * groups + i / gs],
                                  float(read_code(pw, size_t(i), bits)),
                                  biases[r * groups + i / gs]);
  }
}

}  // namespace oracle
