// MLX affine quantization of one lane's 16 consecutive elements of a row,
// shared by the quantize-on-append kernel and the decode kernel's fused
// append, so both write the same bits.
//
// Arithmetic follows MLX's affine_quantize exactly (the oracle's affine.cpp
// states it): f32 throughout, IEEE division (hipcc's default correctly
// rounded divide), roundf = half away from zero, bf16 round-to-nearest-even
// storage of scale and bias, codes from the unrounded f32 scale and bias.
// The reference's recorded digests pin this at 4 bits / gs64
// (golden_tests.rs:425-463).
#pragma once

#include "common.hpp"

namespace tqkv {
namespace aq {

constexpr int kLaneElems = 16;  // elements a lane

// A lane's share of a quantized row: its group's scale and bias (f32, before
// the bf16 store) and its 16 codes as two 64-bit chunks of 8 codes
// (LSB-first, `bits` bits each).
struct LaneCodes {
  float scale, bias;
  uint64_t chunk[2];
};

// The 16 bf16 elements at p (32-byte aligned) as f32.
__device__ __forceinline__ void load_lane(const uint16_t* p, float (&v)[kLaneElems]) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint4 w = *reinterpret_cast<const uint4*>(p + 8 * h);
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[8 * h + 2 * e] = __uint_as_float(ws[e] << 16);
      v[8 * h + 2 * e + 1] = __uint_as_float(ws[e] & 0xffff0000u);
    }
  }
}

// Quantizes N (a multiple of 8) consecutive elements of a row held by each
// lane; a group is `lpg` adjacent lanes (a power of two), whose min and max
// meet in a butterfly. Writes the group's f32 scale and bias and the lane's
// codes as N / 8 chunks of 8. Every lane of the wavefront must call it (the
// butterfly exchanges across lanes).
//
// kFastQuotient: the code of an element is roundf(RN((v - bias) / scale))
// clamped; instead of the correctly rounded division it multiplies by
// RN(1 / scale), whose product is within 3 ulp of the rounded quotient, and
// takes the exact division only where the product lies within 2^-20 of
// its value from a rounding boundary k + 1/2 (where the two could round to
// different integers). The codes are the same bits either way.
template <int N, bool kFastQuotient = false>
__device__ __forceinline__ void quantize_elems(const float (&v)[N], int lpg, int bits,
                                               float& scale_out, float& bias_out,
                                               uint64_t (&chunk)[N / 8]) {
  // The Metal kernel starts w_min at the dtype's max and w_max at 0.
  float w_min = __uint_as_float(0x7f7f0000u);
  float w_max = 0.0f;
#pragma unroll
  for (int e = 0; e < N; ++e) {
    w_min = fminf(w_min, v[e]);
    w_max = fmaxf(w_max, v[e]);
  }
  for (int off = 1; off < lpg; off <<= 1) {
    w_min = fminf(w_min, __shfl_xor(w_min, off, 64));
    w_max = fmaxf(w_max, __shfl_xor(w_max, off, 64));
  }

  const float n_bins = float((1 << bits) - 1);
  float scale = fmaxf((w_max - w_min) / n_bins, 1e-7f);
  const bool side = fabsf(w_min) > fabsf(w_max);
  scale = side ? scale : -scale;
  const float edge = side ? w_min : w_max;
  const float q0 = roundf(edge / scale);
  const bool at_zero = q0 == 0.0f;
  scale = at_zero ? scale : edge / q0;
  const float bias = at_zero ? 0.0f : edge;

  scale_out = scale;
  bias_out = bias;
  if constexpr (kFastQuotient) {
    const float inv = 1.0f / scale;
#pragma unroll
    for (int h = 0; h < N / 8; ++h) {
      uint64_t c = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float num = v[8 * h + e] - bias;
        const float qa = num * inv;
        const float fl = floorf(qa);
        const float fr = qa - fl;  // exact (Sterbenz, or fl = qa)
        float r = fr >= 0.5f ? fl + 1.0f : fl;
        if (__builtin_expect(fabsf(fr - 0.5f) <= fabsf(qa) * 0x1p-20f, 0))
          r = roundf(num / scale);
        const float q = fminf(r, n_bins);
        const uint32_t code = q <= 0.0f ? 0u : uint32_t(q);
        c |= uint64_t(code) << (bits * e);
      }
      chunk[h] = c;
    }
  } else {
#pragma unroll
    for (int h = 0; h < N / 8; ++h) {
      uint64_t c = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float q = fminf(roundf((v[8 * h + e] - bias) / scale), n_bins);
        const uint32_t code = q <= 0.0f ? 0u : uint32_t(q);
        c |= uint64_t(code) << (bits * e);
      }
      chunk[h] = c;
    }
  }
}

// Quantizes the lane's 16 elements; a group is gs / 16 adjacent lanes.
__device__ __forceinline__ LaneCodes quantize_lane(const float (&v)[kLaneElems], int gs, int bits) {
  LaneCodes r;
  quantize_elems<kLaneElems>(v, gs / kLaneElems, bits, r.scale, r.bias, r.chunk);
  return r;
}

// Output word w of a row (bits [32 w, 32 w + 32) of its LSB-first code
// stream), cut from the row's 64-bit chunks of 8 codes: chunk k = 32 w /
// (8 bits) from bit `off`, and chunk k + 1 when the word runs past it.
__device__ __forceinline__ uint32_t packed_word(const uint64_t* ch, int w, int bits) {
  const int ub = 8 * bits;
  const int bit0 = 32 * w, k = bit0 / ub, off = bit0 - k * ub;
  uint64_t word = ch[k] >> off;
  if (off + 32 > ub) word |= ch[k + 1] << (ub - off);
  return uint32_t(word);
}

}  // namespace aq
}  // namespace tqkv
