// Quantize-on-append in MLX's affine format, bit-exact with its Metal kernel,
// and the matching dequantize.
//
// One wavefront per row. Each lane owns EPL = dim / 64 consecutive elements
// (all lanes of a group hold the same group), so a group's min and max are a
// butterfly over gs / EPL lanes. Codes go through LDS as bytes and are packed
// into the LSB-first u32 stream one output word per lane, which handles
// widths whose codes straddle words (3, 5, 6 bits) without special cases.
//
// Arithmetic follows MLX's affine_quantize exactly (see the oracle's
// affine.cpp for the statement): f32 throughout, IEEE division (hipcc's
// default correctly rounded divide), roundf = half away from zero, bf16
// round-to-nearest-even storage of scale and bias, codes from the unrounded
// f32 scale and bias. The reference's recorded digests pin this at 4 bits /
// gs64 (golden_tests.rs:425-463).
#include "common.hpp"

namespace tqkv {
namespace {

constexpr int kWave = 64;

template <int EPL>
__global__ __launch_bounds__(kWave) void affine_quantize_kernel(
    const uint16_t* __restrict__ x, int64_t s, int dim, int gs, int bits,
    uint32_t* __restrict__ packed, uint16_t* __restrict__ scales,
    uint16_t* __restrict__ biases, int64_t dst_cap, int64_t dst_start) {
  __shared__ uint8_t codes[1024];
  const int lane = threadIdx.x;
  const int64_t r = blockIdx.x;
  const int64_t slab = r / s, j = r % s;
  const int64_t dst = slab * dst_cap + dst_start + j;
  const uint16_t* xr = x + r * dim;
  const int base = lane * EPL;
  const bool active = base < dim;  // dim = 32 leaves half the wave idle

  float v[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) v[e] = active ? bf16_to_f32(xr[base + e]) : 0.0f;

  // The Metal kernel starts w_min at the dtype's max and w_max at 0.
  float w_min = __uint_as_float(0x7f7f0000u);
  float w_max = 0.0f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    w_min = fminf(w_min, v[e]);
    w_max = fmaxf(w_max, v[e]);
  }
  const int lanes_per_group = gs / EPL;  // power of two, <= 64
  for (int off = 1; off < lanes_per_group; off <<= 1) {
    w_min = fminf(w_min, __shfl_xor(w_min, off, kWave));
    w_max = fmaxf(w_max, __shfl_xor(w_max, off, kWave));
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

  const int groups = dim / gs;
  if (active && (base % gs) == 0) {
    const int g = base / gs;
    scales[dst * groups + g] = f32_to_bf16(scale);
    biases[dst * groups + g] = f32_to_bf16(bias);
  }
  if (active) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      float q = fminf(roundf((v[e] - bias) / scale), n_bins);
      codes[base + e] = q <= 0.0f ? uint8_t(0) : uint8_t(q);
    }
  }
  __syncthreads();

  const int words = dim * bits / 32;
  uint32_t* out = packed + dst * words;
  for (int w = lane; w < words; w += kWave) {
    const int bit0 = 32 * w;
    const int e0 = bit0 / bits;
    const int e1 = (bit0 + 31) / bits;
    uint32_t word = 0;
    for (int e = e0; e <= e1 && e < dim; ++e) {
      const int sh = e * bits - bit0;
      const uint32_t c = codes[e];
      word |= sh >= 0 ? (c << sh) : (c >> (-sh));
    }
    out[w] = word;
  }
}

__global__ void affine_dequantize_kernel(const uint32_t* __restrict__ packed,
                                         const uint16_t* __restrict__ scales,
                                         const uint16_t* __restrict__ biases, int64_t rows,
                                         int dim, int gs, int bits, uint16_t* __restrict__ out) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * dim) return;
  const int64_t r = i / dim;
  const int e = int(i % dim);
  const uint32_t* pw = packed + r * (dim * bits / 32);
  const int bit = e * bits;
  uint64_t w = pw[bit / 32];
  if ((bit % 32) + bits > 32) w |= uint64_t(pw[bit / 32 + 1]) << 32;
  const uint32_t code = uint32_t(w >> (bit % 32)) & ((1u << bits) - 1);
  const int groups = dim / gs;
  const float sc = bf16_to_f32(scales[r * groups + e / gs]);
  const float bi = bf16_to_f32(biases[r * groups + e / gs]);
  const float prod = bf16_to_f32(f32_to_bf16(sc * float(code)));
  out[i] = f32_to_bf16(prod + bi);
}

bool valid_bits(int bits) {
  return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
}

int32_t check_affine_shape(int32_t dim, int32_t gs, int32_t bits) {
  if (!valid_bits(bits)) return fail(TQKV_EUNSUPPORTED, "affine bits=%d not in {2,3,4,5,6,8}", bits);
  if (!(gs == 32 || gs == 64 || gs == 128))
    return fail(TQKV_EUNSUPPORTED, "group_size=%d not in {32,64,128}", gs);
  if (!(dim == 32 || dim == 64 || dim == 128 || dim == 256 || dim == 512 || dim == 1024))
    return fail(TQKV_EUNSUPPORTED, "dim=%d not in {32,...,1024}", dim);
  if (dim % gs != 0 || (dim * bits) % 32 != 0)
    return fail(TQKV_EINVAL_SHAPE, "dim=%d, group_size=%d, bits=%d do not tile", dim, gs, bits);
  return TQKV_OK;
}

}  // namespace
}  // namespace tqkv

using namespace tqkv;

extern "C" int32_t tqkv_affine_quantize(const uint16_t* x, int64_t n_slabs, int64_t s,
                                        int32_t dim, int32_t group_size, int32_t bits,
                                        uint32_t* packed, uint16_t* scales, uint16_t* biases,
                                        int64_t dst_cap, int64_t dst_start,
                                        tqkv_stream stream) {
  if (int32_t rc = check_affine_shape(dim, group_size, bits)) return rc;
  if (n_slabs < 0 || s < 0 || dst_start < 0 || dst_start + s > dst_cap)
    return fail(TQKV_EINVAL_SHAPE, "rows [%lld, %lld) do not fit a buffer of %lld",
                (long long)dst_start, (long long)(dst_start + s), (long long)dst_cap);
  if (n_slabs == 0 || s == 0) return ok();
  if (!x || !packed || !scales || !biases) return fail(TQKV_EINVAL_ARG, "null pointer");
  const int64_t rows = n_slabs * s;
  if (rows > 0x7fffffffLL) return fail(TQKV_EINVAL_SHAPE, "%lld rows exceed one launch", (long long)rows);
  const int epl = dim < 64 ? 1 : dim / 64;
  const dim3 grid{unsigned(rows)}, block{64u};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
#define TQKV_Q(E)                                                                        \
  case E:                                                                               \
    hipLaunchKernelGGL(affine_quantize_kernel<E>, grid, block, 0, st, x, s, dim,        \
                       group_size, bits, packed, scales, biases, dst_cap, dst_start);   \
    break;
  switch (epl) {
    TQKV_Q(1) TQKV_Q(2) TQKV_Q(4) TQKV_Q(8) TQKV_Q(16)
    default: return fail(TQKV_EUNSUPPORTED, "dim=%d", dim);
  }
#undef TQKV_Q
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_affine_dequantize(const uint32_t* packed, const uint16_t* scales,
                                          const uint16_t* biases, int64_t rows, int32_t dim,
                                          int32_t group_size, int32_t bits, uint16_t* out,
                                          tqkv_stream stream) {
  if (int32_t rc = check_affine_shape(dim, group_size, bits)) return rc;
  if (rows < 0) return fail(TQKV_EINVAL_SHAPE, "rows=%lld", (long long)rows);
  if (rows == 0) return ok();
  if (!packed || !scales || !biases || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  const int64_t n = rows * dim;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffffLL) return fail(TQKV_EINVAL_SHAPE, "too many rows");
  hipLaunchKernelGGL(affine_dequantize_kernel, dim3(unsigned(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), packed, scales, biases, rows, dim,
                     group_size, bits, out);
  TQKV_LAUNCHED();
  return ok();
}
