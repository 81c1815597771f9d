// Seeded synthetic bf16 inputs generated on the device, for benchmarks that
// need gigabytes of K/V without a host round trip. Counter-based: element i
// of the [rows, dim] array hashes (seed, i) with the SplitMix64 finalizer (the
// generator the reference's golden tests use, golden_tests.rs:26-35), turns
// two 32-bit halves into a N(0,1) value by Box-Muller, and scales a seeded
// subset of channels by `outlier_mult`.
#include <cmath>

#include "common.hpp"

namespace tqkv {
namespace {

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

__global__ void synth_kernel(uint16_t* __restrict__ out, int64_t n, int dim, uint64_t seed,
                             uint32_t outlier_threshold, float outlier_mult) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint64_t h = mix64(seed + 0x9e3779b97f4a7c15ull * uint64_t(i + 1));
    const float u1 = (float(uint32_t(h >> 40)) + 1.0f) * 0x1.0p-24f;  // (0, 1]
    const float u2 = float(uint32_t(h) >> 8) * 0x1.0p-24f;           // [0, 1)
    float x = sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2);
    const int c = int(i % dim);
    const uint32_t pick = uint32_t(mix64(seed ^ (0xc0ffee00ull + uint64_t(c))) >> 32);
    if (pick < outlier_threshold) x *= outlier_mult;
    out[i] = f32_to_bf16(x);
  }
}

}  // namespace
}  // namespace tqkv

extern "C" int32_t tqkv_synth_bf16(uint16_t* out, int64_t rows, int32_t dim, uint64_t seed,
                                   float outlier_frac, float outlier_mult, tqkv_stream stream) {
  using namespace tqkv;
  if (rows < 0 || dim <= 0) return fail(TQKV_EINVAL_SHAPE, "rows=%lld dim=%d", (long long)rows, dim);
  if (rows == 0) return ok();
  if (!out) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (!(outlier_frac >= 0.0f && outlier_frac <= 1.0f))
    return fail(TQKV_EINVAL_ARG, "outlier_frac=%g", double(outlier_frac));
  const double thr = double(outlier_frac) * 4294967296.0;
  const uint32_t threshold = thr >= 4294967295.0 ? 0xffffffffu : uint32_t(thr);
  const int64_t n = rows * dim;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(synth_kernel, dim3(unsigned(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), out, n, dim, seed, threshold,
                     outlier_mult);
  TQKV_LAUNCHED();
  return ok();
}
