// The memory-bandwidth probe of the reference (bandwidth.rs:73-100), for this
// GPU: sum an array of floats, reading every byte exactly once, as a ceiling
// for what a streaming kernel can read from HBM. One pass is two launches: a
// grid-stride partial sum per workgroup (16-byte non-temporal loads, eight in
// flight per lane), then one workgroup adding the partials.
#include "common.hpp"

namespace tqkv {
namespace {

constexpr int kThreads = 256;
typedef float f4_t __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void probe_partial(const f4_t* __restrict__ x,
                                                          int64_t n4, float* __restrict__ part) {
  float acc = 0.0f;
  const int64_t stride = int64_t(gridDim.x) * kThreads;
  int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  for (; i + 7 * stride < n4; i += 8 * stride) {
    f4_t v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = __builtin_nontemporal_load(x + i + k * stride);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc += (v[k].x + v[k].y) + (v[k].z + v[k].w);
  }
  for (; i < n4; i += stride) {
    const f4_t v = x[i];
    acc += (v.x + v.y) + (v.z + v.w);
  }
  __shared__ float s[kThreads];
  s[threadIdx.x] = acc;
  __syncthreads();
  for (int w = kThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) s[threadIdx.x] += s[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) part[blockIdx.x] = s[0];
}

__global__ __launch_bounds__(kThreads) void probe_final(const float* __restrict__ part, int n,
                                                        float* __restrict__ out) {
  __shared__ float s[kThreads];
  float acc = 0.0f;
  for (int i = threadIdx.x; i < n; i += kThreads) acc += part[i];
  s[threadIdx.x] = acc;
  __syncthreads();
  for (int w = kThreads / 2; w > 0; w >>= 1) {
    if (threadIdx.x < w) s[threadIdx.x] += s[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = s[0];
}

}  // namespace
}  // namespace tqkv

extern "C" int32_t tqkv_read_probe(const float* data, size_t bytes, float* scratch,
                                   size_t scratch_bytes, float* out, tqkv_stream stream) {
  using namespace tqkv;
  if (!data || !scratch || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (bytes % 16 != 0 || (reinterpret_cast<uintptr_t>(data) & 15u) != 0)
    return fail(TQKV_EINVAL_ARG, "probe buffer must be 16-byte aligned and sized");
  // One workgroup per compute unit, eight 16-byte loads in flight per lane:
  // the fastest streaming shape a sweep of grid sizes, block sizes and loads
  // in flight found on MI355X (about 7 TB/s; a grid of thousands of
  // workgroups reads about 20% slower).
  int dev = 0, cus = 0;
  TQKV_HIP(hipGetDevice(&dev));
  TQKV_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int blocks = cus > 0 && cus <= 4096 ? cus : 256;
  if (scratch_bytes < size_t(blocks) * sizeof(float))
    return fail(TQKV_EINVAL_ARG, "scratch of %zu bytes, need %zu", scratch_bytes,
                size_t(blocks) * sizeof(float));
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(probe_partial, dim3(blocks), dim3(kThreads), 0, st,
                     reinterpret_cast<const f4_t*>(data), int64_t(bytes / 16), scratch);
  TQKV_LAUNCHED();
  hipLaunchKernelGGL(probe_final, dim3(1), dim3(kThreads), 0, st, scratch, blocks, out);
  TQKV_LAUNCHED();
  return ok();
}

namespace tqkv {
namespace {
// Does nothing: the cost of a launch itself.
__global__ void empty_kernel() {}
}  // namespace
}  // namespace tqkv

extern "C" int32_t tqkv_empty_launch(int32_t workgroups, tqkv_stream stream) {
  using namespace tqkv;
  if (workgroups < 1) return fail(TQKV_EINVAL_ARG, "workgroups=%d", workgroups);
  hipLaunchKernelGGL(empty_kernel, dim3(unsigned(workgroups)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream));
  TQKV_LAUNCHED();
  return ok();
}
