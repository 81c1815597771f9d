// Shared internals of libtqkv: status plumbing, HIP checks, bf16 helpers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "tqkv.h"

namespace tqkv {

// Records a failure for tqkv_last_error() and returns `status`.
int32_t fail(int32_t status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Clears the thread's last error and returns TQKV_OK.
int32_t ok();

#define TQKV_HIP(expr)                                                                  \
  do {                                                                                  \
    hipError_t e_ = (expr);                                                             \
    if (e_ != hipSuccess)                                                               \
      return ::tqkv::fail(TQKV_EDEVICE, "%s failed: %s (%s:%d)", #expr,                 \
                          hipGetErrorString(e_), __FILE__, __LINE__);                   \
  } while (0)

#define TQKV_LAUNCHED()                                                                 \
  do {                                                                                  \
    hipError_t e_ = hipGetLastError();                                                  \
    if (e_ != hipSuccess)                                                               \
      return ::tqkv::fail(TQKV_EDEVICE, "kernel launch failed: %s (%s:%d)",             \
                          hipGetErrorString(e_), __FILE__, __LINE__);                   \
  } while (0)

// A device scratch buffer the library keeps per device for callers that pass
// no workspace. Grown on demand (at least doubling, without waiting for
// queued work: outgrown buffers are kept); freed by tqkv_scratch_release.
int32_t scratch_for_current_device(size_t bytes, void** out);
int32_t scratch_release_all();

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(uint32_t(b) << 16);
}

// Round to nearest even; NaN to the canonical quiet NaN (MLX's
// float_to_bfloat_bits).
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  uint32_t b = __float_as_uint(x);
  if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  b += 0x7fffu + ((b >> 16) & 1u);
  return uint16_t(b >> 16);
}

}  // namespace tqkv
