// tqkv_decode_attend_affine_noalloc: the fused affine decode for callers that
// cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).
//
// tqkv_decode_attend_affine writes split partials (f32 [B, H, splits, D] plus
// per-split max and sum) into a caller workspace, or into library scratch it
// allocates on demand. This variant keeps them in a file-scope device array of
// fixed size instead: each device that loads the library holds its own copy
// for the life of the process, and the first call on a device looks up that
// copy's address once (hipGetSymbolAddress) and keeps it. Host code never
// passes the array's own name to a kernel: on the host that name is a
// stand-in, not a device address.
//
// The kernels and the split plan are tqkv_decode_attend_affine's, so the
// results are bit-identical to it. Every call on a device shares that
// device's array: calls that overlap on one device (different streams)
// race. Nothing has to start at zero: every partial slot a call reads, the
// same call's decode kernel writes first.
#include <mutex>

#include "common.hpp"

namespace tqkv {
size_t decode_need_bytes(int B, int H, int H_kv, int D, int group_size, int bits_k, int bits_v,
                         const tqkv_affine_seg* segs, int n_segs, bool app);
}  // namespace tqkv

namespace {

constexpr size_t kScratchBytes = size_t(32) << 20;  // TQKV_NOALLOC_SCRATCH_BYTES
static_assert(kScratchBytes == size_t(TQKV_NOALLOC_SCRATCH_BYTES), "header and library agree");

// The split partials of the no-allocation decode.
static __device__ __attribute__((used)) __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

// The current device's copy of `scratch`, looked up on the first call on
// that device.
int32_t scratch_ptr(void** out) {
  int dev = 0;
  TQKV_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices)
    return tqkv::fail(TQKV_EDEVICE, "device %d beyond the %d this library tracks", dev,
                      kMaxDevices);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return tqkv::fail(TQKV_EDEVICE, "hipGetSymbolAddress(scratch) on device %d: %s", dev,
                        hipGetErrorString(e));
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return TQKV_OK;
}

}  // namespace

extern "C" int32_t tqkv_decode_attend_affine_noalloc(const uint16_t* q, int32_t B, int32_t H,
                                                     int32_t H_kv, int32_t D, int32_t group_size,
                                                     int32_t bits_k, int32_t bits_v, float scale,
                                                     const tqkv_affine_seg* segs, int32_t n_segs,
                                                     uint16_t* out, tqkv_stream stream) {
  using tqkv::fail;
  if (!q || !out || !segs) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv != 0)
    return fail(TQKV_EINVAL_SHAPE, "B=%d H=%d H_kv=%d", B, H, H_kv);
  if (n_segs < 1 || n_segs > 2) return fail(TQKV_EINVAL_ARG, "n_segs=%d", n_segs);
  const size_t need =
      tqkv::decode_need_bytes(B, H, H_kv, D, group_size, bits_k, bits_v, segs, n_segs, false);
  if (need > kScratchBytes)
    return fail(TQKV_EINVAL_SHAPE,
                "this decode needs %zu bytes of split partials; the no-allocation entry's "
                "static scratch holds %zu (use tqkv_decode_attend_affine with a workspace)",
                need, kScratchBytes);
  void* ws = nullptr;
  if (int32_t rc = scratch_ptr(&ws)) return rc;
  return tqkv_decode_attend_affine(q, B, H, H_kv, D, group_size, bits_k, bits_v, scale, segs,
                                   n_segs, out, ws, kScratchBytes, stream);
}
