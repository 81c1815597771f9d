// Status codes, the per-thread last error, the per-device scratch buffer.
#include <cstdarg>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.hpp"

namespace tqkv {

static thread_local char g_last_error[512] = "";

int32_t fail(int32_t status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int32_t ok() {
  g_last_error[0] = '\0';
  return TQKV_OK;
}

namespace {
struct Scratch {
  void* ptr = nullptr;
  size_t bytes = 0;
  std::vector<void*> retired;  // outgrown buffers, freed by tqkv_scratch_release
  size_t retired_bytes = 0;
};
std::mutex g_scratch_mu;
std::vector<Scratch> g_scratch;
}  // namespace

int32_t scratch_for_current_device(size_t bytes, void** out) {
  int dev = 0;
  TQKV_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch.size() <= size_t(dev)) g_scratch.resize(size_t(dev) + 1);
  Scratch& s = g_scratch[size_t(dev)];
  if (s.bytes < bytes) {
    // Work already queued may still use the outgrown buffer, and nothing
    // here waits for it (the calls are asynchronous): it is kept until
    // tqkv_scratch_release. Growth at least doubles, so what is kept stays
    // below the current size.
    size_t want = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
    if (want < 2 * s.bytes) want = 2 * s.bytes;
    void* p = nullptr;
    if (hipMalloc(&p, want) != hipSuccess) {
      // Doubling may ask for too much: the exact size, before giving up.
      if (want > bytes && hipMalloc(&p, bytes) == hipSuccess) {
        want = bytes;
      } else {
        return fail(TQKV_ENOMEM, "scratch hipMalloc of %zu bytes failed", bytes);
      }
    }
    if (s.ptr) {
      s.retired.push_back(s.ptr);
      s.retired_bytes += s.bytes;
    }
    s.ptr = p;
    s.bytes = want;
  }
  *out = s.ptr;
  return TQKV_OK;
}

int32_t scratch_release_all() {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  int dev = 0;
  TQKV_HIP(hipGetDevice(&dev));
  for (size_t d = 0; d < g_scratch.size(); ++d) {
    Scratch& s = g_scratch[d];
    if (!s.ptr && s.retired.empty()) continue;
    TQKV_HIP(hipSetDevice(int(d)));
    TQKV_HIP(hipDeviceSynchronize());
    for (void* p : s.retired) (void)hipFree(p);
    s.retired.clear();
    s.retired_bytes = 0;
    (void)hipFree(s.ptr);
    s.ptr = nullptr;
    s.bytes = 0;
  }
  TQKV_HIP(hipSetDevice(dev));
  return TQKV_OK;
}

size_t scratch_held_bytes() {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  size_t n = 0;
  for (const Scratch& s : g_scratch) n += s.bytes + s.retired_bytes;
  return n;
}

}  // namespace tqkv

extern "C" {

const char* tqkv_status_string(int32_t status) {
  switch (status) {
    case TQKV_OK: return "TQKV_OK";
    case TQKV_EINVAL_SHAPE: return "TQKV_EINVAL_SHAPE";
    case TQKV_EINVAL_TARGET: return "TQKV_EINVAL_TARGET";
    case TQKV_EUNSUPPORTED: return "TQKV_EUNSUPPORTED";
    case TQKV_EDEVICE: return "TQKV_EDEVICE";
    case TQKV_ENOMEM: return "TQKV_ENOMEM";
    case TQKV_EINVAL_ARG: return "TQKV_EINVAL_ARG";
    case TQKV_ECORRUPT: return "TQKV_ECORRUPT";
  }
  return "TQKV_UNKNOWN";
}

const char* tqkv_last_error(void) { return tqkv::g_last_error; }

int32_t tqkv_scratch_release(void) {
  if (int32_t rc = tqkv::scratch_release_all()) return rc;
  return tqkv::ok();
}

size_t tqkv_scratch_bytes(void) { return tqkv::scratch_held_bytes(); }

int32_t tqkv_version(void) { return TQKV_ABI_VERSION; }

}  // extern "C"
