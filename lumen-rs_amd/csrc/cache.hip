// The KV cache object: device buffers in the reference's [B, H_kv, len, row]
// layout, updated by the index math of cache_plan.hpp, with quantize-on-
// append and decode attention over its fetched view.
//
// Replaces the GPU caches of crates/lumen-mlx/src/native_cache.rs:
// NativeKvCache / NativeKvCacheQuantized (growing, :369-1126),
// NativeRotatingKvCache{,Quantized,TurboQuant} (rotating, :1145-1862) and the
// shared-prefix split (SharedPrefixKv / keep_suffix_from, :464-494,
// :2044-2210). Each slot (keys, values, and for the affine format their
// scales and biases) is one allocation with a row capacity; an update grows
// it in place where the plan keeps the old rows as a prefix, and otherwise
// gathers the planned pieces into a second allocation and swaps. Fills and
// copies are small kernels (no hipMemsetAsync, so a caller may capture the
// update-free calls in a graph).
#include <cstring>
#include <new>
#include <vector>

#include "cache_plan.hpp"
#include "common.hpp"

namespace tqkv {
namespace {

constexpr int kMaxSlots = 6;

// Copies rows [src_row, src_row + n) of every slab of src into rows
// [dst_row, ...) of dst (slab strides src_cap / dst_cap rows of `rb` bytes);
// src == nullptr writes zeros. Word copies when everything is 4-aligned.
__global__ void rows_copy_kernel(uint8_t* __restrict__ dst, int64_t dst_cap, int64_t dst_row,
                                 const uint8_t* __restrict__ src, int64_t src_cap,
                                 int64_t src_row, int64_t n, int64_t rb, int words) {
  const int64_t slab = blockIdx.y;
  const int64_t bytes = n * rb;
  uint8_t* d = dst + (slab * dst_cap + dst_row) * rb;
  const uint8_t* s = src ? src + (slab * src_cap + src_row) * rb : nullptr;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  if (words) {
    uint32_t* dw = reinterpret_cast<uint32_t*>(d);
    const uint32_t* sw = reinterpret_cast<const uint32_t*>(s);
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes / 4; i += stride)
      dw[i] = sw ? sw[i] : 0u;
  } else {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes; i += stride)
      d[i] = s ? s[i] : uint8_t(0);
  }
}

struct Buf {
  uint8_t* ptr = nullptr;
  int64_t cap = 0;  // rows per slab
};

int32_t rows_copy(hipStream_t st, int64_t n_slabs, int64_t rb, uint8_t* dst, int64_t dst_cap,
                  int64_t dst_row, const uint8_t* src, int64_t src_cap, int64_t src_row,
                  int64_t n) {
  if (n <= 0 || n_slabs <= 0) return TQKV_OK;
  const int64_t bytes = n * rb;
  const bool words = (rb % 4 == 0) && (reinterpret_cast<uintptr_t>(dst) % 4 == 0) &&
                     (!src || reinterpret_cast<uintptr_t>(src) % 4 == 0);
  const int64_t units = words ? bytes / 4 : bytes;
  int64_t blocks = (units + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  if (n_slabs > 65535) return fail(TQKV_EINVAL_SHAPE, "%lld slabs exceed one launch", (long long)n_slabs);
  hipLaunchKernelGGL(rows_copy_kernel, dim3(unsigned(blocks), unsigned(n_slabs)), dim3(256), 0,
                     st, dst, dst_cap, dst_row, src, src_cap, src_row, n, rb, words ? 1 : 0);
  TQKV_LAUNCHED();
  return TQKV_OK;
}

}  // namespace
}  // namespace tqkv

using namespace tqkv;

struct tqkv_cache {
  tqkv_cache_config cfg{};
  cacheplan::Config pc;
  cacheplan::State st;
  int n_slots = 0;
  int64_t rb[kMaxSlots] = {};  // row bytes per slot
  Buf cur[kMaxSlots], alt[kMaxSlots];
  int64_t n_slabs = 0;
  int64_t view_n = 0;          // rows of the last fetched view
  int64_t base_offset = 0;     // absolute position of row 0 (shared-prefix suffix)
  const tqkv_cache* prefix = nullptr;
  // codebook kind: device tables, built on first use (or given)
  float* R = nullptr;          // [D, D] row-major
  float* phi = nullptr;        // [m, D]
  double* bnd_k = nullptr;     // [2^bits_k + 1]
  double* bnd_v = nullptr;
  float* cent_k = nullptr;     // [2^bits_k], the f64 centroids rounded
  float* cent_v = nullptr;
};

namespace {

void release(Buf& b) {
  if (b.ptr) (void)hipFree(b.ptr);
  b = Buf{};
}

int32_t alloc(tqkv_cache* c, Buf& b, int64_t rows, int slot) {
  void* p = nullptr;
  const size_t bytes = size_t(c->n_slabs) * size_t(rows) * size_t(c->rb[slot]);
  if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess)
    return fail(TQKV_ENOMEM, "cache hipMalloc of %zu bytes failed", bytes);
  b.ptr = static_cast<uint8_t*>(p);
  b.cap = rows;
  return TQKV_OK;
}

// Row capacity to allocate for a buffer of `need` rows: rotating caches are
// bounded by their window plus one chunk; growing caches round up to the
// 256-token step and grow by at least half again, so appends amortize.
int64_t capacity_for(const tqkv_cache* c, int64_t need, int64_t old_cap) {
  int64_t cap = (need + cacheplan::kStep - 1) / cacheplan::kStep * cacheplan::kStep;
  if (c->pc.max_size == 0 && old_cap > 0 && cap < old_cap + old_cap / 2)
    cap = (old_cap + old_cap / 2 + cacheplan::kStep - 1) / cacheplan::kStep * cacheplan::kStep;
  return cap < need ? need : cap;
}

// Carries out a plan's first half (the new buffer from pieces) on every slot.
int32_t execute(tqkv_cache* c, const cacheplan::Plan& p, int64_t old_len, hipStream_t st) {
  // In place when the plan is "rows [0, a) of the old buffer, then zeros".
  int64_t a = 0;
  bool in_place = true;
  for (size_t i = 0; i < p.pieces.size(); ++i) {
    const cacheplan::Piece& q = p.pieces[i];
    if (q.src >= 0) {
      if (i != 0 || q.src != 0) in_place = false;
      else a = q.n;
    }
  }
  (void)old_len;
  for (int s = 0; s < c->n_slots; ++s) {
    Buf& cur = c->cur[s];
    const int64_t rb = c->rb[s];
    if (in_place) {
      if (cur.cap < p.len) {
        Buf nb;
        if (int32_t rc = alloc(c, nb, capacity_for(c, p.len, cur.cap), s)) return rc;
        if (int32_t rc = rows_copy(st, c->n_slabs, rb, nb.ptr, nb.cap, 0, cur.ptr, cur.cap, 0, a))
          return rc;
        if (cur.ptr) TQKV_HIP(hipStreamSynchronize(st));
        release(cur);
        cur = nb;
      }
      if (int32_t rc = rows_copy(st, c->n_slabs, rb, cur.ptr, cur.cap, a, nullptr, 0, 0, p.len - a))
        return rc;
    } else {
      Buf& alt = c->alt[s];
      if (alt.cap < p.len) {
        if (alt.ptr) TQKV_HIP(hipStreamSynchronize(st));
        release(alt);
        if (int32_t rc = alloc(c, alt, capacity_for(c, p.len, cur.cap), s)) return rc;
      }
      int64_t at = 0;
      for (const cacheplan::Piece& q : p.pieces) {
        if (int32_t rc = rows_copy(st, c->n_slabs, rb, alt.ptr, alt.cap, at,
                                   q.src >= 0 ? cur.ptr : nullptr, cur.cap, q.src >= 0 ? q.src : 0,
                                   q.n))
          return rc;
        at += q.n;
      }
      std::swap(cur, alt);
    }
  }
  return TQKV_OK;
}

int32_t upload(void** dst, const void* src, size_t bytes) {
  if (*dst == nullptr && hipMalloc(dst, bytes ? bytes : 1) != hipSuccess)
    return fail(TQKV_ENOMEM, "table hipMalloc of %zu bytes failed", bytes);
  TQKV_HIP(hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice));
  return TQKV_OK;
}

// The codebook kind's tables: Lloyd-Max levels for the key and value widths,
// the rotation (seed) and the QJL matrix (seed + 1), unless given.
int32_t codebook_tables(tqkv_cache* c, const float* R_host, const float* phi_host) {
  const tqkv_cache_config& g = c->cfg;
  const int D = g.k_dim, m = 32 * g.qjl_words;
  if (g.k_dim != g.v_dim) return fail(TQKV_EUNSUPPORTED, "codebook caches need k_dim == v_dim");
  if (!(D == 64 || D == 128 || D == 256 || D == 512))
    return fail(TQKV_EUNSUPPORTED, "codebook dim=%d not in {64,128,256,512}", D);
  for (int kv = 0; kv < 2; ++kv) {
    const int bits = kv ? g.bits_v : g.bits_k;
    const int n = 1 << bits;
    std::vector<double> b(size_t(n) + 1), ce(static_cast<size_t>(n));
    if (int32_t rc = tqkv_lloyd_max(uint32_t(bits), 1000, b.data(), ce.data())) return rc;
    std::vector<float> cf(ce.begin(), ce.end());
    if (int32_t rc = upload(reinterpret_cast<void**>(kv ? &c->bnd_v : &c->bnd_k), b.data(), b.size() * 8)) return rc;
    if (int32_t rc = upload(reinterpret_cast<void**>(kv ? &c->cent_v : &c->cent_k), cf.data(), cf.size() * 4)) return rc;
  }
  std::vector<float> R(size_t(D) * D);
  if (R_host) std::memcpy(R.data(), R_host, R.size() * 4);
  else if (int32_t rc = tqkv_rotation_matrix(D, g.seed, R.data())) return rc;
  if (int32_t rc = upload(reinterpret_cast<void**>(&c->R), R.data(), R.size() * 4)) return rc;
  if (m > 0) {
    std::vector<float> P(size_t(m) * D);
    if (phi_host) std::memcpy(P.data(), phi_host, P.size() * 4);
    else if (int32_t rc = tqkv_qjl_matrix(D, m, g.seed + 1, P.data())) return rc;
    if (int32_t rc = upload(reinterpret_cast<void**>(&c->phi), P.data(), P.size() * 4)) return rc;
  }
  return TQKV_OK;
}

void fill_view(const tqkv_cache* c, int64_t n, tqkv_cache_view* v) {
  std::memset(v, 0, sizeof(*v));
  v->n = n;
  v->cap = c->cur[0].cap;
  v->n_slots = c->n_slots;
  for (int s = 0; s < c->n_slots; ++s) {
    v->slot[s] = c->cur[s].ptr;
    v->row_bytes[s] = c->rb[s];
  }
}

// The affine key segments of a cache: the attached prefix's first
// base_offset rows (shared by every batch row), then the last fetched view.
int affine_segments(const tqkv_cache* c, tqkv_affine_seg* segs) {
  auto seg_of = [](const tqkv_cache* x, int64_t n, int shared) {
    tqkv_affine_seg s{};
    s.k_packed = reinterpret_cast<const uint32_t*>(x->cur[0].ptr);
    s.k_scales = reinterpret_cast<const uint16_t*>(x->cur[1].ptr);
    s.k_biases = reinterpret_cast<const uint16_t*>(x->cur[2].ptr);
    s.v_packed = reinterpret_cast<const uint32_t*>(x->cur[3].ptr);
    s.v_scales = reinterpret_cast<const uint16_t*>(x->cur[4].ptr);
    s.v_biases = reinterpret_cast<const uint16_t*>(x->cur[5].ptr);
    s.cap = x->cur[0].cap;
    s.n = n;
    s.shared = shared;
    return s;
  };
  int n = 0;
  if (c->prefix && c->base_offset > 0) segs[n++] = seg_of(c->prefix, c->base_offset, 1);
  if (c->view_n > 0) segs[n++] = seg_of(c, c->view_n, 0);
  return n;
}

}  // namespace

extern "C" {

int32_t tqkv_cache_create(const tqkv_cache_config* cfg, tqkv_cache** out) {
  if (!cfg || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  *out = nullptr;
  const tqkv_cache_config& k = *cfg;
  if (k.batch <= 0 || k.kv_heads <= 0 || k.k_dim <= 0 || k.v_dim <= 0)
    return fail(TQKV_EINVAL_SHAPE, "batch=%d kv_heads=%d k_dim=%d v_dim=%d", k.batch, k.kv_heads,
                k.k_dim, k.v_dim);
  if (k.max_size < 0 || k.keep < 0 || (k.max_size > 0 && k.keep >= k.max_size))
    return fail(TQKV_EINVAL_ARG, "max_size=%lld keep=%lld", (long long)k.max_size,
                (long long)k.keep);
  tqkv_cache* c = new (std::nothrow) tqkv_cache();
  if (!c) return fail(TQKV_ENOMEM, "cache object");
  c->cfg = k;
  c->pc.max_size = k.max_size;
  c->pc.keep = k.keep;
  c->pc.prealloc = k.prealloc != 0;
  c->n_slabs = int64_t(k.batch) * k.kv_heads;
  switch (k.kind) {
    case TQKV_CACHE_BF16:
      c->n_slots = 2;
      c->rb[0] = int64_t(k.k_dim) * 2;
      c->rb[1] = int64_t(k.v_dim) * 2;
      break;
    case TQKV_CACHE_AFFINE: {
      const int gs = k.group_size;
      auto ok = [&](int dim, int bits) {
        return (bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8) &&
               gs > 0 && dim % gs == 0 && (dim * bits) % 32 == 0;
      };
      if (!ok(k.k_dim, k.bits_k) || !ok(k.v_dim, k.bits_v)) {
        delete c;
        return fail(TQKV_EUNSUPPORTED, "affine layout k_dim=%d v_dim=%d group=%d bits=%d/%d",
                    k.k_dim, k.v_dim, gs, k.bits_k, k.bits_v);
      }
      c->n_slots = 6;
      c->pc.quantized = true;
      c->rb[0] = int64_t(k.k_dim) * k.bits_k / 8;
      c->rb[1] = c->rb[2] = int64_t(k.k_dim / gs) * 2;
      c->rb[3] = int64_t(k.v_dim) * k.bits_v / 8;
      c->rb[4] = c->rb[5] = int64_t(k.v_dim / gs) * 2;
      break;
    }
    case TQKV_CACHE_CODEBOOK:
      // codes u8 [dim], sigma f32 (+ QJL sign words u32 and residual norm f32)
      if (k.qjl_words < 0) {
        delete c;
        return fail(TQKV_EINVAL_ARG, "qjl_words=%d", k.qjl_words);
      }
      if (k.qjl_words > 0) {
        c->n_slots = 6;
        c->rb[0] = k.k_dim;
        c->rb[1] = 4;
        c->rb[2] = int64_t(k.qjl_words) * 4;
        c->rb[3] = 4;
        c->rb[4] = k.v_dim;
        c->rb[5] = 4;
      } else {
        c->n_slots = 4;
        c->rb[0] = k.k_dim;
        c->rb[1] = 4;
        c->rb[2] = k.v_dim;
        c->rb[3] = 4;
      }
      if (k.max_size <= 0) {
        delete c;
        return fail(TQKV_EUNSUPPORTED, "codebook caches are rotating (max_size > 0)");
      }
      break;
    default:
      delete c;
      return fail(TQKV_EINVAL_ARG, "kind=%d", k.kind);
  }
  *out = c;
  return ok();
}

int32_t tqkv_cache_destroy(tqkv_cache* c) {
  if (!c) return ok();
  (void)hipDeviceSynchronize();
  for (int s = 0; s < kMaxSlots; ++s) {
    release(c->cur[s]);
    release(c->alt[s]);
  }
  for (void* p : {static_cast<void*>(c->R), static_cast<void*>(c->phi), static_cast<void*>(c->bnd_k),
                  static_cast<void*>(c->bnd_v), static_cast<void*>(c->cent_k), static_cast<void*>(c->cent_v)})
    if (p) (void)hipFree(p);
  delete c;
  return ok();
}

int32_t tqkv_cache_update(tqkv_cache* c, const void* const* rows, int64_t s,
                          tqkv_cache_view* fetched, tqkv_stream stream) {
  if (!c || !rows) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (s <= 0) return fail(TQKV_EINVAL_SHAPE, "update of %lld rows", (long long)s);
  for (int i = 0; i < c->n_slots; ++i)
    if (!rows[i]) return fail(TQKV_EINVAL_ARG, "slot %d rows are null", i);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t old_len = c->st.has ? c->st.len : 0;
  cacheplan::State next = c->st;
  const cacheplan::Plan p = cacheplan::update(next, c->pc, s);
  if (int32_t rc = execute(c, p, old_len, st)) return rc;
  for (int i = 0; i < c->n_slots; ++i)
    if (int32_t rc = rows_copy(st, c->n_slabs, c->rb[i], c->cur[i].ptr, c->cur[i].cap, p.write_at,
                               static_cast<const uint8_t*>(rows[i]), s, 0, s))
      return rc;
  c->st = next;
  c->view_n = p.view;
  if (fetched) fill_view(c, p.view, fetched);
  return ok();
}

int32_t tqkv_cache_append(tqkv_cache* c, const uint16_t* k, const uint16_t* v, int64_t s,
                          tqkv_cache_view* fetched, tqkv_stream stream) {
  if (!c || !k || !v) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (c->cfg.kind == TQKV_CACHE_BF16) {
    const void* rows[2] = {k, v};
    return tqkv_cache_update(c, rows, s, fetched, stream);
  }
  if (s <= 0) return fail(TQKV_EINVAL_SHAPE, "append of %lld rows", (long long)s);
  if (c->cfg.kind == TQKV_CACHE_CODEBOOK) {
    // TurboQuantCompressor::compress of keys (with the QJL stage when the
    // cache keeps signs) and values, straight into the rotating cache rows.
    if (!c->R)
      if (int32_t rc = codebook_tables(c, nullptr, nullptr)) return rc;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int64_t old_len = c->st.has ? c->st.len : 0;
    cacheplan::State next = c->st;
    const cacheplan::Plan p = cacheplan::update(next, c->pc, s);
    if (int32_t rc = execute(c, p, old_len, st)) return rc;
    const tqkv_cache_config& g = c->cfg;
    const bool qjl = g.qjl_words > 0;
    const int vi = qjl ? 4 : 2;
    if (int32_t rc = tqkv_tq_encode(
            k, 1, c->n_slabs, s, g.k_dim, c->R, c->bnd_k, c->cent_k, g.bits_k, c->phi,
            32 * g.qjl_words, c->cur[0].ptr, reinterpret_cast<float*>(c->cur[1].ptr),
            qjl ? reinterpret_cast<uint32_t*>(c->cur[2].ptr) : nullptr,
            qjl ? reinterpret_cast<float*>(c->cur[3].ptr) : nullptr, c->cur[0].cap, p.write_at,
            stream))
      return rc;
    if (int32_t rc = tqkv_tq_encode(v, 1, c->n_slabs, s, g.v_dim, c->R, c->bnd_v, c->cent_v,
                                    g.bits_v, nullptr, 0, c->cur[vi].ptr,
                                    reinterpret_cast<float*>(c->cur[vi + 1].ptr), nullptr, nullptr,
                                    c->cur[vi].cap, p.write_at, stream))
      return rc;
    c->st = next;
    c->view_n = p.view;
    if (fetched) fill_view(c, p.view, fetched);
    return ok();
  }
  if (c->cfg.kind != TQKV_CACHE_AFFINE) return fail(TQKV_EINVAL_ARG, "kind=%d", c->cfg.kind);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int64_t old_len = c->st.has ? c->st.len : 0;
  cacheplan::State next = c->st;
  const cacheplan::Plan p = cacheplan::update(next, c->pc, s);
  if (int32_t rc = execute(c, p, old_len, st)) return rc;
  const tqkv_cache_config& g = c->cfg;
  if (int32_t rc = tqkv_affine_quantize(
          k, c->n_slabs, s, g.k_dim, g.group_size, g.bits_k,
          reinterpret_cast<uint32_t*>(c->cur[0].ptr), reinterpret_cast<uint16_t*>(c->cur[1].ptr),
          reinterpret_cast<uint16_t*>(c->cur[2].ptr), c->cur[0].cap, p.write_at, stream))
    return rc;
  if (int32_t rc = tqkv_affine_quantize(
          v, c->n_slabs, s, g.v_dim, g.group_size, g.bits_v,
          reinterpret_cast<uint32_t*>(c->cur[3].ptr), reinterpret_cast<uint16_t*>(c->cur[4].ptr),
          reinterpret_cast<uint16_t*>(c->cur[5].ptr), c->cur[3].cap, p.write_at, stream))
    return rc;
  c->st = next;
  c->view_n = p.view;
  if (fetched) fill_view(c, p.view, fetched);
  (void)st;
  return ok();
}

int32_t tqkv_cache_truncate(tqkv_cache* c, int64_t target) {
  if (!c) return fail(TQKV_EINVAL_ARG, "null pointer");
  // As NativeKvCache::truncate_to (native_cache.rs:778-811) compares it, the
  // target counts the tokens this buffer holds (not base_offset + them).
  cacheplan::State next = c->st;
  if (!cacheplan::truncate(next, c->pc, target))
    return fail(TQKV_EINVAL_TARGET, "truncate to %lld refused (offset %lld, idx %lld)",
                (long long)target, (long long)c->st.offset, (long long)c->st.idx);
  c->st = next;
  return ok();
}

int32_t tqkv_cache_clear(tqkv_cache* c) {
  if (!c) return fail(TQKV_EINVAL_ARG, "null pointer");
  c->st = cacheplan::State{};
  c->view_n = 0;
  c->base_offset = 0;
  c->prefix = nullptr;
  return ok();
}

int32_t tqkv_cache_get_state(const tqkv_cache* c, tqkv_cache_state* out) {
  if (!c || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  std::memset(out, 0, sizeof(*out));
  out->offset = c->st.offset + c->base_offset;
  out->idx = c->st.idx;
  out->cached_len = c->st.has ? c->st.len : 0;
  out->base_offset = c->base_offset;
  out->view = c->view_n;
  out->empty = c->st.has ? 0 : 1;
  out->n_slots = c->n_slots;
  return ok();
}

int32_t tqkv_cache_buffers(const tqkv_cache* c, tqkv_cache_view* out) {
  if (!c || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  fill_view(c, c->st.has ? c->st.len : 0, out);
  return ok();
}

int32_t tqkv_cache_keep_suffix_from(tqkv_cache* c, int64_t prefix_len, tqkv_stream stream) {
  if (!c) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (c->pc.max_size > 0)
    return fail(TQKV_EUNSUPPORTED, "shared prefixes split growing caches only");
  if (prefix_len <= 0) return ok();
  const int64_t cur = c->base_offset + c->st.offset;
  if (prefix_len > cur)
    return fail(TQKV_EINVAL_TARGET, "prefix_len=%lld > offset=%lld", (long long)prefix_len,
                (long long)cur);
  if (prefix_len <= c->base_offset) return ok();  // already suffix-only at this boundary
  const int64_t drop = prefix_len - c->base_offset;
  const int64_t new_len = c->st.offset - drop;
  if (c->st.has) {
    cacheplan::Plan p;
    cacheplan::push(p, drop, new_len);
    if (int32_t rc = execute(c, p, c->st.len, reinterpret_cast<hipStream_t>(stream))) return rc;
    c->st.len = new_len;
  }
  c->st.offset = new_len;
  c->base_offset = prefix_len;
  c->view_n = new_len;
  return ok();
}

int32_t tqkv_cache_set_tables(tqkv_cache* c, const float* rotation, const float* qjl) {
  if (!c) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (c->cfg.kind != TQKV_CACHE_CODEBOOK)
    return fail(TQKV_EUNSUPPORTED, "tables belong to codebook caches");
  if (int32_t rc = codebook_tables(c, rotation, qjl)) return rc;
  return ok();
}

int32_t tqkv_cache_attach_prefix(tqkv_cache* c, const tqkv_cache* prefix) {
  if (!c) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (!prefix) {
    c->prefix = nullptr;
    return ok();
  }
  const tqkv_cache_config &a = c->cfg, &p = prefix->cfg;
  if (p.batch != 1 || p.kind != a.kind || p.kv_heads != a.kv_heads || p.k_dim != a.k_dim ||
      p.v_dim != a.v_dim || p.group_size != a.group_size || p.bits_k != a.bits_k ||
      p.bits_v != a.bits_v)
    return fail(TQKV_EINVAL_SHAPE, "prefix cache layout does not match");
  if (prefix->st.offset < c->base_offset)
    return fail(TQKV_EINVAL_TARGET, "prefix holds %lld tokens, the suffix starts at %lld",
                (long long)prefix->st.offset, (long long)c->base_offset);
  c->prefix = prefix;
  return ok();
}

int32_t tqkv_cache_decode_attend(const tqkv_cache* c, const uint16_t* q, int32_t H, float scale,
                                 uint16_t* out, void* workspace, size_t workspace_bytes,
                                 tqkv_stream stream) {
  if (!c || !q || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (c->cfg.kind == TQKV_CACHE_CODEBOOK) {
    if (!c->R) return fail(TQKV_EINVAL_ARG, "codebook cache has no tables yet (append first)");
    if (c->view_n <= 0) return fail(TQKV_EINVAL_SHAPE, "no keys to attend");
    const tqkv_cache_config& g = c->cfg;
    const int vi = g.qjl_words > 0 ? 4 : 2;
    return tqkv_decode_attend_codebook(
        q, g.batch, H, g.kv_heads, g.k_dim, scale, c->R, c->cent_k, g.bits_k, c->cent_v, g.bits_v,
        c->cur[0].ptr, reinterpret_cast<const float*>(c->cur[1].ptr), c->cur[vi].ptr,
        reinterpret_cast<const float*>(c->cur[vi + 1].ptr), c->cur[0].cap, c->view_n, out,
        workspace, workspace_bytes, stream);
  }
  if (c->cfg.kind != TQKV_CACHE_AFFINE)
    return fail(TQKV_EUNSUPPORTED, "decode over this cache kind");
  if (c->cfg.k_dim != c->cfg.v_dim)
    return fail(TQKV_EUNSUPPORTED, "decode needs k_dim == v_dim");
  tqkv_affine_seg segs[2];
  const int n = affine_segments(c, segs);
  if (n == 0) return fail(TQKV_EINVAL_SHAPE, "no keys to attend");
  const tqkv_cache_config& g = c->cfg;
  return tqkv_decode_attend_affine(q, g.batch, H, g.kv_heads, g.k_dim, g.group_size, g.bits_k,
                                   g.bits_v, scale, segs, n, out, workspace, workspace_bytes,
                                   stream);
}

int32_t tqkv_cache_prefill_attend(const tqkv_cache* c, const uint16_t* q, int32_t H, int32_t L,
                                  float scale, int64_t window, uint16_t* out,
                                  tqkv_stream stream) {
  if (!c || !q || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (c->cfg.kind != TQKV_CACHE_AFFINE)
    return fail(TQKV_EUNSUPPORTED, "prefill attention over this cache kind");
  if (c->cfg.k_dim != c->cfg.v_dim)
    return fail(TQKV_EUNSUPPORTED, "prefill attention needs k_dim == v_dim");
  const int64_t offset = c->base_offset + c->st.offset;
  if (L <= 0 || L > offset)
    return fail(TQKV_EINVAL_SHAPE, "L=%d queries but %lld tokens appended", L, (long long)offset);
  tqkv_affine_seg segs[2];
  const int n = affine_segments(c, segs);
  if (n == 0) return fail(TQKV_EINVAL_SHAPE, "no keys to attend");
  const int64_t keys = segs[0].n + (n == 2 ? segs[1].n : 0);
  const tqkv_cache_config& g = c->cfg;
  return tqkv_prefill_attend_affine(q, g.batch, H, g.kv_heads, L, g.k_dim, g.group_size,
                                    g.bits_k, g.bits_v, scale, segs, n, offset - L,
                                    offset - keys, 1, window, out, stream);
}

}  // extern "C"
