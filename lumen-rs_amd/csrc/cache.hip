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
#include <algorithm>
#include <type_traits>
#include <cstring>
#include <new>
#include <vector>

#include "cache_plan.hpp"
#include "common.hpp"
#include "lkv.hpp"

namespace tqkv {
size_t decode_need_bytes(int B, int H, int H_kv, int D, int group_size, int bits_k, int bits_v,
                         const tqkv_affine_seg* segs, int n_segs, bool app);
int32_t prefill_bf16_rows(const uint16_t* q, int B, int H, int H_kv, int L, int D,
                          const uint16_t* k, const uint16_t* v, int64_t cap, int64_t n,
                          int64_t q_start, int64_t k_start, int64_t window, float scale,
                          uint16_t* out, hipStream_t stream);
int32_t codebook_dequantize_slabs(const uint8_t* codes, const float* sigma, const float* cent,
                                  int bits, int64_t slabs, int64_t cap, int64_t rows, int D,
                                  uint16_t* out, hipStream_t st);
int32_t decode_codebook_qjl_rotated(
    const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t D, float scale,
    const float* rotation, const float* centroids_k, int32_t bits_k, const float* centroids_v,
    int32_t bits_v, const uint8_t* k_codes, const float* k_sigma, const uint32_t* k_signs,
    const float* k_rnorm, const float* qjl, int32_t qjl_m, const uint8_t* v_codes,
    const float* v_sigma, int64_t cap, int64_t n, uint16_t* out, void* workspace,
    size_t workspace_bytes, tqkv_stream stream);
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

// The copies of one plan step over every slot, in one launch: job z copies
// rows [src_row, src_row + n) of every slab of src (zeros when src is null)
// into rows [dst_row, ...) of dst, slab strides src_cap / dst_cap rows of rb
// bytes. (Per slot and piece, a step was up to a dozen launches of a few µs
// each.)
struct CopyJob {
  uint8_t* dst;
  const uint8_t* src;
  int64_t dst_cap, dst_row, src_cap, src_row, n, rb;
  int words;  // 4-byte units (everything 4-aligned)
};
constexpr int kMaxJobs = 24;
struct CopyBatch {
  CopyJob job[kMaxJobs];
  int n_jobs;
};

__global__ void rows_copy_batch_kernel(const CopyBatch b) {
  const CopyJob& j = b.job[blockIdx.z];
  const int64_t slab = blockIdx.y;
  const int64_t bytes = j.n * j.rb;
  uint8_t* d = j.dst + (slab * j.dst_cap + j.dst_row) * j.rb;
  const uint8_t* src = j.src ? j.src + (slab * j.src_cap + j.src_row) * j.rb : nullptr;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  if (j.words) {
    uint32_t* dw = reinterpret_cast<uint32_t*>(d);
    const uint32_t* sw = reinterpret_cast<const uint32_t*>(src);
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes / 4; i += stride)
      dw[i] = sw ? sw[i] : 0u;
  } else {
    for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes; i += stride)
      d[i] = src ? src[i] : uint8_t(0);
  }
}

class CopyBatcher {
 public:
  CopyBatcher(hipStream_t st, int64_t n_slabs) : st_(st), n_slabs_(n_slabs) { b_.n_jobs = 0; }
  int32_t add(uint8_t* dst, int64_t dst_cap, int64_t dst_row, const uint8_t* src, int64_t src_cap,
              int64_t src_row, int64_t n, int64_t rb) {
    if (n <= 0 || n_slabs_ <= 0) return TQKV_OK;
    if (b_.n_jobs == kMaxJobs)
      if (int32_t rc = flush()) return rc;
    const bool words = (rb % 4 == 0) && (reinterpret_cast<uintptr_t>(dst) % 4 == 0) &&
                       (!src || reinterpret_cast<uintptr_t>(src) % 4 == 0);
    b_.job[b_.n_jobs++] = CopyJob{dst, src, dst_cap, dst_row, src_cap, src_row, n, rb, words ? 1 : 0};
    const int64_t units = words ? n * rb / 4 : n * rb;
    const int64_t blocks = (units + 255) / 256;
    if (blocks > blocks_) blocks_ = blocks > 1024 ? 1024 : blocks;
    return TQKV_OK;
  }
  int32_t flush() {
    if (b_.n_jobs == 0) return TQKV_OK;
    if (n_slabs_ > 65535)
      return fail(TQKV_EINVAL_SHAPE, "%lld slabs exceed one launch", (long long)n_slabs_);
    hipLaunchKernelGGL(rows_copy_batch_kernel,
                       dim3(unsigned(blocks_), unsigned(n_slabs_), unsigned(b_.n_jobs)), dim3(256),
                       0, st_, b_);
    TQKV_LAUNCHED();
    b_.n_jobs = 0;
    blocks_ = 0;
    return TQKV_OK;
  }

 private:
  hipStream_t st_;
  int64_t n_slabs_;
  CopyBatch b_{};
  int64_t blocks_ = 0;
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
  float* inner_k = nullptr;    // [2^bits_k - 1] inner boundaries as f32 (GPU-path encode)
  float* inner_v = nullptr;
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
  // Every slot's copies go out in one batch; buffers they replace are freed
  // once the stream has drained past them (one wait, not one per slot).
  CopyBatcher cb(st, c->n_slabs);
  Buf retired[kMaxSlots];
  int n_retired = 0;
  // Launches what was batched, then (after the stream has drained past the
  // replaced buffers) frees them; on an error too, so nothing leaks.
  auto finish = [&](int32_t rc) {
    const int32_t frc = cb.flush();
    if (n_retired > 0) {
      const hipError_t e = hipStreamSynchronize(st);
      for (int i = 0; i < n_retired; ++i) release(retired[i]);
      if (rc == TQKV_OK && e != hipSuccess)
        return fail(TQKV_EDEVICE, "hipStreamSynchronize: %s", hipGetErrorString(e));
    }
    return rc != TQKV_OK ? rc : frc;
  };
  for (int s = 0; s < c->n_slots; ++s) {
    Buf& cur = c->cur[s];
    const int64_t rb = c->rb[s];
    if (in_place) {
      if (cur.cap < p.len) {
        Buf nb;
        if (int32_t rc = alloc(c, nb, capacity_for(c, p.len, cur.cap), s)) return finish(rc);
        if (int32_t rc = cb.add(nb.ptr, nb.cap, 0, cur.ptr, cur.cap, 0, a, rb)) {
          release(nb);
          return finish(rc);
        }
        if (cur.ptr) retired[n_retired++] = cur;
        cur = nb;
      }
      if (int32_t rc = cb.add(cur.ptr, cur.cap, a, nullptr, 0, 0, p.len - a, rb))
        return finish(rc);
    } else {
      Buf& alt = c->alt[s];
      if (alt.cap < p.len) {
        if (alt.ptr) retired[n_retired++] = alt;
        alt = Buf{};
        if (int32_t rc = alloc(c, alt, capacity_for(c, p.len, cur.cap), s)) return finish(rc);
      }
      int64_t at = 0;
      for (const cacheplan::Piece& q : p.pieces) {
        if (int32_t rc = cb.add(alt.ptr, alt.cap, at, q.src >= 0 ? cur.ptr : nullptr, cur.cap,
                                q.src >= 0 ? q.src : 0, q.n, rb))
          return finish(rc);
        at += q.n;
      }
      std::swap(cur, alt);
    }
  }
  return finish(TQKV_OK);
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
    std::vector<float> inner(b.begin() + 1, b.end() - 1);  // lloyd_max_boundaries_inner
    if (int32_t rc = upload(reinterpret_cast<void**>(kv ? &c->bnd_v : &c->bnd_k), b.data(), b.size() * 8)) return rc;
    if (int32_t rc = upload(reinterpret_cast<void**>(kv ? &c->cent_v : &c->cent_k), cf.data(), cf.size() * 4)) return rc;
    if (int32_t rc = upload(reinterpret_cast<void**>(kv ? &c->inner_v : &c->inner_k), inner.data(), inner.size() * 4)) return rc;
  }
  std::vector<float> R(size_t(D) * D);
  if (R_host) std::memcpy(R.data(), R_host, R.size() * 4);
  else if (int32_t rc = tqkv_rotation_matrix(D, g.seed, R.data())) return rc;
  if (g.encode == 1) {
    // The GPU path stores x R = R^T x: the cache's rotation (the one its
    // decode and prefill apply to queries, R_eff x) is R^T.
    std::vector<float> Rt(R.size());
    for (int i = 0; i < D; ++i)
      for (int j = 0; j < D; ++j) Rt[size_t(i) * D + j] = R[size_t(j) * D + i];
    R.swap(Rt);
  }
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

// ---- LKV2 snapshots (kv_disk.rs): one cache = one layer.

// One record of a layer: rows [0, rows) of every slab of a slot, or (signs)
// a slot of packed QJL sign words widened to the reference's bf16 +-1
// layout [B, H_kv, S, m] (the TurboQuant cache's keys_signs, native_cache.rs:1524).
struct RecSpec {
  int slot = 0;
  uint8_t dtype = 0;
  std::vector<int64_t> shape;
  int64_t rows = 0;
  bool signs = false;
  uint64_t bytes() const {
    uint64_t n = lkv::elem_size(dtype);
    for (int64_t d : shape) n *= uint64_t(d);
    return n;
  }
};

struct LayerPlan {
  lkv::Layer meta;
  std::vector<RecSpec> recs;
};

lkv::Opt some(uint64_t v) { return lkv::Opt{true, v}; }

// The layer's LayerMeta and records, as the reference's snapshot code lays
// them out: bf16 growing = Full with the logical view [0, offset)
// (gemma4_moe.rs:1638-1645); rotating bf16 = Sliding with the whole ring and
// max_size / keep / idx (:1646-1657); affine = FullQuantized /
// SlidingQuantized with the whole (packed, scales, biases) buffers of K then V
// and group_size / bits (:1658-1679); codebook = FullTurboquant /
// SlidingTurboquant with [keys_codes, keys_sigma, values_codes, values_sigma,
// keys_signs?, keys_residual_norm?] and max_size / keep / idx / bits / qjl_m
// (kv_disk.rs:2005-2025). `first` is the index of its first record.
int32_t plan_layer(const tqkv_cache* c, int64_t first, LayerPlan* out) {
  const tqkv_cache_config& g = c->cfg;
  // A snapshot layer records no encode chain, and import rebuilds a
  // compress_one cache: GPU-path rows would come back in the wrong basis.
  if (g.encode != 0)
    return fail(TQKV_EUNSUPPORTED, "snapshots of GPU-path (encode = 1) codebook caches");
  LayerPlan L;
  const bool ring = g.max_size > 0;
  const int64_t B = g.batch, H = g.kv_heads;
  auto rec = [&](int slot, uint8_t dtype, int64_t rows, int64_t last, bool signs = false) {
    RecSpec r;
    r.slot = slot;
    r.dtype = dtype;
    r.rows = rows;
    r.shape = {B, H, rows, last};
    r.signs = signs;
    L.recs.push_back(r);
    L.meta.arrays.push_back(first + int64_t(L.recs.size()) - 1);
  };
  const bool has = c->st.has;
  const int64_t len = has ? c->st.len : 0;
  L.meta.offset = uint64_t(c->base_offset + c->st.offset);
  L.meta.base_offset = uint64_t(c->base_offset);
  switch (g.kind) {
    case TQKV_CACHE_BF16:
      L.meta.kind = ring ? "Sliding" : "Full";
      if (has) {
        const int64_t rows = ring ? len : c->st.offset;
        rec(0, lkv::kBF16, rows, g.k_dim);
        rec(1, lkv::kBF16, rows, g.v_dim);
      } else {
        L.meta.arrays = {-1, -1};
      }
      break;
    case TQKV_CACHE_AFFINE:
      L.meta.kind = ring ? "SlidingQuantized" : "FullQuantized";
      if (has) {
        rec(0, lkv::kU32, len, int64_t(g.k_dim) * g.bits_k / 32);
        rec(1, lkv::kBF16, len, g.k_dim / g.group_size);
        rec(2, lkv::kBF16, len, g.k_dim / g.group_size);
        rec(3, lkv::kU32, len, int64_t(g.v_dim) * g.bits_v / 32);
        rec(4, lkv::kBF16, len, g.v_dim / g.group_size);
        rec(5, lkv::kBF16, len, g.v_dim / g.group_size);
      } else {
        L.meta.arrays = {-1, -1, -1, -1, -1, -1};
      }
      L.meta.has_group_size = true;
      L.meta.group_size = g.group_size;
      // One width in the reference's metadata; the value width of a K8/V4
      // cache follows from its packed record's shape on import.
      L.meta.bits = some(uint64_t(g.bits_k));
      break;
    case TQKV_CACHE_CODEBOOK: {
      if (g.bits_k != g.bits_v)
        return fail(TQKV_EUNSUPPORTED, "a TurboQuant snapshot layer has one width (bits %d/%d)",
                    g.bits_k, g.bits_v);
      L.meta.kind = g.max_size >= (int64_t(1) << 31) ? "FullTurboquant" : "SlidingTurboquant";
      const bool qjl = g.qjl_words > 0;
      const int vs = qjl ? 4 : 2;
      if (has) {
        rec(0, lkv::kU8, len, g.k_dim);
        rec(1, lkv::kF32, len, 1);
        rec(vs, lkv::kU8, len, g.v_dim);
        rec(vs + 1, lkv::kF32, len, 1);
        if (qjl) {
          rec(2, lkv::kBF16, len, int64_t(32) * g.qjl_words, true);
          rec(3, lkv::kF32, len, 1);
        } else {
          L.meta.arrays.push_back(-1);
          L.meta.arrays.push_back(-1);
        }
      } else {
        L.meta.arrays = {-1, -1, -1, -1, -1, -1};
      }
      L.meta.bits = some(uint64_t(g.bits_k));
      if (qjl) L.meta.qjl_m = some(uint64_t(32) * g.qjl_words);
      break;
    }
    default:
      return fail(TQKV_EUNSUPPORTED, "cache kind %d", g.kind);
  }
  if (ring) {
    L.meta.max_size = some(uint64_t(g.max_size));
    L.meta.keep = some(uint64_t(g.keep));
    L.meta.idx = some(uint64_t(c->st.idx));
  }
  *out = std::move(L);
  return TQKV_OK;
}

// Copies a record's payload from the device into `dst`.
int32_t read_record(const tqkv_cache* c, const RecSpec& r, uint8_t* dst) {
  const Buf& b = c->cur[r.slot];
  const int64_t rb = c->rb[r.slot];
  if (r.rows == 0 || c->n_slabs == 0) return TQKV_OK;
  if (!r.signs) {
    TQKV_HIP(hipMemcpy2D(dst, size_t(r.rows * rb), b.ptr, size_t(b.cap * rb), size_t(r.rows * rb),
                         size_t(c->n_slabs), hipMemcpyDeviceToHost));
    return TQKV_OK;
  }
  const int64_t words = rb / 4, m = 32 * words;
  std::vector<uint32_t> w(size_t(c->n_slabs * r.rows * words));
  TQKV_HIP(hipMemcpy2D(w.data(), size_t(r.rows * rb), b.ptr, size_t(b.cap * rb),
                       size_t(r.rows * rb), size_t(c->n_slabs), hipMemcpyDeviceToHost));
  // Sign bit i set <=> (Phi r)_i >= 0 <=> +1 (qjl.rs:57-74).
  uint16_t* o = reinterpret_cast<uint16_t*>(dst);
  for (size_t row = 0; row < size_t(c->n_slabs * r.rows); ++row)
    for (int64_t i = 0; i < m; ++i)
      o[row * size_t(m) + size_t(i)] = (w[row * size_t(words) + size_t(i / 32)] >> (i % 32)) & 1u
                                           ? uint16_t(0x3F80) : uint16_t(0xBF80);
  return TQKV_OK;
}

// Uploads a record's payload into rows [0, rows) of a slot.
int32_t write_record(tqkv_cache* c, const RecSpec& r, const uint8_t* src) {
  Buf& b = c->cur[r.slot];
  const int64_t rb = c->rb[r.slot];
  if (r.rows == 0 || c->n_slabs == 0) return TQKV_OK;
  if (!r.signs) {
    TQKV_HIP(hipMemcpy2D(b.ptr, size_t(b.cap * rb), src, size_t(r.rows * rb), size_t(r.rows * rb),
                         size_t(c->n_slabs), hipMemcpyHostToDevice));
    return TQKV_OK;
  }
  const int64_t words = rb / 4, m = 32 * words;
  std::vector<uint32_t> w(size_t(c->n_slabs * r.rows * words), 0u);
  for (size_t row = 0; row < size_t(c->n_slabs * r.rows); ++row)
    for (int64_t i = 0; i < m; ++i) {
      uint16_t x;
      std::memcpy(&x, src + 2 * (row * size_t(m) + size_t(i)), 2);
      if (!(x & 0x8000u)) w[row * size_t(words) + size_t(i / 32)] |= 1u << (i % 32);
    }
  TQKV_HIP(hipMemcpy2D(b.ptr, size_t(b.cap * rb), w.data(), size_t(r.rows * rb),
                       size_t(r.rows * rb), size_t(c->n_slabs), hipMemcpyHostToDevice));
  return TQKV_OK;
}

}  // namespace

namespace {

// The reference GPU cache's append of s rows a slab at row `row` (gemma4_moe.rs:
// 4384-4430 with its defaults): keys and values rotated by rotate_last_axis
// (x R, bf16) and encoded by lloyd_max_quantize_stage1 (tqkv_tq_encode_gpu_path
// mode 1; the cache keeps R^T, so x R = x R_eff^T); with QJL, the keys' signs
// and residual norms from the rotated keys against their dequantized codes
// (qjl_encode_stage2_packed).
int32_t append_gpu_path(tqkv_cache* c, const uint16_t* k, const uint16_t* v, int64_t s,
                        int64_t row, hipStream_t st) {
  const tqkv_cache_config& g = c->cfg;
  const int D = g.k_dim;
  const bool qjl = g.qjl_words > 0;
  const int vi = qjl ? 4 : 2;
  const int64_t rows = c->n_slabs * s, cap = c->cur[0].cap;
  const tqkv_stream ts = reinterpret_cast<tqkv_stream>(st);
  if (!qjl) {
    if (int32_t rc = tqkv_tq_encode_gpu_path(k, c->n_slabs, s, D, c->R, 1, 1, c->inner_k, g.bits_k,
                                             c->cur[0].ptr, reinterpret_cast<float*>(c->cur[1].ptr),
                                             cap, row, ts))
      return rc;
  } else {
    const int words = g.qjl_words, m = 32 * words;
    const size_t need = size_t(rows) * D * 2 * 2 + size_t(rows) * (words * 4 + 4) + 64;
    void* ws = nullptr;
    if (int32_t rc = scratch_for_current_device(need, &ws)) return rc;
    uint16_t* k_rot = static_cast<uint16_t*>(ws);
    uint16_t* k_dq = k_rot + size_t(rows) * D;
    uint32_t* sg = reinterpret_cast<uint32_t*>(k_dq + size_t(rows) * D);
    float* rn = reinterpret_cast<float*>(sg + size_t(rows) * words);
    if (int32_t rc = tqkv_rotate_bf16(k, rows, D, c->R, 1, k_rot, ts)) return rc;
    if (int32_t rc = tqkv_tq_encode_gpu_path(k_rot, c->n_slabs, s, D, nullptr, 0, 0, c->inner_k,
                                             g.bits_k, c->cur[0].ptr,
                                             reinterpret_cast<float*>(c->cur[1].ptr), cap, row, ts))
      return rc;
    if (int32_t rc = codebook_dequantize_slabs(c->cur[0].ptr + row * D,
                                               reinterpret_cast<const float*>(c->cur[1].ptr) + row,
                                               c->cent_k, g.bits_k, c->n_slabs, cap, s, D, k_dq, st))
      return rc;
    if (int32_t rc = tqkv_qjl_encode_stage2(k_rot, k_dq, c->phi, rows, D, m, sg, rn, ts))
      return rc;
    // Into rows [row, row + s) of every slab of the signs and norms slots.
    const size_t sw = size_t(words) * 4;
    TQKV_HIP(hipMemcpy2DAsync(c->cur[2].ptr + row * sw, size_t(cap) * sw, sg, size_t(s) * sw,
                              size_t(s) * sw, size_t(c->n_slabs), hipMemcpyDeviceToDevice, st));
    TQKV_HIP(hipMemcpy2DAsync(c->cur[3].ptr + row * 4, size_t(cap) * 4, rn, size_t(s) * 4,
                              size_t(s) * 4, size_t(c->n_slabs), hipMemcpyDeviceToDevice, st));
  }
  return tqkv_tq_encode_gpu_path(v, c->n_slabs, s, D, c->R, 1, 1, c->inner_v, g.bits_v,
                                 c->cur[vi].ptr, reinterpret_cast<float*>(c->cur[vi + 1].ptr),
                                 c->cur[vi].cap, row, ts);
}

// Prefill over a codebook (TurboQuant) cache, as the reference's TurboQuant
// branch does (gemma4_moe.rs:4546-4600): K and V of the view dequantized to
// bf16(centroid * sigma) (lloyd_max_dequantize_scaled), keys with QJL signs
// corrected to K_eff (qjl_apply_correction_packed), V rotated back to the
// original basis (its unrotate_v_dq), then the chunk's attention. The cache
// holds rotated rows (R x), so the queries are rotated by R (bf16, as
// rotate_last_axis returns them) to meet the keys. bf16 caches take the
// attention step directly over their buffers.
int32_t prefill_rows(const tqkv_cache* c, const uint16_t* q, int32_t H, int32_t L, float scale,
                     int64_t window, uint16_t* out, hipStream_t st) {
  const tqkv_cache_config& g = c->cfg;
  const int D = g.k_dim;
  if (g.k_dim != g.v_dim) return fail(TQKV_EUNSUPPORTED, "prefill attention needs k_dim == v_dim");
  if (c->prefix && c->base_offset > 0)
    return fail(TQKV_EUNSUPPORTED, "prefill over an attached prefix of this cache kind");
  const int64_t offset = c->base_offset + c->st.offset;
  if (H <= 0 || H % g.kv_heads != 0 || L <= 0 || L > offset)
    return fail(TQKV_EINVAL_SHAPE, "H=%d L=%d queries but %lld tokens appended", H, L,
                (long long)offset);
  const int64_t n = c->view_n;
  if (n <= 0) return fail(TQKV_EINVAL_SHAPE, "no keys to attend");
  const int64_t cap = c->cur[0].cap;
  const int64_t q_start = offset - L, k_start = offset - n;
  if (g.kind == TQKV_CACHE_BF16)
    return prefill_bf16_rows(q, g.batch, H, g.kv_heads, L, D,
                             reinterpret_cast<const uint16_t*>(c->cur[0].ptr),
                             reinterpret_cast<const uint16_t*>(c->cur[1].ptr), cap, n, q_start,
                             k_start, window, scale, out, st);
  if (!c->R) return fail(TQKV_EINVAL_ARG, "codebook cache has no tables yet (append first)");
  // compress_one's QJL signs are of the original-basis residual; the
  // reference's prefill correction (qjl_apply_correction_packed) adds
  // Phi^T signs in the rotated basis, which holds only for the rotated
  // residual signs its GPU cache stores.
  if (g.qjl_words > 0 && g.encode == 0)
    return fail(TQKV_EUNSUPPORTED, "prefill over compress_one codes with QJL signs (the "
                "reference prefills QJL only over its GPU-path cache)");
  const int64_t slabs = int64_t(g.batch) * g.kv_heads;
  const size_t qe = size_t(g.batch) * H * L * D;  // query / output elements
  const size_t ke = size_t(slabs) * n * D;        // dequantized K or V elements
  const bool qjl = g.qjl_words > 0;
  const size_t need = (qe + 3 * ke + (qjl ? size_t(n) * D : 0)) * sizeof(uint16_t) + 64;
  void* ws = nullptr;
  if (int32_t rc = scratch_for_current_device(need, &ws)) return rc;
  uint16_t* qr = static_cast<uint16_t*>(ws);
  uint16_t* kd = qr + qe;
  uint16_t* vd = kd + ke;   // V_dq in the rotated basis
  uint16_t* vo = vd + ke;   // V_dq rotated back
  uint16_t* tmp = vo + ke;  // one slab's K_dq before the QJL correction
  const int vi = qjl ? 4 : 2;
  if (int32_t rc = tqkv_rotate_bf16(q, int64_t(g.batch) * H * L, D, c->R, 1, qr,
                                    reinterpret_cast<tqkv_stream>(st)))
    return rc;
  if (!qjl) {
    if (int32_t rc = codebook_dequantize_slabs(c->cur[0].ptr,
                                               reinterpret_cast<const float*>(c->cur[1].ptr),
                                               c->cent_k, g.bits_k, slabs, cap, n, D, kd, st))
      return rc;
  } else {
    const int words = g.qjl_words;
    for (int64_t sl = 0; sl < slabs; ++sl) {
      if (int32_t rc = codebook_dequantize_slabs(
              c->cur[0].ptr + sl * cap * D, reinterpret_cast<const float*>(c->cur[1].ptr) + sl * cap,
              c->cent_k, g.bits_k, 1, cap, n, D, tmp, st))
        return rc;
      if (int32_t rc = tqkv_qjl_apply_correction(
              tmp, reinterpret_cast<const uint32_t*>(c->cur[2].ptr) + sl * cap * words,
              reinterpret_cast<const float*>(c->cur[3].ptr) + sl * cap, c->phi, n, D,
              32 * words, kd + sl * n * D, reinterpret_cast<tqkv_stream>(st)))
        return rc;
    }
  }
  if (int32_t rc = codebook_dequantize_slabs(c->cur[vi].ptr,
                                             reinterpret_cast<const float*>(c->cur[vi + 1].ptr),
                                             c->cent_v, g.bits_v, slabs, cap, n, D, vd, st))
    return rc;
  // A row y = R v goes back as y R (= (R^T y)^T).
  if (int32_t rc = tqkv_rotate_bf16(vd, slabs * n, D, c->R, 0, vo,
                                    reinterpret_cast<tqkv_stream>(st)))
    return rc;
  return prefill_bf16_rows(qr, g.batch, H, g.kv_heads, L, D, kd, vo, n, n, q_start, k_start,
                           window, scale, out, st);
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
  if (k.encode < 0 || k.encode > 1 || (k.encode != 0 && k.kind != TQKV_CACHE_CODEBOOK))
    return fail(TQKV_EINVAL_ARG, "encode=%d (0 or 1, and 1 for codebook caches only)", k.encode);
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

int32_t tqkv_cache_clone(const tqkv_cache* src, tqkv_cache** out, tqkv_stream stream) {
  if (!src || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  *out = nullptr;
  tqkv_cache* c = nullptr;
  if (int32_t rc = tqkv_cache_create(&src->cfg, &c)) return rc;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  auto copy = [&](void* dst, const void* from, size_t bytes) -> int32_t {
    TQKV_HIP(hipMemcpyAsync(dst, from, bytes, hipMemcpyDeviceToDevice, st));
    return TQKV_OK;
  };
  auto table = [&](auto** dst, const auto* from, size_t bytes) -> int32_t {
    if (!from) return TQKV_OK;
    void* p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return fail(TQKV_ENOMEM, "table hipMalloc");
    *dst = static_cast<std::remove_pointer_t<decltype(dst)>>(p);
    return copy(p, from, bytes);
  };
  int32_t rc = TQKV_OK;
  for (int s = 0; s < src->n_slots && rc == TQKV_OK; ++s) {
    const Buf& b = src->cur[s];
    if (!b.ptr) continue;
    rc = alloc(c, c->cur[s], b.cap, s);
    if (rc == TQKV_OK)
      rc = copy(c->cur[s].ptr, b.ptr, size_t(src->n_slabs) * size_t(b.cap) * size_t(src->rb[s]));
  }
  if (rc == TQKV_OK && src->R) {
    const size_t D = size_t(src->cfg.k_dim), m = size_t(32) * size_t(src->cfg.qjl_words);
    const size_t nk = size_t(1) << src->cfg.bits_k, nv = size_t(1) << src->cfg.bits_v;
    rc = table(&c->R, src->R, D * D * sizeof(float));
    if (rc == TQKV_OK && m) rc = table(&c->phi, src->phi, m * D * sizeof(float));
    if (rc == TQKV_OK) rc = table(&c->bnd_k, src->bnd_k, (nk + 1) * sizeof(double));
    if (rc == TQKV_OK) rc = table(&c->bnd_v, src->bnd_v, (nv + 1) * sizeof(double));
    if (rc == TQKV_OK) rc = table(&c->cent_k, src->cent_k, nk * sizeof(float));
    if (rc == TQKV_OK) rc = table(&c->cent_v, src->cent_v, nv * sizeof(float));
    if (rc == TQKV_OK) rc = table(&c->inner_k, src->inner_k, (nk - 1) * sizeof(float));
    if (rc == TQKV_OK) rc = table(&c->inner_v, src->inner_v, (nv - 1) * sizeof(float));
  }
  if (rc != TQKV_OK) {
    tqkv_cache_destroy(c);
    return rc;
  }
  c->st = src->st;
  c->view_n = src->view_n;
  c->base_offset = src->base_offset;
  c->prefix = src->prefix;  // a shared prefix stays shared by every fork
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
                  static_cast<void*>(c->bnd_v), static_cast<void*>(c->cent_k), static_cast<void*>(c->cent_v),
                  static_cast<void*>(c->inner_k), static_cast<void*>(c->inner_v)})
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
    if (g.encode == 1) {
      if (int32_t rc = append_gpu_path(c, k, v, s, p.write_at, st)) return rc;
      c->st = next;
      c->view_n = p.view;
      if (fetched) fill_view(c, p.view, fetched);
      return ok();
    }
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
  if (g.k_dim == g.v_dim && c->cur[0].cap == c->cur[3].cap) {
    // Keys and values in one launch.
    if (int32_t rc = tqkv_affine_quantize_kv(
            k, v, c->n_slabs, s, g.k_dim, g.group_size, g.bits_k, g.bits_v,
            reinterpret_cast<uint32_t*>(c->cur[0].ptr), reinterpret_cast<uint16_t*>(c->cur[1].ptr),
            reinterpret_cast<uint16_t*>(c->cur[2].ptr), reinterpret_cast<uint32_t*>(c->cur[3].ptr),
            reinterpret_cast<uint16_t*>(c->cur[4].ptr), reinterpret_cast<uint16_t*>(c->cur[5].ptr),
            c->cur[0].cap, p.write_at, stream))
      return rc;
    c->st = next;
    c->view_n = p.view;
    if (fetched) fill_view(c, p.view, fetched);
    return ok();
  }
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
    if (g.qjl_words > 0)  // keys' QJL residual signs correct the scores
      return (g.encode == 1 ? decode_codebook_qjl_rotated : tqkv_decode_attend_codebook_qjl)(
          q, g.batch, H, g.kv_heads, g.k_dim, scale, c->R, c->cent_k, g.bits_k, c->cent_v,
          g.bits_v, c->cur[0].ptr, reinterpret_cast<const float*>(c->cur[1].ptr),
          reinterpret_cast<const uint32_t*>(c->cur[2].ptr),
          reinterpret_cast<const float*>(c->cur[3].ptr), c->phi, 32 * g.qjl_words,
          c->cur[vi].ptr, reinterpret_cast<const float*>(c->cur[vi + 1].ptr), c->cur[0].cap,
          c->view_n, out, workspace, workspace_bytes, stream);
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

int32_t tqkv_cache_append_decode(tqkv_cache* c, const uint16_t* k, const uint16_t* v,
                                 const uint16_t* q, int32_t H, float scale, uint16_t* out,
                                 void* workspace, size_t workspace_bytes, tqkv_stream stream) {
  if (!c || !k || !v || !q || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  auto two_calls = [&]() -> int32_t {
    if (int32_t rc = tqkv_cache_append(c, k, v, 1, nullptr, stream)) return rc;
    return tqkv_cache_decode_attend(c, q, H, scale, out, workspace, workspace_bytes, stream);
  };
  const tqkv_cache_config& g = c->cfg;
  if (g.kind != TQKV_CACHE_AFFINE || g.k_dim != g.v_dim || H <= 0 || H % g.kv_heads != 0)
    return two_calls();
  // TQKV_FUSED_APPEND=0 keeps the two calls (tests compare the paths).
  const char* env = getenv("TQKV_FUSED_APPEND");
  if (env && strcmp(env, "0") == 0) return two_calls();
  if (strcmp(tqkv_decode_kernel_name(H, g.kv_heads, g.k_dim, g.group_size, g.bits_k, g.bits_v),
             "mfma") != 0 ||
      (reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) % 16 != 0)
    return two_calls();
  cacheplan::State next = c->st;
  const cacheplan::Plan p = cacheplan::update(next, c->pc, 1);
  // The attended rows are the new view without the new row: [0, view - 1)
  // when the row lands last, else (a ring written in place) the rows either
  // side of it, which with an attached prefix would be a third segment.
  const bool has_prefix = c->prefix && c->base_offset > 0;
  const bool last = p.write_at == p.view - 1;
  if (p.write_at < 0 || p.write_at >= p.view || (!last && has_prefix)) return two_calls();
  if (c->cur[0].cap != c->cur[3].cap)
    return fail(TQKV_EINVAL_ARG, "K and V buffers of different capacity");
  // The decode must not fail once the update is committed (its row is only
  // written by the decode kernel): the kernel it will pick and the
  // workspace it will need are settled first, from the segment lengths it
  // will attend (a segment too long for the MFMA kernel's 32-bit offsets
  // takes the dot2 kernel, which cannot append: two calls then).
  {
    tqkv_affine_seg vs[2]{};
    int vn = 0;
    if (has_prefix) {
      vs[vn].n = c->base_offset;
      vs[vn++].shared = 1;
    }
    if (last) {
      vs[vn++].n = p.view - 1;
    } else {
      vs[vn++].n = p.write_at;
      vs[vn++].n = p.view - p.write_at - 1;
    }
    int64_t max_rows = 0;
    for (int i = 0; i < vn; ++i) max_rows = vs[i].n > max_rows ? vs[i].n : max_rows;
    if (strcmp(tqkv_decode_kernel_for_rows(H, g.kv_heads, g.k_dim, g.group_size, g.bits_k,
                                           g.bits_v, max_rows),
               "mfma") != 0)
      return two_calls();
    const size_t need = decode_need_bytes(g.batch, H, g.kv_heads, g.k_dim, g.group_size,
                                          g.bits_k, g.bits_v, vs, vn, true);
    if (need > 0) {
      if (!workspace) {
        void* ws = nullptr;
        if (int32_t rc = scratch_for_current_device(need, &ws)) return rc;
      } else if (workspace_bytes < need) {
        return fail(TQKV_EINVAL_ARG, "workspace of %zu bytes, need %zu", workspace_bytes, need);
      }
    }
  }
  const int64_t old_len = c->st.has ? c->st.len : 0;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (int32_t rc = execute(c, p, old_len, st)) return rc;
  c->st = next;
  c->view_n = p.view;
  tqkv_affine_seg segs[2];
  int n = affine_segments(c, segs);
  tqkv_affine_seg& own = segs[n - 1];  // the cache's own rows (view >= 1)
  if (last) {
    own.n -= 1;
  } else {
    // [0, write_at) and [write_at + 1, view) of the same slabs.
    const int64_t r1 = p.write_at + 1;
    const int kr = g.k_dim * g.bits_k / 32, vr = g.v_dim * g.bits_v / 32;
    const int ng = g.k_dim / g.group_size;
    tqkv_affine_seg hi = own;
    hi.k_packed += r1 * kr;
    hi.k_scales += r1 * ng;
    hi.k_biases += r1 * ng;
    hi.v_packed += r1 * vr;
    hi.v_scales += r1 * ng;
    hi.v_biases += r1 * ng;
    hi.n = p.view - r1;
    own.n = p.write_at;
    segs[n++] = hi;
  }
  return tqkv_decode_attend_affine_append(
      q, g.batch, H, g.kv_heads, g.k_dim, g.group_size, g.bits_k, g.bits_v, scale, segs, n, k, v,
      reinterpret_cast<uint32_t*>(c->cur[0].ptr), reinterpret_cast<uint16_t*>(c->cur[1].ptr),
      reinterpret_cast<uint16_t*>(c->cur[2].ptr), reinterpret_cast<uint32_t*>(c->cur[3].ptr),
      reinterpret_cast<uint16_t*>(c->cur[4].ptr), reinterpret_cast<uint16_t*>(c->cur[5].ptr),
      c->cur[0].cap, p.write_at, out, workspace, workspace_bytes, stream);
}

int32_t tqkv_cache_prefill_attend(const tqkv_cache* c, const uint16_t* q, int32_t H, int32_t L,
                                  float scale, int64_t window, uint16_t* out,
                                  tqkv_stream stream) {
  if (!c || !q || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (c->cfg.kind == TQKV_CACHE_CODEBOOK || c->cfg.kind == TQKV_CACHE_BF16)
    return prefill_rows(c, q, H, L, scale, window, out, reinterpret_cast<hipStream_t>(stream));
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

int32_t tqkv_lkv_export(const tqkv_cache* const* layers, int32_t n_layers,
                        const tqkv_lkv_info* info, uint8_t* out, size_t capacity,
                        size_t* bytes, tqkv_stream stream) {
  if (!layers || !info || !bytes || n_layers < 0) return fail(TQKV_EINVAL_ARG, "null pointer");
  lkv::Manifest m;
  m.model_fingerprint = info->model_fingerprint ? info->model_fingerprint : "";
  m.created_at_unix = info->created_at_unix;
  m.position = info->position;
  if (info->n_prefix_tokens < 0 || (info->n_prefix_tokens > 0 && !info->prefix_tokens))
    return fail(TQKV_EINVAL_ARG, "prefix tokens");
  m.prefix_tokens.assign(info->prefix_tokens, info->prefix_tokens + info->n_prefix_tokens);
  if (info->has_last_token) m.last_token = lkv::Opt{true, info->last_token};
  m.is_deep = info->is_deep != 0;
  std::vector<LayerPlan> plans(static_cast<size_t>(n_layers));
  int64_t n_records = 0;
  for (int32_t i = 0; i < n_layers; ++i) {
    if (!layers[i]) return fail(TQKV_EINVAL_ARG, "layer %d is null", i);
    if (int32_t rc = plan_layer(layers[i], n_records, &plans[size_t(i)])) return rc;
    n_records += int64_t(plans[size_t(i)].recs.size());
    m.layers.push_back(plans[size_t(i)].meta);
  }
  if (n_records > 0xFFFFFFFFll) return fail(TQKV_EINVAL_SHAPE, "too many records");
  const std::string json = lkv::manifest_json(m);
  if (json.size() > 0xFFFFFFFFull) return fail(TQKV_EINVAL_SHAPE, "manifest too large");
  uint64_t total = lkv::header_size(json.size());
  for (const LayerPlan& p : plans)
    for (const RecSpec& r : p.recs) total += lkv::record_size(r.shape.size(), r.bytes());
  *bytes = size_t(total);
  if (!out) return ok();
  if (capacity < total)
    return fail(TQKV_EINVAL_ARG, "snapshot needs %llu bytes, %zu given", (unsigned long long)total,
                capacity);
  // The caches' pending updates (on `stream`) come first.
  TQKV_HIP(hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)));
  uint64_t at = lkv::write_header(out, json, uint32_t(n_records));
  for (int32_t i = 0; i < n_layers; ++i)
    for (const RecSpec& r : plans[size_t(i)].recs) {
      uint8_t* rec = out + at;
      const uint64_t h = lkv::write_record_header(rec, r.dtype, r.shape, r.bytes());
      if (int32_t rc = read_record(layers[i], r, rec + h)) return rc;
      lkv::finish_record(rec, h + r.bytes());
      at += lkv::record_size(r.shape.size(), r.bytes());
    }
  return ok();
}

int32_t tqkv_lkv_import(const uint8_t* data, size_t nbytes, int32_t layer, uint64_t seed,
                        tqkv_cache** out, tqkv_stream stream) {
  if (!data || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  *out = nullptr;
  lkv::Manifest m;
  std::vector<lkv::RecordView> recs;
  std::string err;
  if (!lkv::parse(data, nbytes, &m, &recs, &err)) return fail(TQKV_ECORRUPT, "kv_disk: %s", err.c_str());
  if (layer < 0 || size_t(layer) >= m.layers.size())
    return fail(TQKV_EINVAL_ARG, "layer %d of %zu", layer, m.layers.size());
  const lkv::Layer& L = m.layers[size_t(layer)];
  const std::string& k = L.kind;
  tqkv_cache_config g{};
  g.prealloc = 1;
  g.seed = seed;
  int n_arr = 0;
  bool ring = false;
  if (k == "Full" || k == "Sliding") {
    g.kind = TQKV_CACHE_BF16;
    n_arr = 2;
    ring = k == "Sliding";
  } else if (k == "FullQuantized" || k == "SlidingQuantized") {
    g.kind = TQKV_CACHE_AFFINE;
    n_arr = 6;
    ring = k == "SlidingQuantized";
  } else if (k == "FullTurboquant" || k == "SlidingTurboquant") {
    g.kind = TQKV_CACHE_CODEBOOK;
    n_arr = 6;
    ring = true;
  } else {
    return fail(TQKV_EUNSUPPORTED, "layer kind %s holds no attention cache", k.c_str());
  }
  auto bad = [&](const char* what) {
    return fail(TQKV_ECORRUPT, "kv_disk: %s layer %d: %s", k.c_str(), layer, what);
  };
  if (ring && (!L.max_size.has || !L.keep.has || !L.idx.has)) return bad("missing max_size, keep or idx");
  // Record of array slot i, or null.
  auto at = [&](int i) -> const lkv::RecordView* {
    if (size_t(i) >= L.arrays.size() || L.arrays[size_t(i)] < 0) return nullptr;
    const uint64_t id = uint64_t(L.arrays[size_t(i)]);
    return id < recs.size() ? &recs[size_t(id)] : nullptr;
  };
  for (int i = 0; i < n_arr && size_t(i) < L.arrays.size(); ++i)
    if (L.arrays[size_t(i)] >= 0 && uint64_t(L.arrays[size_t(i)]) >= recs.size())
      return bad("array index out of range");
  const lkv::RecordView* r0 = at(0);
  const bool has = r0 != nullptr;
  int64_t B = 0, H = 0, len = 0;
  auto geom = [&](const lkv::RecordView* r, uint8_t dtype, int64_t* last) {
    if (!r || r->dtype != dtype || r->shape.size() != 4) return false;
    if (B == 0 && H == 0) {
      B = r->shape[0];
      H = r->shape[1];
      len = r->shape[2];
    }
    if (r->shape[0] != B || r->shape[1] != H || r->shape[2] != len) return false;
    *last = r->shape[3];
    return true;
  };
  std::vector<RecSpec> specs;
  auto spec = [&](int slot, const lkv::RecordView* r, bool signs = false) {
    RecSpec s;
    s.slot = slot;
    s.dtype = r->dtype;
    s.shape = r->shape;
    s.rows = r->shape[2];
    s.signs = signs;
    specs.push_back(s);
  };
  if (has) {
    int64_t d0 = 0, d1 = 0, d2 = 0, d3 = 0, d4 = 0, d5 = 0;
    if (g.kind == TQKV_CACHE_BF16) {
      if (!geom(at(0), lkv::kBF16, &d0) || !geom(at(1), lkv::kBF16, &d1))
        return bad("keys/values must be bf16 [B, H_kv, S, D]");
      g.k_dim = int32_t(d0);
      g.v_dim = int32_t(d1);
      spec(0, at(0));
      spec(1, at(1));
    } else if (g.kind == TQKV_CACHE_AFFINE) {
      if (!L.has_group_size || !L.bits.has) return bad("missing group_size or bits");
      if (!geom(at(0), lkv::kU32, &d0) || !geom(at(1), lkv::kBF16, &d1) ||
          !geom(at(2), lkv::kBF16, &d2) || !geom(at(3), lkv::kU32, &d3) ||
          !geom(at(4), lkv::kBF16, &d4) || !geom(at(5), lkv::kBF16, &d5) || d1 != d2 || d4 != d5)
        return bad("(packed u32, scales bf16, biases bf16) x {K, V} of one [B, H_kv, S] shape expected");
      const int64_t gs = L.group_size;
      if (gs <= 0 || gs > 4096) return bad("group_size");
      g.group_size = int32_t(gs);
      g.k_dim = int32_t(d1 * gs);
      g.v_dim = int32_t(d4 * gs);
      g.bits_k = int32_t(L.bits.v);
      if (g.k_dim <= 0 || g.v_dim <= 0 || d0 * 32 != int64_t(g.k_dim) * g.bits_k || (d3 * 32) % g.v_dim)
        return bad("packed widths do not match group_size and bits");
      g.bits_v = int32_t(d3 * 32 / g.v_dim);
      for (int i = 0; i < 6; ++i) spec(i, at(i));
    } else {
      if (!L.bits.has) return bad("missing bits");
      if (!geom(at(0), lkv::kU8, &d0) || !geom(at(1), lkv::kF32, &d1) ||
          !geom(at(2), lkv::kU8, &d2) || !geom(at(3), lkv::kF32, &d3) || d1 != 1 || d3 != 1)
        return bad("codes u8 [B, H_kv, S, D] and sigma f32 [B, H_kv, S, 1] expected");
      g.k_dim = int32_t(d0);
      g.v_dim = int32_t(d2);
      g.bits_k = g.bits_v = int32_t(L.bits.v);
      const lkv::RecordView* sg = at(4);
      const lkv::RecordView* rn = at(5);
      if ((sg == nullptr) != (rn == nullptr)) return bad("QJL slots partially present");
      const int vs = sg ? 4 : 2;
      if (sg) {
        if (!L.qjl_m.has) return bad("missing qjl_m");
        if (!geom(sg, lkv::kBF16, &d4) || !geom(rn, lkv::kF32, &d5) || d5 != 1 ||
            uint64_t(d4) != L.qjl_m.v)
          return bad("keys_signs bf16 [B, H_kv, S, qjl_m] and residual norm f32 expected");
        if (d4 % 32 != 0)
          return fail(TQKV_EUNSUPPORTED, "qjl_m=%lld is not a multiple of 32", (long long)d4);
        g.qjl_words = int32_t(d4 / 32);
      }
      spec(0, at(0));
      spec(1, at(1));
      spec(vs, at(2));
      spec(vs + 1, at(3));
      if (sg) {
        spec(2, sg, true);
        spec(3, rn);
      }
    }
    if (B <= 0 || H <= 0 || B > 65535 || H > 65535) return bad("batch or heads out of range");
  } else {
    for (int i = 0; i < n_arr; ++i)
      if (at(i)) return bad("arrays partially present");
    return fail(TQKV_EUNSUPPORTED, "an empty layer carries no geometry to rebuild from");
  }
  g.batch = int32_t(B);
  g.kv_heads = int32_t(H);
  if (ring) {
    g.max_size = L.max_size.v > uint64_t(INT64_MAX) ? INT64_MAX : int64_t(L.max_size.v);
    g.keep = int64_t(L.keep.v);
  }
  if (L.offset < L.base_offset) return bad("offset below base_offset");
  tqkv_cache* c = nullptr;
  if (int32_t rc = tqkv_cache_create(&g, &c)) return rc;
  auto undo = [&](int32_t rc) {
    tqkv_cache_destroy(c);
    return rc;
  };
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  TQKV_HIP(hipStreamSynchronize(st));
  const int64_t cap = capacity_for(c, len > 0 ? len : 1, 0);
  for (int s = 0; s < c->n_slots; ++s)
    if (int32_t rc = alloc(c, c->cur[s], cap, s)) return undo(rc);
  // specs[i] was made from array slot i's record.
  for (size_t i = 0; i < specs.size(); ++i)
    if (int32_t rc = write_record(c, specs[i], at(int(i))->data)) return undo(rc);
  c->st.has = true;
  c->st.len = len;
  c->st.offset = int64_t(L.offset - L.base_offset);
  c->st.idx = ring ? int64_t(L.idx.v) : 0;
  c->base_offset = int64_t(L.base_offset);
  c->view_n = !ring ? c->st.offset : (c->st.offset >= g.max_size ? len : std::min(c->st.offset, len));
  if (g.kind == TQKV_CACHE_CODEBOOK)
    if (int32_t rc = codebook_tables(c, nullptr, nullptr)) return undo(rc);
  *out = c;
  return ok();
}

}  // extern "C"
