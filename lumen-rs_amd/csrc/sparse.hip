// Page-sparse decode, the digest and page-choice halves (the attention over
// the chosen pages is the paged decode kernel, decode_mfma.hpp).
//
// Page digest (PageDigest / page_digest, native_cache.rs:352-364, 407-445):
// the elementwise min and max over each full 64-token page of the keys. The
// keys of an affine cache are its mlx::dequantize'd rows, bf16(fma(scale,
// code, bias)) rounded once, so min and max are exact bf16 values. One workgroup per
// (slab, page), one thread per channel: the 64 rows' codes of a channel come
// from the same words for every thread of a group, so the reads coalesce.
//
// Page choice (sdpa_page_sparse, native_attention.rs:240-271): per (batch
// row, KV head), page p's bound is the max over the query group of
// sum_d max(q_d kmax_pd, q_d kmin_pd), summed in f32; the first page and the
// last four full pages are pinned (+inf); the keep largest bounds are chosen
// (ties to the lower page index, where the reference leaves the order of
// tied pages to its argpartition), and written in ascending page order. Two
// launches: the bounds, streamed from the digest by many workgroups (it is
// the larger read), into the workspace; then one workgroup per (batch row,
// KV head) turns them into 64-bit keys (bound descending, then page) in LDS,
// finds the keep smallest (by rank up to 1,024 pages, else a bitonic sort)
// and compacts them in page order.
#include <cmath>

#include "common.hpp"

namespace tqkv {
namespace sparse {
namespace {

constexpr int kPage = 64;
constexpr int kThreads = 256;
constexpr int kMaxPages = 4096;     // pages a (batch row, KV head) may digest
constexpr int kRankPages = 1024;    // the page choice ranks up to this many, else sorts

__device__ __forceinline__ uint32_t code_at(const uint32_t* row, int d, int bits) {
  const int bit = d * bits, w = bit / 32, sh = bit % 32;
  uint64_t x = row[w];
  if (sh + bits > 32) x |= uint64_t(row[w + 1]) << 32;
  return uint32_t(x >> sh) & ((1u << bits) - 1u);
}

__global__ __launch_bounds__(kThreads) void digest_kernel(
    const uint32_t* __restrict__ kw, const uint16_t* __restrict__ ks,
    const uint16_t* __restrict__ kb, int64_t cap, int D, int gs, int bits, int64_t page_from,
    uint16_t* __restrict__ kmin, uint16_t* __restrict__ kmax, int64_t max_pages) {
  const int64_t page = page_from + blockIdx.x, slab = blockIdx.y;
  const int words = D * bits / 32, groups = D / gs;
  for (int d = threadIdx.x; d < D; d += kThreads) {
    float mn = INFINITY, mx = -INFINITY;
    const int g = d / gs;
#pragma unroll 8
    for (int t = 0; t < kPage; ++t) {
      const int64_t r = slab * cap + page * kPage + t;
      const float s = bf16_to_f32(ks[r * groups + g]), b = bf16_to_f32(kb[r * groups + g]);
      const float c = float(code_at(kw + r * words, d, bits));
      const float v = bf16_to_f32(f32_to_bf16(fmaf(s, c, b)));
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
    const int64_t o = (slab * max_pages + page) * D + d;
    kmin[o] = f32_to_bf16(mn);
    kmax[o] = f32_to_bf16(mx);
  }
}

// Bounds of pages [blockIdx.x * kBoundPages, +kBoundPages) of one (batch
// row, KV head): each lane reads 8 channels (16 bytes) of a page's key_min
// and key_max rows, a page takes D / 8 lanes, and the group's partial sums
// meet in a butterfly. The pinned pages get +inf.
constexpr int kBoundPages = 64;

template <int D>
__global__ __launch_bounds__(kThreads) void bounds_kernel(
    const uint16_t* __restrict__ q, int H, int H_kv, int G, const uint16_t* __restrict__ kmin,
    const uint16_t* __restrict__ kmax, int64_t max_pages, int pages, float* __restrict__ bounds) {
  constexpr int LPP = D / 8;                  // lanes a page
  constexpr int PPP = kThreads / LPP;         // pages a pass
  const int unit = blockIdx.y, b = unit / H_kv, kvh = unit % H_kv;
  const int sub = threadIdx.x % LPP, slot = threadIdx.x / LPP;
  const uint16_t* qb = q + (int64_t(b) * H + int64_t(kvh) * G) * D + sub * 8;
  const uint16_t* mn0 = kmin + int64_t(unit) * max_pages * D + sub * 8;
  const uint16_t* mx0 = kmax + int64_t(unit) * max_pages * D + sub * 8;
  const int p_begin = blockIdx.x * kBoundPages;
  const int p_end = p_begin + kBoundPages < pages ? p_begin + kBoundPages : pages;
  for (int p0 = p_begin; p0 < p_end; p0 += 2 * PPP) {
    // Two pages a thread in flight.
    const int pa = p0 + slot, pb = p0 + PPP + slot;
    const bool va = pa < p_end, vb = pb < p_end;
    uint4 na{}, xa{}, nb{}, xb{};
    if (va) {
      na = *reinterpret_cast<const uint4*>(mn0 + int64_t(pa) * D);
      xa = *reinterpret_cast<const uint4*>(mx0 + int64_t(pa) * D);
    }
    if (vb) {
      nb = *reinterpret_cast<const uint4*>(mn0 + int64_t(pb) * D);
      xb = *reinterpret_cast<const uint4*>(mx0 + int64_t(pb) * D);
    }
    const uint32_t wna[4] = {na.x, na.y, na.z, na.w}, wxa[4] = {xa.x, xa.y, xa.z, xa.w};
    const uint32_t wnb[4] = {nb.x, nb.y, nb.z, nb.w}, wxb[4] = {xb.x, xb.y, xb.z, xb.w};
    float best_a = -INFINITY, best_b = -INFINITY;
    for (int g = 0; g < G; ++g) {
      const uint4 qw = *reinterpret_cast<const uint4*>(qb + int64_t(g) * D);
      const uint32_t wq[4] = {qw.x, qw.y, qw.z, qw.w};
      float sa = 0.0f, sb = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int w = e / 2, sh = (e % 2) * 16;
        const float qd = __uint_as_float(((wq[w] >> sh) & 0xffffu) << 16);
        const uint32_t ka = qd > 0.0f ? wxa[w] : wna[w], kb = qd > 0.0f ? wxb[w] : wnb[w];
        sa = fmaf(qd, __uint_as_float(((ka >> sh) & 0xffffu) << 16), sa);
        sb = fmaf(qd, __uint_as_float(((kb >> sh) & 0xffffu) << 16), sb);
      }
#pragma unroll
      for (int off = 1; off < LPP; off <<= 1) {
        sa += __shfl_xor(sa, off, 64);
        sb += __shfl_xor(sb, off, 64);
      }
      best_a = fmaxf(best_a, sa);
      best_b = fmaxf(best_b, sb);
    }
    if (sub == 0) {
      float* out = bounds + int64_t(unit) * pages;
      if (va) out[pa] = (pa < 1 || pa + 4 >= pages) ? INFINITY : best_a;
      if (vb) out[pb] = (pb < 1 || pb + 4 >= pages) ? INFINITY : best_b;
    }
  }
}

// f32 bits in an order that sorts like the values (finite or infinite).
__device__ __forceinline__ uint32_t ordered(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The keep largest bounds of one (batch row, KV head), ties to the lower
// page, written in ascending page order. 1,024 threads: the rank pass is
// P^2 compares of LDS-broadcast keys, and four wavefronts a SIMD hide the
// LDS latency.
constexpr int kSelThreads = 1024;
__global__ __launch_bounds__(kSelThreads) void select_kernel(const float* __restrict__ bounds,
                                                          int pages, int keep,
                                                          int32_t* __restrict__ chosen) {
  __shared__ uint64_t key[kMaxPages];
  __shared__ int flag[kMaxPages];
  __shared__ int cnt[kSelThreads / 64];
  const int unit = blockIdx.x, tid = threadIdx.x;
  const float* bd = bounds + int64_t(unit) * pages;
  int n2 = 1;
  while (n2 < pages) n2 <<= 1;
  for (int i = tid; i < n2; i += kSelThreads) {
    key[i] = i < pages ? (uint64_t(~ordered(bd[i])) << 32) | uint32_t(i) : ~0ull;
    if (i < pages) flag[i] = 0;
  }
  __syncthreads();
  if (pages <= kRankPages) {
    // Up to 1,024 pages: each key's rank is the count of smaller keys (keys
    // are distinct), read from LDS by every thread in the same order (a
    // broadcast); the chosen are the ranks below keep. (One 64-bit compare
    // and add a pair: cheaper in VALU issue than 32-bit keys with an index
    // tie-break or register broadcasts, both measured slower.)
    for (int i = tid; i < pages; i += kSelThreads) {
      const uint64_t mine = key[i];
      int rank = 0;
      for (int j = 0; j < pages; ++j) rank += key[j] < mine;
      flag[i] = rank < keep;
    }
    __syncthreads();
  } else {
    // Bitonic sort, ascending: bound descending, then page ascending.
    for (int k = 2; k <= n2; k <<= 1)
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < n2; i += kSelThreads) {
          const int l = i ^ j;
          if (l > i) {
            const uint64_t x = key[i], y = key[l];
            const bool up = (i & k) == 0;
            if ((x > y) == up) {
              key[i] = y;
              key[l] = x;
            }
          }
        }
        __syncthreads();
      }
    for (int i = tid; i < keep; i += kSelThreads) flag[int(uint32_t(key[i]))] = 1;
    __syncthreads();
  }
  // Compaction in page order: thread t takes a contiguous block of pages;
  // an exclusive scan of the block counts (within each wavefront by
  // shuffles, then over the wavefronts' totals) gives its first slot.
  const int per = (pages + kSelThreads - 1) / kSelThreads;
  const int p0 = tid * per, p1 = p0 + per < pages ? p0 + per : pages;
  int c = 0;
  for (int p = p0; p < p1; ++p) c += flag[p];
  const int lane = tid % 64, wave = tid / 64;
  int incl = c;
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (lane == 63) cnt[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += cnt[w];
  int at = base + incl - c;
  int32_t* out = chosen + int64_t(unit) * keep;
  for (int p = p0; p < p1; ++p)
    if (flag[p]) out[at++] = p;
}

}  // namespace
}  // namespace sparse
}  // namespace tqkv

using namespace tqkv;
using namespace tqkv::sparse;

extern "C" int64_t tqkv_sparse_keep_pages(int64_t pages) {
  return pages / 8 > 64 ? pages / 8 : 64;
}

extern "C" int32_t tqkv_page_digest_affine(const uint32_t* k_packed, const uint16_t* k_scales,
                                           const uint16_t* k_biases, int64_t n_slabs, int64_t cap,
                                           int32_t dim, int32_t group_size, int32_t bits,
                                           int64_t page_from, int64_t page_to, uint16_t* key_min,
                                           uint16_t* key_max, int64_t max_pages,
                                           tqkv_stream stream) {
  if (!(bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8))
    return fail(TQKV_EUNSUPPORTED, "bits=%d", bits);
  if (!(group_size == 32 || group_size == 64 || group_size == 128) || dim % group_size != 0 ||
      dim <= 0 || dim > 1024 || (dim * bits) % 32 != 0)
    return fail(TQKV_EUNSUPPORTED, "dim=%d group_size=%d bits=%d", dim, group_size, bits);
  if (n_slabs < 0 || page_from < 0 || page_to < page_from || page_to > max_pages ||
      page_to * kPage > cap || n_slabs > 65535)
    return fail(TQKV_EINVAL_SHAPE, "pages [%lld, %lld) of %lld (cap %lld rows, %lld slabs)",
                (long long)page_from, (long long)page_to, (long long)max_pages, (long long)cap,
                (long long)n_slabs);
  if (n_slabs == 0 || page_to == page_from) return ok();
  if (!k_packed || !k_scales || !k_biases || !key_min || !key_max)
    return fail(TQKV_EINVAL_ARG, "null pointer");
  if (page_to - page_from > 0x7fffffffLL) return fail(TQKV_EINVAL_SHAPE, "too many pages");
  hipLaunchKernelGGL(digest_kernel, dim3(unsigned(page_to - page_from), unsigned(n_slabs)),
                     dim3(kThreads), 0, reinterpret_cast<hipStream_t>(stream), k_packed, k_scales,
                     k_biases, cap, dim, group_size, bits, page_from, key_min, key_max, max_pages);
  TQKV_LAUNCHED();
  return ok();
}

extern "C" size_t tqkv_page_select_workspace_size(int32_t B, int32_t H_kv, int64_t pages) {
  if (B <= 0 || H_kv <= 0 || pages <= 0) return 0;
  return (size_t(B) * H_kv * size_t(pages) * sizeof(float) + 255) / 256 * 256;
}

extern "C" int32_t tqkv_page_select(const uint16_t* q, int32_t B, int32_t H, int32_t H_kv,
                                    int32_t D, const uint16_t* key_min, const uint16_t* key_max,
                                    int64_t max_pages, int64_t pages, int32_t keep,
                                    int32_t* chosen, void* workspace, size_t workspace_bytes,
                                    tqkv_stream stream) {
  if (!q || !key_min || !key_max || !chosen) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv != 0 || !(D == 64 || D == 128 || D == 256 ||
                                                             D == 512))
    return fail(TQKV_EINVAL_SHAPE, "B=%d H=%d H_kv=%d D=%d", B, H, H_kv, D);
  if (pages < 1 || pages > max_pages || pages > kMaxPages)
    return fail(TQKV_EINVAL_SHAPE, "pages=%lld (max %lld, at most %d)", (long long)pages,
                (long long)max_pages, kMaxPages);
  if (keep < 1 || keep > pages)
    return fail(TQKV_EINVAL_SHAPE, "keep=%d of %lld pages", keep, (long long)pages);
  const int64_t units = int64_t(B) * H_kv;
  if (units > 65535) return fail(TQKV_EINVAL_SHAPE, "%lld (batch row, KV head) units", (long long)units);
  const size_t need = tqkv_page_select_workspace_size(B, H_kv, pages);
  if (!workspace || workspace_bytes < need)
    return fail(TQKV_EINVAL_ARG, "workspace of %zu bytes, need %zu", workspace_bytes, need);
  float* bounds = static_cast<float*>(workspace);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(unsigned((pages + kBoundPages - 1) / kBoundPages), unsigned(units));
  const int G = H / H_kv;
  switch (D) {
    case 64: hipLaunchKernelGGL(bounds_kernel<64>, grid, dim3(kThreads), 0, st, q, H, H_kv, G, key_min, key_max, max_pages, int(pages), bounds); break;
    case 128: hipLaunchKernelGGL(bounds_kernel<128>, grid, dim3(kThreads), 0, st, q, H, H_kv, G, key_min, key_max, max_pages, int(pages), bounds); break;
    case 256: hipLaunchKernelGGL(bounds_kernel<256>, grid, dim3(kThreads), 0, st, q, H, H_kv, G, key_min, key_max, max_pages, int(pages), bounds); break;
    default: hipLaunchKernelGGL(bounds_kernel<512>, grid, dim3(kThreads), 0, st, q, H, H_kv, G, key_min, key_max, max_pages, int(pages), bounds); break;
  }
  TQKV_LAUNCHED();
  hipLaunchKernelGGL(select_kernel, dim3(unsigned(units)), dim3(kSelThreads), 0, st, bounds,
                     int(pages), keep, chosen);
  TQKV_LAUNCHED();
  return ok();
}
