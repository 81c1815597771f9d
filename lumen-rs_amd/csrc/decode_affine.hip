// Host side of the fused affine decode: split planning, workspace, dispatch.
// The kernel itself (and its design notes) is in decode_affine.hpp.
#include <cstdlib>
#include <cstring>

#include "decode_mfma.hpp"

namespace tqkv {
namespace prefill {
int32_t shared_prefix_partials(const uint16_t* q, int B, int H, int H_kv, int D, int gs, int bk,
                               int bv, float scale, const tqkv_affine_seg& prefix, int n_splits,
                               int split_len, int n_part, float* part_o, float* part_m,
                               float* part_l, hipStream_t st);
int shared_prefix_block_rows(int D);
bool tile_decode_supported(int D, int bk, int bv);
int tile_decode_rows();
int32_t tile_decode(const uint16_t* q, int B, int H, int H_kv, int D, int gs, int bk, int bv,
                    float scale, const tqkv_affine_seg* segs, int n_segs, int n_splits,
                    int split_len, int n_part, float* part_o, float* part_m, float* part_l,
                    uint16_t* out, hipStream_t st);
}  // namespace prefill
namespace decode {
namespace {

// Merges the splits of one (batch row, query head):
// out = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), as bf16. Each split's
// weight 2^(m_s - M) is computed once (into LDS), then every thread sums
// its channel over the splits with coalesced reads of the partials.
constexpr int kMergeThreads = 256;
constexpr int kMergeChunk = 1024;

__device__ __forceinline__ float block_max(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  const int w = threadIdx.x / 64;
  __syncthreads();
  if (threadIdx.x % 64 == 0) red[w] = v;
  __syncthreads();
  v = red[0];
  for (int i = 1; i < kMergeThreads / 64; ++i) v = fmaxf(v, red[i]);
  return v;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  const int w = threadIdx.x / 64;
  __syncthreads();
  if (threadIdx.x % 64 == 0) red[w] = v;
  __syncthreads();
  v = red[0];
  for (int i = 1; i < kMergeThreads / 64; ++i) v += red[i];
  return v;
}

__global__ __launch_bounds__(kMergeThreads) void decode_merge_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_m,
    const float* __restrict__ part_l, int n_splits, int D, uint16_t* __restrict__ out) {
  __shared__ float wgt[kMergeChunk];
  __shared__ float red[kMergeThreads / 64];
  const int64_t bh = blockIdx.x;
  const float* pm = part_m + bh * n_splits;
  const float* pl = part_l + bh * n_splits;
  float mx = -INFINITY;
  for (int s = threadIdx.x; s < n_splits; s += kMergeThreads) mx = fmaxf(mx, pm[s]);
  mx = block_max(mx, red);
  float ls = 0.0f;
  float os[2] = {0.0f, 0.0f};  // channels threadIdx.x and + 256 (D <= 512)
  for (int c0 = 0; c0 < n_splits; c0 += kMergeChunk) {
    const int n = n_splits - c0 < kMergeChunk ? n_splits - c0 : kMergeChunk;
    __syncthreads();  // the previous chunk's weights are used up
    for (int s = threadIdx.x; s < n; s += kMergeThreads) {
      const float m = pm[c0 + s];
      const float w = m == -INFINITY ? 0.0f : exp2f(m - mx);
      wgt[s] = w;
      ls += w * pl[c0 + s];
    }
    __syncthreads();
    for (int k = 0; k < 2; ++k) {
      const int d = threadIdx.x + k * kMergeThreads;
      if (d >= D) break;
      const float* po = part_o + (bh * n_splits + c0) * D + d;
      float acc = os[k];
      // Sixteen slots' loads issued before any is used (a load a slot in
      // turn paid the L2 round trip per slot: 5.4 us for 36 slots).
      int s = 0;
      for (; s + 16 <= n; s += 16) {
        float x[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) x[u] = po[int64_t(s + u) * D];
#pragma unroll
        for (int u = 0; u < 16; ++u) acc += wgt[s + u] * x[u];
      }
      for (; s + 4 <= n; s += 4) {
        float x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = po[int64_t(s + u) * D];
#pragma unroll
        for (int u = 0; u < 4; ++u) acc += wgt[s + u] * x[u];
      }
      for (; s < n; ++s) acc += wgt[s] * po[int64_t(s) * D];
      os[k] = acc;
    }
  }
  ls = block_sum(ls, red);
  for (int k = 0; k < 2; ++k) {
    const int d = threadIdx.x + k * kMergeThreads;
    if (d < D) out[bh * D + d] = f32_to_bf16(ls > 0.0f ? os[k] / ls : 0.0f);
  }
}

// The merge for at most NMAX splits (4, 8, 16 or 32), in one round of
// loads: every thread loads all the splits' (m, l) (the same addresses
// across the block, served by the caches) and its two channels' partial
// outputs, then combines them in registers: no LDS, no barrier, no second
// trip to memory.
constexpr int kMergeSmall = 32;

template <int NMAX>
__global__ __launch_bounds__(kMergeThreads) void decode_merge_small_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_m,
    const float* __restrict__ part_l, int n_splits, int D, uint16_t* __restrict__ out) {
  const int64_t bh = blockIdx.x;
  const float* pm = part_m + bh * n_splits;
  const float* pl = part_l + bh * n_splits;
  const float* po = part_o + bh * n_splits * D;
  const int d0 = threadIdx.x, d1 = threadIdx.x + kMergeThreads;
  const bool has0 = d0 < D, has1 = d1 < D;
  float m[NMAX], l[NMAX], o0[NMAX], o1[NMAX];
#pragma unroll
  for (int s = 0; s < NMAX; ++s) {
    const bool live = s < n_splits;
    m[s] = live ? pm[s] : -INFINITY;
    l[s] = live ? pl[s] : 0.0f;
    o0[s] = live && has0 ? po[int64_t(s) * D + d0] : 0.0f;
    o1[s] = live && has1 ? po[int64_t(s) * D + d1] : 0.0f;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int s = 0; s < NMAX; ++s) mx = fmaxf(mx, m[s]);
  float ls = 0.0f, os0 = 0.0f, os1 = 0.0f;
#pragma unroll
  for (int s = 0; s < NMAX; ++s) {
    const float w = m[s] == -INFINITY ? 0.0f : exp2f(m[s] - mx);
    ls += w * l[s];
    os0 += w * o0[s];
    os1 += w * o1[s];
  }
  if (has0) out[bh * D + d0] = f32_to_bf16(ls > 0.0f ? os0 / ls : 0.0f);
  if (has1) out[bh * D + d1] = f32_to_bf16(ls > 0.0f ? os1 / ls : 0.0f);
}

// The merge launch for n_splits partial slots of every (batch row, head).
void launch_merge(const float* po, const float* pm, const float* pl, int n_splits, int D,
                  int64_t rows, uint16_t* out, hipStream_t st) {
  auto small = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(unsigned(rows)), dim3(kMergeThreads), 0, st, po, pm, pl,
                       n_splits, D, out);
  };
  if (n_splits <= 4)
    small(decode_merge_small_kernel<4>);
  else if (n_splits <= 8)
    small(decode_merge_small_kernel<8>);
  else if (n_splits <= 16)
    small(decode_merge_small_kernel<16>);
  else if (n_splits <= kMergeSmall)
    small(decode_merge_small_kernel<kMergeSmall>);
  else
    hipLaunchKernelGGL(decode_merge_kernel, dim3(unsigned(rows)), dim3(kMergeThreads), 0, st, po,
                       pm, pl, n_splits, D, out);
}

// Splits per (batch row, KV head). With at least ~2048 wavefronts of whole
// (batch row, KV head) units the chip is full and each workgroup owns its
// keys (one launch); otherwise the keys are split until the grid holds ~2048
// wavefronts, never below kMinSplitKeys keys per split. TQKV_DECODE_SPLITS=k
// caps the count (tests reach the one-split and the merging paths with it).
// A 1,024-key ring at B = 4 x 8 KV heads (config 3's sliding layers) takes 8
// splits of 128 keys, one 16-key step a wavefront: 0.443 ms a 30-layer step
// against 0.474 with a 256-key floor (4 splits) and 0.526 with 512.
constexpr int64_t kMinSplitKeys = 128;

int wanted_splits(int B, int H_kv, int waves, int64_t total) {
  const int64_t units = int64_t(B) * H_kv;
  const int64_t target_wgs = 2048 / waves;
  int64_t want = units >= target_wgs ? 1 : (target_wgs + units - 1) / units;
  const int64_t most = (total + kMinSplitKeys - 1) / kMinSplitKeys;
  if (want > most) want = most;
  if (const char* env = getenv("TQKV_DECODE_SPLITS")) {
    const long k = strtol(env, nullptr, 10);
    if (k >= 1 && k < want) want = k;
  }
  return want < 1 ? 1 : int(want);
}

void plan_splits(int B, int H_kv, int waves, int64_t total, int* n_splits, int64_t* split_len) {
  const int want = wanted_splits(B, H_kv, waves, total);
  int64_t len = (total + want - 1) / want;
  len = (len + 63) / 64 * 64;
  if (len < 64) len = 64;
  *split_len = len;
  *n_splits = int((total + len - 1) / len);
  if (*n_splits < 1) *n_splits = 1;
}

// An upper bound on the split count for any context up to `total` keys and
// any wavefront count, so a workspace sized for a capacity serves every
// shorter context.
int max_splits(int B, int H_kv, int64_t total) {
  const int64_t units = int64_t(B) * H_kv;
  int64_t want = (512 + units - 1) / units;
  const int64_t most = (total + kMinSplitKeys - 1) / kMinSplitKeys;
  if (want > most) want = most;
  return want < 1 ? 1 : int(want);
}

// Workgroups of the shared-prefix pass: one per CU of an MI355X (256). The
// pass holds one workgroup per CU, and each workgroup's fixed costs (query
// load, first tile, partials) favour one long key range per CU over several
// short ones (measured: 54 us at 256 against 57, 70, 74 and 102 us at 512,
// 192, 384 and 1,024 on config 4's 65,536-token prefix).
constexpr int kPrefixWgs = 256;

// Prefix splits of the shared-prefix path: about kPrefixWgs workgroups over
// the (KV head, row block) units, never under 256 keys a split.
int prefix_splits(int H_kv, int64_t rows, int block_rows, int64_t P, int* split_len) {
  const int64_t units = int64_t(H_kv) * ((rows + block_rows - 1) / block_rows);
  int64_t want = (kPrefixWgs + units - 1) / units;
  const int64_t most = (P + 255) / 256;
  if (want > most) want = most;
  if (want < 1) want = 1;
  int64_t len = (P + want - 1) / want;
  len = (len + 63) / 64 * 64;
  *split_len = int(len);
  return int((P + len - 1) / len);
}

int prefix_splits_max(int H_kv, int64_t total) {
  int64_t want = (kPrefixWgs + H_kv - 1) / H_kv;
  const int64_t most = (total + 255) / 256;
  if (want > most) want = most;
  return want < 1 ? 1 : int(want);
}

// The MFMA-scored kernel where its layout applies, else the dot2 kernel.
// TQKV_DECODE_KERNEL=dot2 forces the dot2 kernel (tests cover both).
// max_rows: the longest segment; the MFMA kernel addresses a segment's rows
// of one (batch row, KV head) through 32-bit buffer offsets.
KernelFn pick(int D, int bk, int bv, int G, int gs, int64_t max_rows = 0) {
  const char* env = getenv("TQKV_DECODE_KERNEL");
  const bool dot2_only = (env && strcmp(env, "dot2") == 0) || max_rows * D >= (int64_t(1) << 31);
  if (!dot2_only) {
    KernelFn f = nullptr;
    switch (D) {
      case 64: f = pick_mfma_d64(bk, bv, G, gs); break;
      case 128: f = pick_mfma_d128(bk, bv, G, gs); break;
      case 256: f = pick_mfma_d256(bk, bv, G, gs); break;
    }
    if (f) return f;
  }
  switch (D) {
    case 64: return pick_d64(bk, bv, G);
    case 128: return pick_d128(bk, bv, G);
    case 256: return pick_d256(bk, bv, G);
    case 512: return pick_d512(bk, bv, G);
  }
  return nullptr;
}

// The MFMA kernel for a layout (nullptr where none applies).
KernelFn pick_mfma_only(int D, int bk, int bv, int G, int gs) {
  switch (D) {
    case 64: return pick_mfma_d64(bk, bv, G, gs);
    case 128: return pick_mfma_d128(bk, bv, G, gs);
    case 256: return pick_mfma_d256(bk, bv, G, gs);
  }
  return nullptr;
}

// The heads a KV head that one kernel instantiation is picked for: G where
// a kernel takes G heads, else (G up to 32, the reference's limit,
// native_quant_attention.rs:253) the largest divisor of G a kernel takes,
// run as G / divisor launches that each read the keys once (Gemma 4's
// full-attention layers: 16 heads a KV head). 0 when none applies.
int group_heads(int D, int bk, int bv, int G, int gs, int64_t max_rows = 0) {
  KernelFn whole = pick(D, bk, bv, G, gs, max_rows);
  // Where only the dot2 kernel takes the whole group, two MFMA launches of
  // half the heads (each reading the keys) beat it: 8 heads at D = 256,
  // 4-bit, 8,192 keys: 2 x 50.7 against 222 us.
  if (whole && whole != pick_mfma_only(D, bk, bv, G, gs) && G % 2 == 0 &&
      pick(D, bk, bv, G / 2, gs, max_rows) == pick_mfma_only(D, bk, bv, G / 2, gs) &&
      pick_mfma_only(D, bk, bv, G / 2, gs))
    return G / 2;
  if (whole) return G;
  if (G > 32) return 0;
  for (int d : {8, 6, 4, 3, 2, 1})
    if (d < G && G % d == 0 && pick(D, bk, bv, d, gs, max_rows)) return d;
  return 0;
}

// Head dim 512 decodes through the tile kernel (the prefill kernel's f16
// variant, a sequence's heads as the rows of a block): its scores and
// values run on the matrix cores, where the dot2 kernel spends a 64-lane
// reduction per token and head at that width (measured 3-9x slower). No
// fused append there (that needs the MFMA decode kernel), and
// TQKV_DECODE_KERNEL=dot2 keeps the dot2 kernel.
bool use_tile(int D, int bk, int bv, int G, bool app) {
  const char* env = getenv("TQKV_DECODE_KERNEL");
  if (env && strcmp(env, "dot2") == 0) return false;
  return D == 512 && !app && G <= 32 && prefill::tile_decode_supported(D, bk, bv);
}

// Query heads one launch serves: the group's G, or G / 2 where the dot2
// kernel takes the group in two launches (split_heads).
int kernel_heads(int D, int bk, int bv, int G, int gs, int64_t max_rows) {
  KernelFn fn = pick(D, bk, bv, G, gs, max_rows);
  if (!fn || fn == pick_mfma_only(D, bk, bv, G, gs)) return G;
  return split_heads_rt(bk, bv, G) ? G / 2 : G;
}

}  // namespace
}  // namespace decode
}  // namespace tqkv

using namespace tqkv;
using namespace tqkv::decode;

extern "C" const char* tqkv_decode_kernel_for_rows(int32_t H, int32_t H_kv, int32_t D,
                                                   int32_t group_size, int32_t bits_k,
                                                   int32_t bits_v, int64_t max_rows) {
  if (H <= 0 || H_kv <= 0 || H % H_kv != 0 || max_rows < 0) return "";
  if (use_tile(D, bits_k, bits_v, H / H_kv, false)) return "tiles";
  const int Gp = group_heads(D, bits_k, bits_v, H / H_kv, group_size, max_rows);
  if (!Gp) return "";
  KernelFn fn = pick(D, bits_k, bits_v, Gp, group_size, max_rows);
  return fn == pick_mfma_only(D, bits_k, bits_v, Gp, group_size) ? "mfma" : "dot2";
}

extern "C" const char* tqkv_decode_kernel_name(int32_t H, int32_t H_kv, int32_t D,
                                               int32_t group_size, int32_t bits_k,
                                               int32_t bits_v) {
  return tqkv_decode_kernel_for_rows(H, H_kv, D, group_size, bits_k, bits_v, 0);
}

extern "C" size_t tqkv_decode_workspace_size(int32_t B, int32_t H, int32_t H_kv, int32_t D,
                                             int64_t total_tokens) {
  if (B <= 0 || H <= 0 || H_kv <= 0 || D <= 0 || total_tokens <= 0) return 0;
  // Enough for either path: per-sequence splits, or prefix splits plus the
  // suffix's splits.
  const size_t ns = size_t(max_splits(B, H_kv, total_tokens)) +
                    size_t(prefix_splits_max(H_kv, total_tokens));
  return size_t(B) * H * ns * (size_t(D) + 2) * sizeof(float);
}

namespace {

// The cache rows a fused append writes (tqkv_decode_attend_affine_append).
struct AppendDst {
  const uint16_t* k;
  const uint16_t* v;
  uint32_t* kw;
  uint16_t* ks;
  uint16_t* kb;
  uint32_t* vw;
  uint16_t* vs;
  uint16_t* vb;
  int64_t cap, row;
};

// How a decode call splits its keys, and the workspace bytes that needs (0:
// none). Only the segments' lengths and shared flags matter.
struct DecodePlan {
  bool tile = false;  // the tile kernel (use_tile), splits as below
  bool shared_path = false;
  // Shared prefix read once: prefix splits, then the suffix's.
  int sp_p = 0, split_len_p = 0, sp_s = 0;
  int64_t split_len_s = 0;
  // Per-sequence: splits of the whole context.
  int n_splits = 1;
  int64_t split_len = 0;
  int n_part = 1;
  size_t need = 0;
};

// Gk: the query heads one decode launch serves (kernel_heads).
// waves: the launch's wavefronts a workgroup (decode_waves); tile: the
// tile kernel decodes (use_tile).
DecodePlan plan_decode(int B, int H, int H_kv, int D, int Gk, int waves,
                       const tqkv_affine_seg* segs, int n_segs, bool app, bool tile = false) {
  DecodePlan pl;
  const int G = H / H_kv;
  const int64_t total = segs[0].n + (n_segs == 2 ? segs[1].n : 0);
  // A prefix shared by B >= 2 sequences: read it once per KV head for all of
  // them (the prefill kernel with the sequences as query rows, split over
  // the prefix, into partials), each sequence's own suffix with the decode
  // kernel into further partial slots, then one merge. TQKV_SHARED_PREFIX=0
  // reads the prefix per sequence instead (tests compare the two).
  const char* sp_env = getenv("TQKV_SHARED_PREFIX");
  pl.shared_path = n_segs == 2 && segs[0].shared && B >= 2 && segs[0].n > 0 &&
                   (D == 64 || D == 128 || D == 256) && !(sp_env && strcmp(sp_env, "0") == 0);
  const size_t row = size_t(D) + 2;
  if (pl.shared_path) {
    pl.sp_p = prefix_splits(H_kv, int64_t(B) * G, prefill::shared_prefix_block_rows(D),
                            segs[0].n, &pl.split_len_p);
    const int64_t S = segs[1].n;
    if (S > 0) plan_splits(B, H_kv, waves, S, &pl.sp_s, &pl.split_len_s);
    if (app && pl.sp_s == 0) {  // the new row needs a suffix launch
      pl.sp_s = 1;
      pl.split_len_s = 64;
    }
    pl.n_part = pl.sp_p + pl.sp_s;
    pl.need = size_t(B) * H * pl.n_part * row * sizeof(float);
    return pl;
  }
  if (tile) {
    // About 256 workgroups (one a CU: the tile kernel's LDS holds one),
    // never under 256 keys a split.
    const int rows = prefill::tile_decode_rows();
    const int64_t units = int64_t(B) * H_kv * ((G + rows - 1) / rows);
    int64_t want = (256 + units - 1) / units;
    const int64_t most = (total + 255) / 256;
    if (want > most) want = most;
    if (want < 1) want = 1;
    int64_t len = (total + want - 1) / want;
    len = (len + 63) / 64 * 64;
    pl.tile = true;
    pl.split_len = len;
    pl.n_splits = int((total + len - 1) / len);
    pl.n_part = pl.n_splits;
    pl.need = pl.n_splits > 1 ? size_t(B) * H * pl.n_splits * row * sizeof(float) : 0;
    return pl;
  }
  plan_splits(B, H_kv, waves, total, &pl.n_splits, &pl.split_len);
  pl.n_part = pl.n_splits;
  pl.need = pl.n_splits > 1 ? size_t(B) * H * pl.n_splits * row * sizeof(float) : 0;
  return pl;
}

int32_t decode_affine(const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t D,
                      int32_t group_size, int32_t bits_k, int32_t bits_v, float scale,
                      const tqkv_affine_seg* segs, int32_t n_segs, const AppendDst* app,
                      uint16_t* out, void* workspace, size_t workspace_bytes,
                      tqkv_stream stream) {
  if (!q || !out || !segs) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv != 0)
    return fail(TQKV_EINVAL_SHAPE, "B=%d H=%d H_kv=%d", B, H, H_kv);
  if (n_segs < 1 || n_segs > 2) return fail(TQKV_EINVAL_ARG, "n_segs=%d", n_segs);
  if (!(group_size == 32 || group_size == 64 || group_size == 128) || D % group_size != 0)
    return fail(TQKV_EUNSUPPORTED, "group_size=%d with D=%d", group_size, D);
  const int G = H / H_kv;
  int64_t max_rows = 0;
  for (int i = 0; i < n_segs; ++i) max_rows = segs[i].n > max_rows ? segs[i].n : max_rows;
  // Gp: the heads the kernel is picked for (G, or a divisor of G whose
  // launches cover the group).
  const int Gp = group_heads(D, bits_k, bits_v, G, group_size, max_rows);
  KernelFn fn = Gp ? pick(D, bits_k, bits_v, Gp, group_size, max_rows) : nullptr;
  const bool tile = use_tile(D, bits_k, bits_v, G, app != nullptr);
  if (!fn && !tile)
    return fail(TQKV_EUNSUPPORTED, "decode layout D=%d bits_k=%d bits_v=%d gqa=%d", D, bits_k,
                bits_v, G);
  const bool mfma = fn && fn == pick_mfma_only(D, bits_k, bits_v, Gp, group_size);
  const int epl = epl_rt(bits_k, bits_v, Gp);
  if (!tile && !mfma && group_size < epl)
    return fail(TQKV_EUNSUPPORTED, "group_size=%d below %d", group_size, epl);
  // Heads a launch: Gp, or half of it where the dot2 kernel takes 6 or 8
  // heads of 2/3/5/6-bit caches as two launches (each launch reads the keys).
  const int Gk = Gp ? kernel_heads(D, bits_k, bits_v, Gp, group_size, max_rows) : G;

  Args a{};
  a.q = q;
  a.H = H;
  a.H_kv = H_kv;
  a.Gt = G;
  a.h_off = 0;
  a.gs = group_size;
  a.qscale = scale * kLog2e;
  for (int i = 0; i < n_segs; ++i) {
    const tqkv_affine_seg& s = segs[i];
    if (s.n < 0 || s.n > s.cap) return fail(TQKV_EINVAL_SHAPE, "segment %d: n=%lld cap=%lld", i,
                                            (long long)s.n, (long long)s.cap);
    if (s.n > 0 && (!s.k_packed || !s.k_scales || !s.k_biases || !s.v_packed || !s.v_scales ||
                    !s.v_biases))
      return fail(TQKV_EINVAL_ARG, "segment %d has a null buffer", i);
    a.seg[i] = Seg{s.k_packed, s.k_scales, s.k_biases, s.v_packed, s.v_scales, s.v_biases,
                   s.cap, s.n, s.shared ? 0 : int64_t(H_kv) * s.cap};
  }
  if (n_segs == 1) a.seg[1] = a.seg[0];
  a.n0 = segs[0].n;
  a.total = segs[0].n + (n_segs == 2 ? segs[1].n : 0);
  if (app) {
    // Only the MFMA kernels quantize in place.
    if (!mfma)
      return fail(TQKV_EUNSUPPORTED, "fused append needs the MFMA decode kernel (D=%d bits %d/%d "
                  "gqa=%d gs=%d)", D, bits_k, bits_v, G, group_size);
    if (app->row < 0 || app->row >= app->cap)
      return fail(TQKV_EINVAL_SHAPE, "append row %lld of %lld", (long long)app->row,
                  (long long)app->cap);
    a.app_k = app->k;
    a.app_v = app->v;
    a.app_kw = app->kw;
    a.app_ks = app->ks;
    a.app_kb = app->kb;
    a.app_vw = app->vw;
    a.app_vs = app->vs;
    a.app_vb = app->vb;
    a.app_cap = app->cap;
    a.app_row = app->row;
  } else if (a.total <= 0) {
    return fail(TQKV_EINVAL_SHAPE, "no keys to attend");
  }

  const int waves = decode_waves(D, bits_k, bits_v, Gk, group_size, mfma);
  a.out = out;
  const DecodePlan pl = plan_decode(B, H, H_kv, D, Gk, waves, segs, n_segs, app != nullptr, tile);
  void* ws = workspace;
  if (pl.need > 0) {
    if (!ws) {
      if (int32_t rc = scratch_for_current_device(pl.need, &ws)) return rc;
    } else if (workspace_bytes < pl.need) {
      return fail(TQKV_EINVAL_ARG, "workspace of %zu bytes, need %zu", workspace_bytes, pl.need);
    }
  }
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);

  if (pl.tile) {
    float* po = static_cast<float*>(ws);
    float* pm = po ? po + size_t(B) * H * pl.n_part * D : nullptr;
    float* pl_ = pm ? pm + size_t(B) * H * pl.n_part : nullptr;
    if (int32_t rc = prefill::tile_decode(q, B, H, H_kv, D, group_size, bits_k, bits_v, scale,
                                          segs, n_segs, pl.n_splits, int(pl.split_len),
                                          pl.n_part, po, pm, pl_, out, st))
      return rc;
    if (pl.n_splits > 1) {
      launch_merge(po, pm, pl_, pl.n_part, D, int64_t(B) * H, out, st);
      TQKV_LAUNCHED();
    }
    return ok();
  }
  if (pl.shared_path) {
    Args s = a;
    s.seg[0] = a.seg[1];
    s.n0 = segs[1].n;
    s.total = segs[1].n;
    s.split_len = pl.split_len_s;
    float* po = static_cast<float*>(ws);
    float* pm = po + size_t(B) * H * pl.n_part * D;
    float* pl_ = pm + size_t(B) * H * pl.n_part;
    if (int32_t rc = prefill::shared_prefix_partials(q, B, H, H_kv, D, group_size, bits_k, bits_v,
                                                     scale, segs[0], pl.sp_p, pl.split_len_p,
                                                     pl.n_part, po, pm, pl_, st))
      return rc;
    if (pl.sp_s > 0) {
      // The suffix kernel is the one the whole call picked (its longest
      // segment decides between the MFMA and dot2 kernels).
      s.n_splits = pl.sp_s;
      s.split_base = pl.sp_p;
      s.n_part = pl.n_part;
      s.part_o = po;
      s.part_m = pm;
      s.part_l = pl_;
      for (s.h_off = 0; s.h_off < G; s.h_off += Gk) {
        hipLaunchKernelGGL(fn, dim3(unsigned(pl.sp_s), unsigned(H_kv), unsigned(B)),
                           dim3(kWave * waves), 0, st, s);
        TQKV_LAUNCHED();
      }
    }
    launch_merge(po, pm, pl_, pl.n_part, D, int64_t(B) * H, out, st);
    TQKV_LAUNCHED();
    return ok();
  }

  a.n_splits = pl.n_splits;
  a.split_len = pl.split_len;
  a.split_base = 0;
  a.n_part = a.n_splits;
  if (a.n_splits > 1) {
    a.part_o = static_cast<float*>(ws);
    a.part_m = a.part_o + size_t(B) * H * a.n_splits * D;
    a.part_l = a.part_m + size_t(B) * H * a.n_splits;
  }
  for (a.h_off = 0; a.h_off < G; a.h_off += Gk) {
    hipLaunchKernelGGL(fn, dim3(unsigned(a.n_splits), unsigned(H_kv), unsigned(B)),
                       dim3(kWave * waves), 0, st, a);
    TQKV_LAUNCHED();
  }
  if (a.n_splits > 1) {
    launch_merge(a.part_o, a.part_m, a.part_l, a.n_splits, D, int64_t(B) * H, out, st);
    TQKV_LAUNCHED();
  }
  return ok();
}

}  // namespace

extern "C" int32_t tqkv_decode_attend_affine(const uint16_t* q, int32_t B, int32_t H,
                                             int32_t H_kv, int32_t D, int32_t group_size,
                                             int32_t bits_k, int32_t bits_v, float scale,
                                             const tqkv_affine_seg* segs, int32_t n_segs,
                                             uint16_t* out, void* workspace,
                                             size_t workspace_bytes, tqkv_stream stream) {
  return decode_affine(q, B, H, H_kv, D, group_size, bits_k, bits_v, scale, segs, n_segs,
                       nullptr, out, workspace, workspace_bytes, stream);
}

extern "C" int32_t tqkv_decode_attend_affine_append(
    const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t D, int32_t group_size,
    int32_t bits_k, int32_t bits_v, float scale, const tqkv_affine_seg* segs, int32_t n_segs,
    const uint16_t* k, const uint16_t* v, uint32_t* k_packed, uint16_t* k_scales,
    uint16_t* k_biases, uint32_t* v_packed, uint16_t* v_scales, uint16_t* v_biases,
    int64_t dst_cap, int64_t dst_row, uint16_t* out, void* workspace, size_t workspace_bytes,
    tqkv_stream stream) {
  if (!k || !v || !k_packed || !k_scales || !k_biases || !v_packed || !v_scales || !v_biases)
    return fail(TQKV_EINVAL_ARG, "null pointer");
  if ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v)) % 16 != 0)
    return fail(TQKV_EINVAL_ARG, "new K/V rows must be 16-byte aligned");
  const AppendDst app{k, v, k_packed, k_scales, k_biases, v_packed, v_scales, v_biases,
                      dst_cap, dst_row};
  return decode_affine(q, B, H, H_kv, D, group_size, bits_k, bits_v, scale, segs, n_segs, &app,
                       out, workspace, workspace_bytes, stream);
}

namespace tqkv {
// The workspace bytes a decode over segments of these lengths needs (0: it
// writes no split partials). tqkv_cache_append_decode checks it before it
// commits a cache update.
size_t decode_need_bytes(int B, int H, int H_kv, int D, int group_size, int bits_k, int bits_v,
                         const tqkv_affine_seg* segs, int n_segs, bool app) {
  if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv != 0 || n_segs < 1 || n_segs > 2) return 0;
  int64_t max_rows = 0;
  for (int i = 0; i < n_segs; ++i) max_rows = segs[i].n > max_rows ? segs[i].n : max_rows;
  const int G = H / H_kv;
  const int Gp = group_heads(D, bits_k, bits_v, G, group_size, max_rows);
  const bool tile = use_tile(D, bits_k, bits_v, G, app);
  if (!Gp && !tile) return 0;
  const int Gk = Gp ? kernel_heads(D, bits_k, bits_v, Gp, group_size, max_rows) : G;
  KernelFn fn = Gp ? pick(D, bits_k, bits_v, Gp, group_size, max_rows) : nullptr;
  const bool mfma = fn && fn == pick_mfma_only(D, bits_k, bits_v, Gp, group_size);
  return plan_decode(B, H, H_kv, D, Gk, decode_waves(D, bits_k, bits_v, Gk, group_size, mfma),
                     segs, n_segs, app, tile).need;
}
}  // namespace tqkv

// Decode over chosen 64-row pages of one cache segment plus its undigested
// tail (the attention half of sdpa_page_sparse, native_attention.rs:272-291):
// rows [0, keep * 64) of the first kernel segment stand for the pages in
// `chosen` (read through the paged kernel's page table), the second segment
// is rows [pages * 64, n) of the same buffers. With one query and no mask,
// attention does not depend on key order.
extern "C" int32_t tqkv_decode_attend_affine_pages(
    const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t D, int32_t group_size,
    int32_t bits_k, int32_t bits_v, float scale, const tqkv_affine_seg* seg,
    const int32_t* chosen, int32_t keep, int64_t pages, uint16_t* out, void* workspace,
    size_t workspace_bytes, tqkv_stream stream) {
  if (!q || !out || !seg || !chosen) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv != 0)
    return fail(TQKV_EINVAL_SHAPE, "B=%d H=%d H_kv=%d", B, H, H_kv);
  const tqkv_affine_seg& s = *seg;
  if (s.shared) return fail(TQKV_EUNSUPPORTED, "page-sparse decode over a shared segment");
  if (keep < 1 || pages < keep || pages * kPageRows > s.n || s.n > s.cap)
    return fail(TQKV_EINVAL_SHAPE, "keep=%d pages=%lld n=%lld cap=%lld", keep, (long long)pages,
                (long long)s.n, (long long)s.cap);
  if (!s.k_packed || !s.k_scales || !s.k_biases || !s.v_packed || !s.v_scales || !s.v_biases)
    return fail(TQKV_EINVAL_ARG, "null buffer");
  const int G = H / H_kv;
  KernelFn fn = nullptr;
  if (s.cap * D < (int64_t(1) << 31)) {
    switch (D) {
      case 64: fn = pick_mfma_d64(bits_k, bits_v, G, group_size, true); break;
      case 128: fn = pick_mfma_d128(bits_k, bits_v, G, group_size, true); break;
      case 256: fn = pick_mfma_d256(bits_k, bits_v, G, group_size, true); break;
    }
  }
  if (!fn)
    return fail(TQKV_EUNSUPPORTED, "page-sparse decode layout D=%d bits %d/%d gqa=%d gs=%d", D,
                bits_k, bits_v, G, group_size);
  Args a{};
  a.q = q;
  a.H = H;
  a.H_kv = H_kv;
  a.Gt = G;
  a.h_off = 0;
  a.gs = group_size;
  a.qscale = scale * kLog2e;
  const int64_t tail0 = pages * kPageRows;
  const int64_t bs = int64_t(H_kv) * s.cap;
  a.seg[0] = Seg{s.k_packed, s.k_scales, s.k_biases, s.v_packed, s.v_scales, s.v_biases,
                 s.cap, int64_t(keep) * kPageRows, bs};
  const int kr = D * bits_k / 32, vr = D * bits_v / 32, ng = D / group_size;
  a.seg[1] = Seg{s.k_packed + tail0 * kr, s.k_scales + tail0 * ng, s.k_biases + tail0 * ng,
                 s.v_packed + tail0 * vr, s.v_scales + tail0 * ng, s.v_biases + tail0 * ng,
                 s.cap, s.n - tail0, bs};
  a.n0 = int64_t(keep) * kPageRows;
  a.total = a.n0 + (s.n - tail0);
  a.pages = chosen;
  a.n_pages = keep;
  a.out = out;
  const int waves = decode_waves(D, bits_k, bits_v, G, group_size, true);
  plan_splits(B, H_kv, waves, a.total, &a.n_splits, &a.split_len);
  // A wavefront holds its page numbers one a lane: at most kMaxWavePages
  // pages a wavefront, so a split spans at most waves * kMaxWavePages.
  const int64_t most = int64_t(waves) * kMaxWavePages * kPageRows;
  if (a.split_len > most) {
    a.split_len = most;
    a.n_splits = int((a.total + a.split_len - 1) / a.split_len);
  }
  a.split_base = 0;
  a.n_part = a.n_splits;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (a.n_splits > 1) {
    const size_t need = size_t(B) * H * a.n_splits * (size_t(D) + 2) * sizeof(float);
    void* ws = workspace;
    if (!ws) {
      if (int32_t rc = scratch_for_current_device(need, &ws)) return rc;
    } else if (workspace_bytes < need) {
      return fail(TQKV_EINVAL_ARG, "workspace of %zu bytes, need %zu", workspace_bytes, need);
    }
    a.part_o = static_cast<float*>(ws);
    a.part_m = a.part_o + size_t(B) * H * a.n_splits * D;
    a.part_l = a.part_m + size_t(B) * H * a.n_splits;
  }
  hipLaunchKernelGGL(fn, dim3(unsigned(a.n_splits), unsigned(H_kv), unsigned(B)),
                     dim3(kWave * waves), 0, st, a);
  TQKV_LAUNCHED();
  if (a.n_splits > 1) {
    launch_merge(a.part_o, a.part_m, a.part_l, a.n_splits, D, int64_t(B) * H, out, st);
    TQKV_LAUNCHED();
  }
  return ok();
}

// Workspace of the page-sparse call: the chosen-page table, the page bounds,
// then the decode's split partials.
size_t sparse_table_bytes(int32_t B, int32_t H_kv, int32_t keep) {
  return (size_t(B) * H_kv * size_t(keep) * sizeof(int32_t) + 255) / 256 * 256;
}

extern "C" size_t tqkv_sparse_workspace_size(int32_t B, int32_t H, int32_t H_kv, int32_t D,
                                             int64_t total_tokens, int32_t keep) {
  if (B <= 0 || H <= 0 || H_kv <= 0 || keep < 0 || total_tokens <= 0) return 0;
  return sparse_table_bytes(B, H_kv, keep) +
         tqkv_page_select_workspace_size(B, H_kv, total_tokens / kPageRows + 1) +
         tqkv_decode_workspace_size(B, H, H_kv, D, total_tokens) +
         size_t(B) * H * (size_t(D) + 2) * sizeof(float) *
             size_t(total_tokens / (int64_t(4) * kMaxWavePages * kPageRows) + 1);
}

// sdpa_page_sparse whole (native_attention.rs:210-291): with keep or fewer
// digested pages, dense decode over the segment; otherwise the page choice
// into the workspace's table, then decode over the chosen pages and the tail.
extern "C" int32_t tqkv_decode_attend_affine_sparse(
    const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t D, int32_t group_size,
    int32_t bits_k, int32_t bits_v, float scale, const tqkv_affine_seg* seg,
    const uint16_t* key_min, const uint16_t* key_max, int64_t max_pages, int64_t pages,
    int32_t keep, uint16_t* out, int32_t* chosen_out, void* workspace, size_t workspace_bytes,
    tqkv_stream stream) {
  if (!seg) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (pages <= keep)
    return tqkv_decode_attend_affine(q, B, H, H_kv, D, group_size, bits_k, bits_v, scale, seg, 1,
                                     out, workspace, workspace_bytes, stream);
  if (!workspace) return fail(TQKV_EINVAL_ARG, "page-sparse decode needs a workspace");
  if (B <= 0 || H_kv <= 0 || keep < 1) return fail(TQKV_EINVAL_SHAPE, "B=%d H_kv=%d keep=%d", B, H_kv, keep);
  const size_t table = sparse_table_bytes(B, H_kv, keep);
  const size_t bnd = tqkv_page_select_workspace_size(B, H_kv, pages);
  if (workspace_bytes < table + bnd)
    return fail(TQKV_EINVAL_ARG, "workspace of %zu bytes, need more than %zu", workspace_bytes,
                table + bnd);
  char* w = static_cast<char*>(workspace);
  int32_t* chosen = chosen_out ? chosen_out : reinterpret_cast<int32_t*>(w);
  if (int32_t rc = tqkv_page_select(q, B, H, H_kv, D, key_min, key_max, max_pages, pages, keep,
                                    chosen, w + table, bnd, stream))
    return rc;
  return tqkv_decode_attend_affine_pages(q, B, H, H_kv, D, group_size, bits_k, bits_v, scale, seg,
                                         chosen, keep, pages, out, w + table + bnd,
                                         workspace_bytes - table - bnd, stream);
}
