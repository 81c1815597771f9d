// Host side of the affine prefill-chunk attention: argument checks, the
// kernel choice and the launch. The kernel and its design notes are in
// prefill_affine.hpp.
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "prefill_affine.hpp"

namespace tqkv {
namespace prefill {
namespace {

bool valid_bits(int bits) {
  return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
}

KernelFn pick(int D, int bk, int bv, bool h16 = false) {
  switch (D) {
    case 64: return pick_d64(bk, bv, h16);
    case 128: return pick_d128(bk, bv, h16);
    case 256: return pick_d256(bk, bv, h16);
    case 512: return pick_d512(bk, bv, h16);
  }
  return nullptr;
}

// Dequantize-once: keys [0, total) of every (batch row, KV head), K into kd
// as bf16 rows [B * H_kv, slab_rows, D] with mlx::dequantize's arithmetic
// (bf16(fma(scale, code, bias)), one rounding), V into vd as the prefill
// kernel's V operands (those bf16 values times 2^-kVShift, in f16; see
// v_operand_run): rows like K, or with vt (D = 128) transposed 64-key tiles
// (width kPreF16T; slab_rows a multiple of 64, zeros past the last key).
// Grid: (row-run chunks, slab, K and/or V); a thread takes one run of 32
// values of one row: its BITS words in one or two wide loads, its group's
// scale and bias (a run never straddles a group: gs is a multiple of 32).
// A wavefront's 64 runs are 4 KB of consecutive rows; they pass through LDS
// so that each of the wavefront's four 16-byte store instructions writes 1
// KB contiguously (measured on MI355X: 64-byte strided 16-byte stores reach
// 3.5 TB/s, contiguous ones 7.0). A V^T tile is a workgroup's 256 runs (64
// keys at D = 128), transposed through LDS with the transposing read, its
// 16 KB written 1 KB a store instruction. kinds: 1 = K, 2 = V, 3 = both
// (blockIdx.z picks). Keys [0, n0) come from segment 0, the rest from
// segment 1.
template <int D, int BITS>
__global__ __launch_bounds__(256) void dequantize_rows_kernel(const Args a, int kinds,
                                                              int64_t slab_rows, int vt,
                                                              uint16_t* kd, uint16_t* vd) {
  constexpr int kRuns = D / 32;
  static_assert(64 % kRuns == 0, "a wavefront covers whole rows");
  constexpr int kChunkRows = D / 8;  // 16-byte chunks a row
  constexpr int KSTR = kKStride<D>;
  // A wavefront's 64 runs x 4 chunks each (rows), or the tile's 64 keys
  // row-major at the prefill kernel's stride (V^T).
  constexpr int kLds = D == 128 ? 64 * KSTR / 8 : 1024;
  __shared__ uint4 s_buf[kLds];
  const int wv = threadIdx.x / 64, l = threadIdx.x % 64;
  const uint32_t j = blockIdx.x * 256u + threadIdx.x;
  const uint32_t total = uint32_t(a.total);
  if (total == 0) return;  // (uniform: no wavefront reaches the exchange)
  const uint32_t row = j / kRuns;
  const uint32_t lrow = row < total ? row : total - 1;  // past the end: load a live row
  const int run = int(j % kRuns);
  const int slab = int(blockIdx.y), bb = slab / a.H_kv, kv = slab % a.H_kv;
  const bool isv = kinds == 3 ? blockIdx.z != 0 : kinds == 2;
  const bool first = lrow < uint32_t(a.n0);
  const Seg& s = a.seg[first ? 0 : 1];
  const int64_t src = int64_t(bb) * s.b_stride + int64_t(kv) * s.cap +
                      (first ? lrow : lrow - uint32_t(a.n0));
  const uint32_t* pw = (isv ? s.vw : s.kw) + src * (D * BITS / 32) + run * BITS;
  const int64_t g = src * (D / a.gs) + (run * 32) / a.gs;
  const uint32_t sb = uint32_t((isv ? s.vs : s.ks)[g]) | (uint32_t((isv ? s.vb : s.kb)[g]) << 16);
  uint32_t w[BITS], out[16];
  load_words<BITS>(w, pw);
  if (isv)
    v_operand_run<BITS>(w, sb, out);
  else
    dequant_run<BITS, false>(w, sb, out);
  if constexpr (D == 128) {
    if (isv && vt) {  // (block-uniform)
      // Keys past the end are zeros: their weights are exactly 0, and 0
      // times a zero operand stays 0.
      const int key = int(threadIdx.x) / kRuns;
      uint4* d = reinterpret_cast<uint4*>(reinterpret_cast<uint16_t*>(s_buf) + key * KSTR + run * 32);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        d[i] = row < total ? uint4{out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]}
                           : uint4{0u, 0u, 0u, 0u};
      __syncthreads();
      // Store pass (u, tt) of wavefront wv: lane (grp, lr) takes channel
      // 16 tt + lr of keys 32 u + 4 grp + [0, 4) and 32 u + 16 + 4 grp +
      // [0, 4) (two transposing reads), the 16 bytes at slot 8 grp of V^T
      // row u D + 16 tt + lr; the wavefront's 64 chunks are 16 whole rows.
      const int grp = l / 16, lr = l % 16;
      uint4* tile = reinterpret_cast<uint4*>(vd + (int64_t(slab) * slab_rows + int64_t(blockIdx.x) * kTile) * D);
      const uint16_t* sv = reinterpret_cast<const uint16_t*>(s_buf);
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int pass = 4 * wv + it, u = pass / 8, tt = pass % 8;
        const uint16_t* vrow = sv + (32 * u + 4 * grp + lr / 4) * KSTR + 16 * tt + 4 * (lr % 4);
        const u32x2_t lo = tr_read(vrow);
        const u32x2_t hi = tr_read(vrow + 16 * KSTR);
        tile[(u * D + 16 * tt + lr) * 4 + grp] = uint4{lo.x, lo.y, hi.x, hi.y};
      }
      return;
    }
  }
  // Lane l's run is chunks 4 l .. 4 l + 3 of the wavefront's block; store i
  // of lane l writes chunk 64 i + l. The exchange stays inside one
  // wavefront, so a wavefront-scope fence orders it (no workgroup barrier).
  uint4* s_t = s_buf + 256 * wv;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    s_t[4 * l + i] = uint4{out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]};
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const uint32_t row0 = (blockIdx.x * 256u + wv * 64u) / kRuns;
  uint4* d = reinterpret_cast<uint4*>((isv ? vd : kd) + (int64_t(slab) * slab_rows + row0) * D);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = 64 * i + l;
    if (row0 + uint32_t(c / kChunkRows) < total) d[c] = s_t[c];
  }
}

template <int D>
void launch_dequantize_rows(const Args& a, int bits, int kinds, int64_t slab_rows, int vt,
                            dim3 grid, hipStream_t st, uint16_t* kd, uint16_t* vd) {
#define TQKV_DQ(B)                                                                            \
  hipLaunchKernelGGL((dequantize_rows_kernel<D, B>), grid, dim3(256), 0, st, a, kinds, slab_rows, \
                     vt, kd, vd)
  switch (bits) {
    case 2: TQKV_DQ(2); break;
    case 3: TQKV_DQ(3); break;
    case 4: TQKV_DQ(4); break;
    case 5: TQKV_DQ(5); break;
    case 6: TQKV_DQ(6); break;
    default: TQKV_DQ(8); break;
  }
#undef TQKV_DQ
}

// V as transposed tiles (width kPreF16T) at this head dim.
constexpr bool v_tiles(int D) { return D == 128; }
// Rows a slab of the dequantize-once scratch holds: total, padded to whole
// 64-key tiles where V is tiled (K shares the stride).
int64_t once_slab_rows(int D, int64_t total) {
  return v_tiles(D) ? (total + kTile - 1) / kTile * kTile : total;
}

// Both halves of the dequantize-once pass: one launch when K and V share a
// width, else one each. (At D = 128 a chunk of 256 runs is one 64-key tile.)
template <int D>
void dequantize_rows(const Args& a, int bk, int bv, int64_t slabs, hipStream_t st, uint16_t* kd,
                     uint16_t* vd) {
  const unsigned chunks = unsigned((a.total * (D / 32) + 255) / 256);
  const int64_t sr = once_slab_rows(D, a.total);
  const int vt = v_tiles(D) ? 1 : 0;
  if (bk == bv) {
    launch_dequantize_rows<D>(a, bk, 3, sr, vt, dim3(chunks, unsigned(slabs), 2), st, kd, vd);
  } else {
    launch_dequantize_rows<D>(a, bk, 1, sr, vt, dim3(chunks, unsigned(slabs), 1), st, kd, vd);
    launch_dequantize_rows<D>(a, bv, 2, sr, vt, dim3(chunks, unsigned(slabs), 1), st, kd, vd);
  }
}

// Row blocks sharing one (batch row, KV head) from which the keys are
// dequantized once into scratch instead of in every block: the blocks would
// otherwise repeat the same dequantization, the kernel's VALU-bound part.
constexpr int64_t kOnceBlocks = 8;
// The scratch that path may take (bf16 K and V of every visible key); larger
// contexts dequantize in every block instead.
constexpr size_t kOnceMaxBytes = size_t(4) << 30;

}  // namespace
}  // namespace prefill
}  // namespace tqkv

using namespace tqkv;
using namespace tqkv::prefill;

namespace tqkv {
namespace prefill {

// The shared-prefix half of a decode step: the queries of all B sequences
// (one position each) against a prefix every sequence shares, read once per
// KV head. The B sequences act as B query positions of one batch row
// (rows (b, g) of a KV head), the prefix's keys are split over the grid,
// and each split's (o, m, l) go to slots [0, n_splits) of the decode's
// partials [B, H, n_part]. Rows b * H + h line up with the decode kernel's.
bool tile_decode_supported(int D, int bk, int bv) { return D == 512 && pick(D, bk, bv, true); }
int tile_decode_rows() { return Shape<512, true>::kRows; }

// Decode through the tile kernel (f16 operands): each sequence's G query
// heads of a KV head are the rows of one block (one position, L = 1), the
// keys of up to two segments split over the grid; with n_splits > 1 each
// split's (o, m, l) go to slots [0, n_splits) of the decode's partials
// [B, H, n_part] (the decode's merge finishes), else the block writes out.
// Serves head_dim 512, which no decode kernel takes on the matrix cores.
int32_t tile_decode(const uint16_t* q, int B, int H, int H_kv, int D, int gs, int bk, int bv,
                    float scale, const tqkv_affine_seg* segs, int n_segs, int n_splits,
                    int split_len, int n_part, float* part_o, float* part_m, float* part_l,
                    uint16_t* out, hipStream_t st) {
  KernelFn fn = pick(D, bk, bv, true);
  if (!fn || D != 512) return fail(TQKV_EUNSUPPORTED, "tile decode D=%d bits %d/%d", D, bk, bv);
  Args a{};
  a.q = q;
  a.out = out;
  a.qs_b = int64_t(H) * D;
  a.qs_h = D;
  a.qs_l = int64_t(H) * D;
  a.H = H;
  a.H_kv = H_kv;
  a.G = H / H_kv;
  a.L = 1;
  a.gs = gs;
  a.causal = 0;
  a.qscale = scale * kLog2e;
  for (int i = 0; i < n_segs; ++i) {
    const tqkv_affine_seg& sg = segs[i];
    // Rows of a slab are addressed with 32-bit word offsets.
    if (sg.cap > 0 && sg.cap * int64_t(D) * (bk > bv ? bk : bv) / 32 >= (int64_t(1) << 32))
      return fail(TQKV_EINVAL_SHAPE, "segment %d: cap=%lld rows too large", i, (long long)sg.cap);
    a.seg[i] = Seg{sg.k_packed, sg.k_scales, sg.k_biases, sg.v_packed, sg.v_scales, sg.v_biases,
                   sg.cap, sg.shared ? 0 : int64_t(H_kv) * sg.cap};
  }
  if (n_segs == 1) a.seg[1] = a.seg[0];
  a.n0 = segs[0].n;
  a.total = segs[0].n + (n_segs == 2 ? segs[1].n : 0);
  if (a.total > (int64_t(1) << 31) - 2 * kTile)
    return fail(TQKV_EINVAL_SHAPE, "%lld keys exceed the kernel's 32-bit key index",
                (long long)a.total);
  a.n_splits = n_splits;
  a.split_len = split_len;
  a.split_base = 0;
  a.n_part = n_part;
  a.part_o = n_splits > 1 ? part_o : nullptr;
  a.part_m = n_splits > 1 ? part_m : nullptr;
  a.part_l = n_splits > 1 ? part_l : nullptr;
  using S = Shape<512, true>;
  const int64_t blocks = (a.G + S::kRows - 1) / S::kRows;
  a.n_blocks = int(blocks);
  const int64_t grid = blocks * n_splits * H_kv * int64_t(B);
  if (grid > 0x7fffffff) return fail(TQKV_EINVAL_SHAPE, "grid too large");
  hipLaunchKernelGGL(fn, dim3(unsigned(grid)), dim3(S::kThreads), 0, st, a);
  TQKV_LAUNCHED();
  return TQKV_OK;
}

int shared_prefix_block_rows(int D) {
  switch (D) {
    case 64: return Shape<64, true>::kRows;
    case 128: return Shape<128, true>::kRows;
    default: return Shape<256, true>::kRows;
  }
}

int32_t shared_prefix_partials(const uint16_t* q, int B, int H, int H_kv, int D, int gs, int bk,
                               int bv, float scale, const tqkv_affine_seg& prefix, int n_splits,
                               int split_len, int n_part, float* part_o, float* part_m,
                               float* part_l, hipStream_t st) {
  // f16 operands: decode's bar is the exact dequantization, and f16's
  // three more significand bits keep the shared-prefix path within it.
  KernelFn fn = pick(D, bk, bv, true);
  if (!fn) return fail(TQKV_EUNSUPPORTED, "shared-prefix decode D=%d bits %d/%d", D, bk, bv);
  Args a{};
  a.q = q;
  a.out = nullptr;
  a.qs_b = 0;
  a.qs_h = D;
  a.qs_l = int64_t(H) * D;  // position l of the one batch row = sequence l
  a.H = H;
  a.H_kv = H_kv;
  a.G = H / H_kv;
  a.L = B;
  a.gs = gs;
  a.causal = 0;
  a.qscale = scale * kLog2e;
  a.seg[0] = Seg{prefix.k_packed, prefix.k_scales, prefix.k_biases, prefix.v_packed,
                 prefix.v_scales, prefix.v_biases, prefix.cap, 0};
  a.seg[1] = a.seg[0];
  a.n0 = prefix.n;
  a.total = prefix.n;
  a.n_splits = n_splits;
  a.split_len = split_len;
  a.split_base = 0;
  a.n_part = n_part;
  a.part_o = part_o;
  a.part_m = part_m;
  a.part_l = part_l;
  int rows_per_block = 0, threads = 0;
  switch (D) {
    case 64: rows_per_block = Shape<64, true>::kRows, threads = Shape<64, true>::kThreads; break;
    case 128: rows_per_block = Shape<128, true>::kRows, threads = Shape<128, true>::kThreads; break;
    default: rows_per_block = Shape<256, true>::kRows, threads = Shape<256, true>::kThreads; break;
  }
  const int64_t blocks = (int64_t(B) * a.G + rows_per_block - 1) / rows_per_block;
  a.n_blocks = int(blocks);
  const int64_t grid = blocks * n_splits * H_kv;
  if (grid > 0x7fffffff) return fail(TQKV_EINVAL_SHAPE, "grid too large");
  hipLaunchKernelGGL(fn, dim3(unsigned(grid)), dim3(threads), 0, st, a);
  TQKV_LAUNCHED();
  return TQKV_OK;
}

}  // namespace prefill
}  // namespace tqkv

namespace {

// The prefill launch over affine segments, or (bf16_rows) over one segment
// whose "packed" arrays are bf16 rows of D values (K and V already
// dequantized or stored in bf16; scales and biases unused).
int32_t prefill_launch(const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t L,
                       int32_t D, int32_t group_size, int32_t bits_k, int32_t bits_v, float scale,
                       const tqkv_affine_seg* segs, int32_t n_segs, int64_t q_start,
                       int64_t k_start, int32_t causal, int64_t window, uint16_t* out,
                       tqkv_stream stream, bool bf16_rows, bool library_scratch = true,
                       void* workspace = nullptr, size_t workspace_bytes = 0) {
  if (!q || !out || !segs) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv != 0 || L <= 0)
    return fail(TQKV_EINVAL_SHAPE, "B=%d H=%d H_kv=%d L=%d", B, H, H_kv, L);
  if (n_segs < 1 || n_segs > 2 || (bf16_rows && n_segs != 1))
    return fail(TQKV_EINVAL_ARG, "n_segs=%d", n_segs);
  if (bf16_rows) {
    bits_k = bits_v = kPreBits;
  } else if (!valid_bits(bits_k) || !valid_bits(bits_v)) {
    return fail(TQKV_EUNSUPPORTED, "affine bits_k=%d bits_v=%d not in {2,3,4,5,6,8}", bits_k,
                bits_v);
  }
  if (!(group_size == 32 || group_size == 64 || group_size == 128) || D % group_size != 0)
    return fail(TQKV_EUNSUPPORTED, "group_size=%d with D=%d", group_size, D);
  KernelFn fn = pick(D, bits_k, bits_v);
  if (!fn) return fail(TQKV_EUNSUPPORTED, "prefill head dim D=%d (64, 128, 256 or 512)", D);
  if (causal && window == 0) return fail(TQKV_EINVAL_ARG, "window=0 hides every key");
  if (!(scale > 0.0f) || !std::isfinite(scale))
    return fail(TQKV_EINVAL_ARG, "softmax scale %g must be positive and finite", double(scale));
  if (int64_t(B) * H * L * D >= (int64_t(1) << 40))
    return fail(TQKV_EINVAL_SHAPE, "query tensor too large");

  Args a{};
  a.q = q;
  a.out = out;
  a.qs_l = D;
  a.qs_h = int64_t(L) * D;
  a.qs_b = int64_t(H) * L * D;
  a.H = H;
  a.H_kv = H_kv;
  a.G = H / H_kv;
  a.L = L;
  a.gs = group_size;
  a.causal = causal ? 1 : 0;
  a.qscale = scale * kLog2e;
  for (int i = 0; i < n_segs; ++i) {
    const tqkv_affine_seg& s = segs[i];
    if (s.n < 0 || s.n > s.cap)
      return fail(TQKV_EINVAL_SHAPE, "segment %d: n=%lld cap=%lld", i, (long long)s.n,
                  (long long)s.cap);
    if (s.n > 0 && (!s.k_packed || !s.k_scales || !s.k_biases || !s.v_packed || !s.v_scales ||
                    !s.v_biases))
      return fail(TQKV_EINVAL_ARG, "segment %d has a null buffer", i);
    // Rows of a slab are addressed with 32-bit word offsets.
    if (s.cap > 0 && s.cap * int64_t(D) * (bits_k > bits_v ? bits_k : bits_v) / 32 >= (int64_t(1) << 32))
      return fail(TQKV_EINVAL_SHAPE, "segment %d: cap=%lld rows too large", i, (long long)s.cap);
    a.seg[i] = Seg{s.k_packed, s.k_scales, s.k_biases, s.v_packed, s.v_scales, s.v_biases,
                   s.cap, s.shared ? 0 : int64_t(H_kv) * s.cap};
  }
  if (n_segs == 1) a.seg[1] = a.seg[0];
  a.n0 = segs[0].n;
  a.total = segs[0].n + (n_segs == 2 ? segs[1].n : 0);
  if (a.total <= 0) return fail(TQKV_EINVAL_SHAPE, "no keys to attend");
  if (a.total > (int64_t(1) << 31) - 2 * kTile)
    return fail(TQKV_EINVAL_SHAPE, "%lld keys exceed the kernel's 32-bit key index",
                (long long)a.total);
  a.q_start = q_start;
  a.k_start = k_start;
  a.window = window < 0 ? -1 : window;
  a.n_splits = 1;
  a.split_len = int(a.total + kTile - 1) / kTile * kTile;
  a.split_base = 0;
  a.n_part = 1;

  int rows_per_block = 0, threads = 0;
  switch (D) {
    case 64: rows_per_block = Shape<64, false>::kRows, threads = Shape<64, false>::kThreads; break;
    case 128: rows_per_block = Shape<128, false>::kRows, threads = Shape<128, false>::kThreads; break;
    case 256: rows_per_block = Shape<256, false>::kRows, threads = Shape<256, false>::kThreads; break;
    default: rows_per_block = Shape<512, false>::kRows, threads = Shape<512, false>::kThreads; break;
  }
  const int64_t blocks = (int64_t(L) * a.G + rows_per_block - 1) / rows_per_block;
  const int64_t grid = blocks * a.n_splits * H_kv * B;
  if (grid > 0x7fffffff) return fail(TQKV_EINVAL_SHAPE, "grid too large");
  a.n_blocks = int(blocks);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  // TQKV_PREFILL_DEQUANT_ONCE=0 / 1 forces the choice (tests compare them).
  const char* once_env = getenv("TQKV_PREFILL_DEQUANT_ONCE");
  const int64_t slabs = int64_t(B) * H_kv;
  const int64_t slab_rows = once_slab_rows(D, a.total);
  const size_t need = 2 * size_t(slabs) * size_t(slab_rows) * size_t(D) * 2;
  // With a caller workspace (the _ws entry) the dequantized rows go there
  // when it holds them, else every block dequantizes for itself.
  const bool fits = library_scratch || (workspace && workspace_bytes >= need);
  const bool once = !bf16_rows && fits &&
                    (once_env ? strcmp(once_env, "0") != 0
                              : blocks >= kOnceBlocks && need <= kOnceMaxBytes);
  if (once) {
    void* ws = workspace;
    if (library_scratch)
      if (int32_t rc = scratch_for_current_device(need, &ws)) return rc;
    uint16_t* kd = static_cast<uint16_t*>(ws);
    uint16_t* vd = kd + size_t(slabs) * size_t(slab_rows) * size_t(D);
    if (slabs > 65535) return fail(TQKV_EINVAL_SHAPE, "B * H_kv = %lld slabs", (long long)slabs);
    switch (D) {
      case 64: dequantize_rows<64>(a, bits_k, bits_v, slabs, st, kd, vd); break;
      case 128: dequantize_rows<128>(a, bits_k, bits_v, slabs, st, kd, vd); break;
      case 256: dequantize_rows<256>(a, bits_k, bits_v, slabs, st, kd, vd); break;
      default: dequantize_rows<512>(a, bits_k, bits_v, slabs, st, kd, vd); break;
    }
    TQKV_LAUNCHED();
    Args p = a;
    const uint16_t* none = kd;  // scales and biases: never read at this width
    p.seg[0] = Seg{reinterpret_cast<const uint32_t*>(kd), none, none,
                   reinterpret_cast<const uint32_t*>(vd), none, none, slab_rows,
                   int64_t(H_kv) * slab_rows};
    p.seg[1] = p.seg[0];
    p.n0 = a.total;
    hipLaunchKernelGGL(pick(D, kPreBits, v_tiles(D) ? kPreF16T : kPreF16), dim3(unsigned(grid)),
                       dim3(threads), 0, st, p);
    TQKV_LAUNCHED();
    return ok();
  }
  hipLaunchKernelGGL(fn, dim3(unsigned(grid)), dim3(threads), 0, st, a);
  TQKV_LAUNCHED();
  return ok();
}

}  // namespace

extern "C" int32_t tqkv_prefill_attend_affine(const uint16_t* q, int32_t B, int32_t H,
                                              int32_t H_kv, int32_t L, int32_t D,
                                              int32_t group_size, int32_t bits_k, int32_t bits_v,
                                              float scale, const tqkv_affine_seg* segs,
                                              int32_t n_segs, int64_t q_start, int64_t k_start,
                                              int32_t causal, int64_t window, uint16_t* out,
                                              tqkv_stream stream) {
  return prefill_launch(q, B, H, H_kv, L, D, group_size, bits_k, bits_v, scale, segs, n_segs,
                        q_start, k_start, causal, window, out, stream, false);
}

extern "C" size_t tqkv_prefill_workspace_size(int32_t B, int32_t H_kv, int32_t D,
                                              int64_t total_keys) {
  if (B <= 0 || H_kv <= 0 || D <= 0 || total_keys <= 0) return 0;
  return 2 * size_t(B) * size_t(H_kv) * size_t(once_slab_rows(D, total_keys)) * size_t(D) * 2;
}

extern "C" int32_t tqkv_prefill_attend_affine_ws(
    const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t L, int32_t D,
    int32_t group_size, int32_t bits_k, int32_t bits_v, float scale, const tqkv_affine_seg* segs,
    int32_t n_segs, int64_t q_start, int64_t k_start, int32_t causal, int64_t window,
    uint16_t* out, void* workspace, size_t workspace_bytes, tqkv_stream stream) {
  return prefill_launch(q, B, H, H_kv, L, D, group_size, bits_k, bits_v, scale, segs, n_segs,
                        q_start, k_start, causal, window, out, stream, false, false, workspace,
                        workspace_bytes);
}

namespace tqkv {
// Prefill-chunk attention over bf16 K and V rows ([B, H_kv, cap, D], keys
// [0, n) of each slab): the same MFMA kernel with the dequantization left
// out (codebook caches after tqkv_codebook_dequantize, bf16 caches).
int32_t prefill_bf16_rows(const uint16_t* q, int B, int H, int H_kv, int L, int D,
                          const uint16_t* k, const uint16_t* v, int64_t cap, int64_t n,
                          int64_t q_start, int64_t k_start, int64_t window, float scale,
                          uint16_t* out, hipStream_t stream) {
  tqkv_affine_seg s{};
  s.k_packed = reinterpret_cast<const uint32_t*>(k);
  s.v_packed = reinterpret_cast<const uint32_t*>(v);
  s.k_scales = s.k_biases = k;  // never read at this width
  s.v_scales = s.v_biases = v;
  s.cap = cap;
  s.n = n;
  return prefill_launch(q, B, H, H_kv, L, D, 64, 0, 0, scale, &s, 1, q_start, k_start, 1, window,
                        out, reinterpret_cast<tqkv_stream>(stream), true);
}
}  // namespace tqkv
