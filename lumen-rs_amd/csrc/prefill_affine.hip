// Host side of the affine prefill-chunk attention: argument checks, the
// kernel choice and the launch. The kernel and its design notes are in
// prefill_affine.hpp.
#include <cmath>

#include "prefill_affine.hpp"

using namespace tqkv;
using namespace tqkv::prefill;

namespace {

bool valid_bits(int bits) {
  return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
}

KernelFn pick(int D, int bk, int bv) {
  switch (D) {
    case 64: return pick_d64(bk, bv);
    case 128: return pick_d128(bk, bv);
    case 256: return pick_d256(bk, bv);
  }
  return nullptr;
}

}  // namespace

extern "C" int32_t tqkv_prefill_attend_affine(const uint16_t* q, int32_t B, int32_t H,
                                              int32_t H_kv, int32_t L, int32_t D,
                                              int32_t group_size, int32_t bits_k, int32_t bits_v,
                                              float scale, const tqkv_affine_seg* segs,
                                              int32_t n_segs, int64_t q_start, int64_t k_start,
                                              int32_t causal, int64_t window, uint16_t* out,
                                              tqkv_stream stream) {
  if (!q || !out || !segs) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv != 0 || L <= 0)
    return fail(TQKV_EINVAL_SHAPE, "B=%d H=%d H_kv=%d L=%d", B, H, H_kv, L);
  if (n_segs < 1 || n_segs > 2) return fail(TQKV_EINVAL_ARG, "n_segs=%d", n_segs);
  if (!valid_bits(bits_k) || !valid_bits(bits_v))
    return fail(TQKV_EUNSUPPORTED, "affine bits_k=%d bits_v=%d not in {2,3,4,5,6,8}", bits_k,
                bits_v);
  if (!(group_size == 32 || group_size == 64 || group_size == 128) || D % group_size != 0)
    return fail(TQKV_EUNSUPPORTED, "group_size=%d with D=%d", group_size, D);
  KernelFn fn = pick(D, bits_k, bits_v);
  if (!fn) return fail(TQKV_EUNSUPPORTED, "prefill head dim D=%d (64, 128 or 256)", D);
  if (causal && window == 0) return fail(TQKV_EINVAL_ARG, "window=0 hides every key");
  if (!(scale > 0.0f) || !std::isfinite(scale))
    return fail(TQKV_EINVAL_ARG, "softmax scale %g must be positive and finite", double(scale));
  if (int64_t(B) * H * L * D >= (int64_t(1) << 40))
    return fail(TQKV_EINVAL_SHAPE, "query tensor too large");

  Args a{};
  a.q = q;
  a.out = out;
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

  int rows_per_block = 0, threads = 0;
  switch (D) {
    case 64: rows_per_block = Shape<64>::kRows, threads = Shape<64>::kThreads; break;
    case 128: rows_per_block = Shape<128>::kRows, threads = Shape<128>::kThreads; break;
    default: rows_per_block = Shape<256>::kRows, threads = Shape<256>::kThreads; break;
  }
  const int64_t blocks = (int64_t(L) * a.G + rows_per_block - 1) / rows_per_block;
  const int64_t grid = blocks * H_kv * B;
  if (grid > 0x7fffffff) return fail(TQKV_EINVAL_SHAPE, "grid too large");
  a.n_blocks = int(blocks);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(fn, dim3(unsigned(grid)), dim3(threads), 0, st, a);
  TQKV_LAUNCHED();
  return ok();
}
