// Prefill-chunk attention over affine-packed K/V on the matrix cores.
//
// What it computes (the reference's dequantized_prefill_attention,
// gemma4_moe.rs:2382-2411): K and V are dequantized the way mlx::dequantize
// does for bf16 (each of scale * code and + bias rounds to bf16), then
// softmax(scale * Q K^T + mask) V with bf16 operands and f32 accumulation.
// The mask is build_causal_mask_abs (native_attention.rs:545-622) in absolute
// positions: query row l sits at q_start + l, key k at k_start + k, and key k
// is visible to query l iff k_abs <= q_abs and, with a window W,
// q_abs < k_abs + W. It covers the reference's three prefill branches (causal
// SDPA, lumen_sdpa_windowed, sdpa_with_mask) with one kernel.
//
// Work split: one workgroup per (block of kRows flattened query rows, KV
// head, batch row). The G = H / H_kv query heads of a KV head share its keys,
// so their rows are flattened as (position l, head g), g fastest: a block of
// 128 rows covers 128 / G consecutive positions of all G heads, and the keys
// it must see are nearly the same for all of its rows (tile skipping stays
// effective under a causal or sliding mask).
//
// Per key tile (64 keys): the workgroup's threads each take one run of 32
// codes of one key (bits words) for K and for V, dequantize it and write K
// row-major [key][D] and V transposed [D][key] into LDS; the next tile's
// words are fetched into registers while the matrix cores work on this one.
// Each wavefront owns RW query rows:
//   S^T = K . Q^T: A = K rows from LDS (ds_read_b128), B = the wavefront's Q
//   rows held in registers for the whole kernel; lane l ends up with the
//   scores of query row l % 16 for keys 16i + 4(l / 16) + r.
//   Online softmax per row: the 64-key maximum is a 16-value local max plus
//   two lane exchanges (l ^ 16, l ^ 32); the running maximum may lag the true
//   one by up to kTau (log2 units), so the O accumulators are rescaled only
//   when some row moves by more. Row sums (of the bf16-rounded weights, one
//   v_dot2 per pair) stay per lane until the end.
//   O^T += V^T . P^T: the score registers of key tiles 2u and 2u + 1 are,
//   rounded to bf16, exactly the B operand (k slot 8(l / 16) + s holds key
//   32u + 4(l / 16) + s, s < 4, or 32u + 16 + 4(l / 16) + s - 4); the A
//   operand reads the same keys of V^T with two ds_read_b64.
// Only tiles that some row of the block can see are visited, and the
// per-element mask runs only on tiles that are not wholly visible.
#pragma once

#include <cmath>
#include <utility>

#include "common.hpp"

namespace tqkv {
namespace prefill {

constexpr int kWave = 64;
constexpr int kTile = 64;  // keys per tile
constexpr int kXcds = 8;   // accelerator dies (each with its own L2) on MI355X
// LDS row strides (bf16 elements). K rows: D + 8 keeps ds_read_b128 rows
// 16-byte aligned and 8 consecutive rows on distinct banks. V^T rows:
// kTile + 4 = 34 dwords, so the 16 rows one ds_read_b64 touches start on
// distinct even banks.
template <int D>
constexpr int kKStride = D + 8;
constexpr int kVStride = kTile + 4;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kTau = 8.0f;

typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
typedef float f2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct Seg {
  const uint32_t* kw;
  const uint16_t* ks;
  const uint16_t* kb;
  const uint32_t* vw;
  const uint16_t* vs;
  const uint16_t* vb;
  int64_t cap;
  int64_t b_stride;  // rows between batch rows: H_kv * cap, or 0 when shared
};

struct Args {
  const uint16_t* q;  // [B, H, L, D] bf16
  uint16_t* out;      // [B, H, L, D] bf16
  int H, H_kv, G, L, gs;
  int n_blocks;   // row blocks per (batch row, KV head)
  int causal;
  float qscale;   // softmax scale * log2(e)
  Seg seg[2];
  int64_t n0, total;  // keys in segment 0; keys in all
  int64_t q_start, k_start, window;
};

// Launch shape per head dim: wavefronts per workgroup and query rows per
// wavefront. More rows a workgroup spread the dequantization of a tile over
// more matrix-core work; the O accumulators (RW rows x D channels a
// wavefront) and two wavefronts per SIMD bound RW; D = 256 stays at 128 rows.
// Loader tasks: 64 keys x D/32 runs x {K, V}, kPer a thread.
template <int D>
struct Shape {
  static constexpr int kWaves = D == 64 ? 4 : 8;
  static constexpr int kRW = D == 256 ? 16 : 32;
  static constexpr int kRows = kWaves * kRW;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kPer = 4 * D / kThreads;
  static_assert(kPer * kThreads == 4 * D, "whole loader tasks per thread");
};

template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Code I of a run of 32 codes packed LSB-first in BITS words.
template <int BITS, int I>
__device__ __forceinline__ uint32_t code_at(const uint32_t* w) {
  constexpr int bit = I * BITS, wi = bit / 32, sh = bit % 32;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  if constexpr (sh + BITS <= 32)
    return (w[wi] >> sh) & mask;
  else
    return __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh) & mask;
}

template <int N>
__device__ __forceinline__ void load_words(uint32_t* dst, const uint32_t* src) {
  if constexpr (N >= 4) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(src);
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
    dst[3] = v.w;
    if constexpr (N > 4) load_words<N - 4>(dst + 4, src + 4);
  } else if constexpr (N == 3) {
    const u32x3_t v = *reinterpret_cast<const u32x3_t*>(src);
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
  } else if constexpr (N == 2) {
    const u32x2_t v = *reinterpret_cast<const u32x2_t*>(src);
    dst[0] = v.x;
    dst[1] = v.y;
  } else if constexpr (N == 1) {
    dst[0] = *src;
  }
}

// Takes the word by value: hipcc (clang 22) miscompiles __builtin_bit_cast
// of an ext_vector element expression such as w[1] (it reads element 0).
__device__ __forceinline__ bf2_t as_bf2(uint32_t x) { return __builtin_bit_cast(bf2_t, x); }

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  const f2_t f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf2_t));
}

// One loader task's share of a key tile: a run of 32 codes of one key of K
// or V (NW >= bits words), with the run's scale and bias (bf16 bits, scale
// low).
template <int NW>
struct Stage {
  uint32_t w[NW];
  uint32_t s, b;  // bf16 bits; combined only when used, so the loads stay in flight
  bool ok;
};

// Where the workgroup's loads start: the (batch row, KV head) slab of each
// segment (uniform, so it stays in scalar registers); rows and the thread's
// run are 32-bit offsets from there (the host checks that a slab fits).
struct SlabPtrs {  // one of K or V; segments 0 and 1 as separate fields (no
                  // indexed array, which would live in scratch memory)
  const uint32_t* w0;
  const uint32_t* w1;
  const uint16_t* s0;
  const uint16_t* s1;
  const uint16_t* b0;
  const uint16_t* b1;
};

template <int D, int BITS>
__device__ __forceinline__ SlabPtrs slabs_for(const Seg& s0, const Seg& s1, const uint32_t* w0,
                                              const uint32_t* w1, const uint16_t* sc0,
                                              const uint16_t* sc1, const uint16_t* bi0,
                                              const uint16_t* bi1, int gs, int b, int kvh) {
  const int64_t r0 = int64_t(b) * s0.b_stride + int64_t(kvh) * s0.cap;
  const int64_t r1 = int64_t(b) * s1.b_stride + int64_t(kvh) * s1.cap;
  const int groups = D / gs;
  return SlabPtrs{w0 + r0 * (D * BITS / 32), w1 + r1 * (D * BITS / 32), sc0 + r0 * groups,
                  sc1 + r1 * groups,         bi0 + r0 * groups,         bi1 + r1 * groups};
}

// Loads run `run` of key kk (counted across both segments) of K or V.
template <int D, int BITS, int NW>
__device__ __forceinline__ void load_stage(Stage<NW>& st, const SlabPtrs& p, const Args& a, int kk,
                                           int run) {
  st.ok = kk < a.total;
  if (!st.ok) return;
  const bool first = kk < a.n0;
  const uint32_t row = uint32_t(first ? kk : kk - int(a.n0));
  const uint32_t g = row * uint32_t(D / a.gs) + uint32_t(run * 32) / uint32_t(a.gs);
  const uint32_t* w = first ? p.w0 : p.w1;
  const uint16_t* sc = first ? p.s0 : p.s1;
  const uint16_t* bi = first ? p.b0 : p.b1;
  load_words<BITS>(st.w, w + (row * (D * BITS / 32) + run * BITS));
  st.s = sc[g];
  st.b = bi[g];
}

// The 32 codes of a run as floats. 2-, 4- and 8-bit codes are split into
// bytes first so each converts with one v_cvt_f32_ubyteN.
__device__ __forceinline__ float ubyte(uint32_t x, int j) { return float((x >> (8 * j)) & 0xffu); }

template <int BITS>
__device__ __forceinline__ void run_codes(const uint32_t* w, float* f) {
  if constexpr (BITS == 8) {
#pragma unroll
    for (int i = 0; i < 32; ++i) f[i] = ubyte(w[i / 4], i % 4);
  } else if constexpr (BITS == 4) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t e = w[k] & 0x0F0F0F0Fu, o = (w[k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f[8 * k + 2 * j] = ubyte(e, j);
        f[8 * k + 2 * j + 1] = ubyte(o, j);
      }
    }
  } else if constexpr (BITS == 2) {
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const uint32_t x = (w[k] >> (2 * s)) & 0x03030303u;
#pragma unroll
        for (int j = 0; j < 4; ++j) f[16 * k + 4 * j + s] = ubyte(x, j);
      }
  } else {
    static_for<32>([&](auto i) { f[i.value] = float(code_at<BITS, i.value>(w)); });
  }
}

// mlx::dequantize for bf16: bf16(bf16(scale * code) + bias), two codes at a
// time; out[i] holds codes 2i (low half) and 2i + 1. scale * code is exact in
// f32 (8-bit by at most 8-bit significands), so each rounding is a single
// RNE conversion, as in MLX's bf16 arithmetic.
template <int BITS>
__device__ __forceinline__ void dequant_run(const uint32_t* w, uint32_t sb, uint32_t* out) {
  float f[32];
  run_codes<BITS>(w, f);
  const float s = __uint_as_float(sb << 16), bias = __uint_as_float(sb & 0xffff0000u);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t m = pack_bf16(s * f[2 * i], s * f[2 * i + 1]);
    out[i] = pack_bf16(__uint_as_float(m << 16) + bias, __uint_as_float(m & 0xffff0000u) + bias);
  }
}

// Writes a K task into LDS: row `key` of K at channels [32 run, 32 run + 32).
// Keys past the end are zero (their scores are masked).
template <int D, int BITS, int NW>
__device__ __forceinline__ void store_k(const Stage<NW>& st, uint16_t* Ks, int key, int run) {
  constexpr int KSTR = kKStride<D>;
  uint32_t v[16];
  if (st.ok) {
    dequant_run<BITS>(st.w, st.s | (st.b << 16), v);
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = 0u;
  }
  u32x4_t* d = reinterpret_cast<u32x4_t*>(Ks + key * KSTR + run * 32);
#pragma unroll
  for (int i = 0; i < 4; ++i) d[i] = u32x4_t{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
}

// Writes a V task into column `key` of V^T, channels [32 run, 32 run + 32).
// Keys past the end are zero (0 * v stays finite).
template <int D, int BITS, int NW>
__device__ __forceinline__ void store_v(const Stage<NW>& st, uint16_t* Vt, int key, int run) {
  constexpr int VSTR = kVStride;
  uint32_t v[16];
  if (st.ok) {
    dequant_run<BITS>(st.w, st.s | (st.b << 16), v);
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = 0u;
  }
  uint16_t* d = Vt + (run * 32) * VSTR + key;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    d[(2 * i) * VSTR] = uint16_t(v[i]);
    d[(2 * i + 1) * VSTR] = uint16_t(v[i] >> 16);
  }
}

// Two wavefronts per SIMD (at most 256 registers a lane): one wavefront's
// softmax and dequantization then overlap the other's matrix-core work.
template <int D, int BK, int BV>
__global__ __launch_bounds__(Shape<D>::kWaves* kWave) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_affine_kernel(const Args a) {
  constexpr int kWaves = Shape<D>::kWaves, RW = Shape<D>::kRW, kRows = Shape<D>::kRows;
  constexpr int NR = RW / 16, ND = D / 32, NT = D / 16;
  constexpr int KSTR = kKStride<D>, VSTR = kVStride;
  constexpr int kPer = Shape<D>::kPer, kThreads = Shape<D>::kThreads;
  constexpr int NW = BK > BV ? BK : BV;
  // Two tile buffers: tile t is read from one while tile t + 1 is written
  // into the other, so a tile costs one barrier.
  __shared__ __attribute__((aligned(16))) uint16_t Ks2[2][kTile * KSTR];
  __shared__ __attribute__((aligned(16))) uint16_t Vt2[2][D * VSTR];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave, lr = lane % 16, lg = lane / 16;
  // Workgroup i runs on XCD i % 8 (round-robin dispatch). Consecutive
  // logical blocks, which share a (batch row, KV head) and so its keys, are
  // placed on one XCD's L2; within a unit the longest key ranges go first.
  const int n_wg = int(gridDim.x);
  int lin = int(blockIdx.x);
  if (n_wg % kXcds == 0) lin = (lin % kXcds) * (n_wg / kXcds) + lin / kXcds;
  const int blk = a.n_blocks - 1 - lin % a.n_blocks;
  const int kvh = (lin / a.n_blocks) % a.H_kv, b = lin / (a.n_blocks * a.H_kv);
  const int64_t rows = int64_t(a.L) * a.G;
  const int64_t row0 = int64_t(blk) * kRows;
  const int64_t row_end = row0 + kRows < rows ? row0 + kRows : rows;
  const int64_t qa_lo = a.q_start + row0 / a.G, qa_hi = a.q_start + (row_end - 1) / a.G;

  // Visible key indices of the block.
  int64_t kk_lo = 0, kk_hi = a.total - 1;
  if (a.causal) {
    if (qa_hi - a.k_start < kk_hi) kk_hi = qa_hi - a.k_start;
    if (a.window >= 0 && qa_lo - a.window + 1 - a.k_start > kk_lo)
      kk_lo = qa_lo - a.window + 1 - a.k_start;
  }

  bf8_t qf[NR][ND];
  int64_t qabs[NR], orow[NR];
  bool rvalid[NR];
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    const int64_t r = row0 + wave * RW + 16 * j + lr;
    rvalid[j] = r < rows;
    const int64_t rr = rvalid[j] ? r : rows - 1;
    const int64_t l = rr / a.G, g = rr % a.G;
    qabs[j] = a.q_start + l;
    orow[j] = ((int64_t(b) * a.H + int64_t(kvh) * a.G + g) * a.L + l) * D;
#pragma unroll
    for (int s = 0; s < ND; ++s)
      qf[j][s] = *reinterpret_cast<const bf8_t*>(a.q + orow[j] + 32 * s + 8 * lg);
  }

  float m[NR], lsum[NR];
  f4_t o[NT][NR];
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    m[j] = -INFINITY;
    lsum[j] = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }

  if (kk_lo <= kk_hi) {
    const int64_t t_lo = kk_lo / kTile, t_hi = kk_hi / kTile;
    const SlabPtrs kp = slabs_for<D, BK>(a.seg[0], a.seg[1], a.seg[0].kw, a.seg[1].kw,
                                         a.seg[0].ks, a.seg[1].ks, a.seg[0].kb, a.seg[1].kb,
                                         a.gs, b, kvh);
    const SlabPtrs vp = slabs_for<D, BV>(a.seg[0], a.seg[1], a.seg[0].vw, a.seg[1].vw,
                                         a.seg[0].vs, a.seg[1].vs, a.seg[0].vb, a.seg[1].vb,
                                         a.gs, b, kvh);
    // Task i of this thread: tid + i * kThreads; the first 2D tasks are K
    // runs, the rest V runs (a whole wavefront takes one kind, so the kind
    // and its pointers are uniform).
    Stage<NW> st[kPer];
    SlabPtrs tp[kPer];
    bool tv[kPer];
    int tkey[kPer], trun[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int task = tid + i * kThreads, r = task % (2 * D);
      tv[i] = wave * kWave + i * kThreads >= 2 * D;
      tkey[i] = r % kTile;
      trun[i] = r / kTile;
      tp[i].w0 = tv[i] ? vp.w0 : kp.w0;
      tp[i].w1 = tv[i] ? vp.w1 : kp.w1;
      tp[i].s0 = tv[i] ? vp.s0 : kp.s0;
      tp[i].s1 = tv[i] ? vp.s1 : kp.s1;
      tp[i].b0 = tv[i] ? vp.b0 : kp.b0;
      tp[i].b1 = tv[i] ? vp.b1 : kp.b1;
    }
#define TQKV_LOAD_TILE(T)                                                        \
  _Pragma("unroll") for (int i = 0; i < kPer; ++i) {                             \
    if (tv[i])                                                                   \
      load_stage<D, BV>(st[i], tp[i], a, (T) * kTile + tkey[i], trun[i]);        \
    else                                                                         \
      load_stage<D, BK>(st[i], tp[i], a, (T) * kTile + tkey[i], trun[i]);        \
  }
#define TQKV_STORE_TILE(BUF)                                                     \
  _Pragma("unroll") for (int i = 0; i < kPer; ++i) {                             \
    if (tv[i])                                                                   \
      store_v<D, BV>(st[i], Vt2[BUF], tkey[i], trun[i]);                         \
    else                                                                         \
      store_k<D, BK>(st[i], Ks2[BUF], tkey[i], trun[i]);                         \
  }
    TQKV_LOAD_TILE(int(t_lo))
    // Everything loaded so far (the Q fragments, the first tile) has landed:
    // without this the compiler's loop-carried wait analysis keeps the Q
    // loads pending and makes every tile's MFMAs wait for the next tile's
    // prefetch. (vmcnt(0); expcnt and lgkmcnt unchanged.)
    __builtin_amdgcn_s_waitcnt(0x0F70);
    TQKV_STORE_TILE(0)
    if (t_lo < t_hi) {
      TQKV_LOAD_TILE(int(t_lo) + 1)
    }
    __syncthreads();
    // The two wavefronts on a SIMD (w and w + kWaves / 2) take the tile's
    // work in opposite orders, so one's dequantization (VALU) runs while the
    // other's products (MFMA) do.
    const bool dequant_first = wave >= kWaves / 2;
    int cur = 0;
    for (int t = int(t_lo); t <= int(t_hi); ++t, cur ^= 1) {
      // Tile t + 1 into the other buffer (last read in iteration t - 1,
      // before the barrier that ended it), then fetch tile t + 2.
      if (dequant_first && t < t_hi) {
        TQKV_STORE_TILE(cur ^ 1)
        if (t + 1 < t_hi) {
          TQKV_LOAD_TILE(t + 2)
        }
      }
      const uint16_t* Ks = Ks2[cur];
      const uint16_t* Vt = Vt2[cur];

      f4_t sc[4][NR];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NR; ++j) sc[i][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < ND; ++s)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bf8_t ka = *reinterpret_cast<const bf8_t*>(Ks + (16 * i + lr) * KSTR + 32 * s + 8 * lg);
#pragma unroll
          for (int j = 0; j < NR; ++j)
            sc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qf[j][s], sc[i][j], 0, 0, 0);
        }

      // Mask: only on tiles some row of the block sees in part. Key offset
      // o in the tile is visible to a row iff lo <= o <= hi.
      const int64_t kbase = a.k_start + int64_t(t) * kTile;
      const int rem = a.total - int64_t(t) * kTile < kTile ? int(a.total - int64_t(t) * kTile) : kTile;
      const bool full = rem == kTile &&
                        (!a.causal || (kbase + kTile - 1 <= qa_lo &&
                                       (a.window < 0 || qa_hi < kbase + a.window)));
      if (!full) {
#pragma unroll
        for (int j = 0; j < NR; ++j) {
          int hi = rem - 1, lo = 0;
          if (a.causal) {
            const int64_t dq = qabs[j] - kbase;  // the row's own offset
            if (dq < hi) hi = dq < -1 ? -1 : int(dq);
            if (a.window >= 0) {
              const int64_t first = dq - a.window + 1;
              lo = first < 0 ? 0 : (first > kTile ? kTile : int(first));
            }
          }
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int o = 16 * i + 4 * lg + r;
              if (o < lo || o > hi) sc[i][j][r] = -INFINITY;
            }
        }
      }
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sc[i][j][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        mx *= a.qscale;  // qscale > 0: the max of the scaled scores
        const bool up = mx > m[j] + kTau;
        if (__any(up)) {
          const float mn = up ? mx : m[j];
          const float alpha = up ? __builtin_amdgcn_exp2f(m[j] - mn) : 1.0f;
          lsum[j] *= alpha;
#pragma unroll
          for (int t2 = 0; t2 < NT; ++t2) o[t2][j] *= alpha;
          m[j] = mn;
        }
        const float nm = m[j] == -INFINITY ? 0.0f : -m[j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            sc[i][j][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i][j][r], a.qscale, nm));
      }

      const bf2_t kOnes = {__bf16(1.0f), __bf16(1.0f)};
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        bf8_t pb[NR];
#pragma unroll
        for (int j = 0; j < NR; ++j) {
          const f4_t p0 = sc[2 * u][j], p1 = sc[2 * u + 1][j];
          const u32x4_t w = {pack_bf16(p0[0], p0[1]), pack_bf16(p0[2], p0[3]),
                             pack_bf16(p1[0], p1[1]), pack_bf16(p1[2], p1[3])};
          pb[j] = __builtin_bit_cast(bf8_t, w);
          // The row sum counts the weights as rounded for the matrix cores,
          // so the output stays an exact convex combination of them.
#pragma unroll
          for (int e = 0; e < 4; ++e)
            lsum[j] = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(w[e]), kOnes, lsum[j], false);
        }
#pragma unroll
        for (int t2 = 0; t2 < NT; ++t2) {
          const uint16_t* vrow = Vt + (16 * t2 + lr) * VSTR + 32 * u + 4 * lg;
          const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(vrow);
          const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(vrow + 16);
          const bf8_t va = __builtin_bit_cast(bf8_t, u32x4_t{lo.x, lo.y, hi.x, hi.y});
#pragma unroll
          for (int j = 0; j < NR; ++j)
            o[t2][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[j], o[t2][j], 0, 0, 0);
        }
      }

      if (!dequant_first && t < t_hi) {
        TQKV_STORE_TILE(cur ^ 1)
        if (t + 1 < t_hi) {
          TQKV_LOAD_TILE(t + 2)
        }
      }
      __syncthreads();
    }
  }
#undef TQKV_STORE_TILE

#undef TQKV_LOAD_TILE
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    float tot = lsum[j];
    tot += __shfl_xor(tot, 16, kWave);
    tot += __shfl_xor(tot, 32, kWave);
    const float inv = tot > 0.0f ? 1.0f / tot : 0.0f;
    if (rvalid[j]) {
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2) {
        const f4_t v = o[t2][j] * inv;
        *reinterpret_cast<u32x2_t*>(a.out + orow[j] + 16 * t2 + 4 * lg) =
            u32x2_t{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])};
      }
    }
  }
}

typedef void (*KernelFn)(Args);

// The kernel for (D, bits_k, bits_v), bits in {2, 3, 4, 5, 6, 8}; null if
// unsupported.
KernelFn pick_d64(int bk, int bv);
KernelFn pick_d128(int bk, int bv);
KernelFn pick_d256(int bk, int bv);

template <int D, int BK>
KernelFn pick_bv(int bv) {
  switch (bv) {
    case 2: return prefill_affine_kernel<D, BK, 2>;
    case 3: return prefill_affine_kernel<D, BK, 3>;
    case 4: return prefill_affine_kernel<D, BK, 4>;
    case 5: return prefill_affine_kernel<D, BK, 5>;
    case 6: return prefill_affine_kernel<D, BK, 6>;
    case 8: return prefill_affine_kernel<D, BK, 8>;
  }
  return nullptr;
}

template <int D>
KernelFn pick_for(int bk, int bv) {
  switch (bk) {
    case 2: return pick_bv<D, 2>(bv);
    case 3: return pick_bv<D, 3>(bv);
    case 4: return pick_bv<D, 4>(bv);
    case 5: return pick_bv<D, 5>(bv);
    case 6: return pick_bv<D, 6>(bv);
    case 8: return pick_bv<D, 8>(bv);
  }
  return nullptr;
}

}  // namespace prefill
}  // namespace tqkv
