// Prefill-chunk attention over affine-packed K/V on the matrix cores.
//
// What it computes (the reference's dequantized_prefill_attention,
// gemma4_moe.rs:2382-2411): K and V are dequantized the way mlx::dequantize
// does for bf16 (scale * code + bias as one f32 multiply-add, rounded once
// to bf16), then softmax(scale * Q K^T + mask) V with f32 accumulation.
// Operands of the prefill variant: Q K^T in bf16 (the products of bf16
// values are exact in f32), P V in f16: the weights P and the dequantized
// bf16 values of V, the latter scaled by 2^-kVShift so |v| up to 2^24
// stays inside f16's range (the output scales back). f16 weights carry 11
// significant bits where the reference's bf16 SDPA rounds them to 8, so the
// output stays within the f32-level band of the exact result. The f16
// variant (decode over a shared prefix, head dim 512 decode) takes every
// operand in f16.
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
// codes of one key (bits words) for K and for V, dequantize it and write
// both row-major [key][D] into LDS; the next tile's
// words are fetched into registers while the matrix cores work on this one.
// Each wavefront owns RW query rows:
//   S^T = K . Q^T: A = K rows from LDS (ds_read_b128), B = the wavefront's Q
//   rows held in registers for the whole kernel; lane l ends up with the
//   scores of query row l % 16 for keys 16i + 4(l / 16) + r.
//   Online softmax per row: the running maximum may lag the true one by up
//   to kTau (log2 units), so the O accumulators are rescaled only when some
//   row moves by more; a lane compares its own 16-key maximum with the
//   row's threshold, and only when some lane passes it are the row's lanes
//   combined (two lane exchanges, l ^ 16 and l ^ 32). Row sums (of the
//   f16-rounded weights, one v_dot2 per pair) stay per lane until the end.
//   O^T += V^T . P^T: the score registers of key tiles 2u and 2u + 1 are,
//   rounded to f16, exactly the B operand (k slot 8(l / 16) + s holds key
//   32u + 4(l / 16) + s, s < 4, or 32u + 16 + 4(l / 16) + s - 4); the A
//   operand takes the same keys of V^T from the row-major V tile with two
//   transposing ds_read_b64_tr_b16 (the V stores are four 16-byte stores a
//   run, where a transposed tile took 32 two-byte stores).
// Keys dequantized beforehand (widths 16, 17, 18 below) skip the
// dequantization: the loader copies their rows. With V^T tiles (width 18,
// D = 128) the tiles go from HBM straight into LDS two tiles ahead, and
// the A operand of P V is one 16-byte read.
// Only tiles that some row of the block can see are visited, and the
// per-element mask runs only on tiles that are not wholly visible.
#pragma once

#include <cmath>
#include <type_traits>
#include <utility>

#include "common.hpp"

namespace tqkv {
namespace prefill {

constexpr int kWave = 64;
constexpr int kTile = 64;  // keys per tile
constexpr int kXcds = 8;   // accelerator dies (each with its own L2) on MI355X
// LDS row stride (16-bit elements) of the K and V tiles, both row-major
// [key][D]. D + 16 (rows 32 bytes past a multiple of 128) leaves both reads
// of the products free of bank conflicts, as counted on gfx950
// (SQ_LDS_BANK_CONFLICT of each access pattern alone): the K operand's
// ds_read_b128 (16 rows x 2 chunks a half-wavefront) and V's transposing
// ds_read_b64_tr_b16 (8 rows x 32 bytes a half-wavefront). The loader's
// 16-byte stores (64 consecutive rows, one chunk) then conflict 2-way; D + 8
// made the stores conflict-free but cost 4 cycles per K read and 2 per V
// read, 4x more conflict cycles a tile.
template <int D>
constexpr int kKStride = D + 16;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kTau = 8.0f;
// V operands of the prefill variant hold v * 2^-kVShift in f16: |v| below
// 65504 * 2^8 (about 1.68e7) fits, and values under 2^-6 in magnitude, which
// become f16 subnormals, move by at most 2^-17.
constexpr int kVShift = 8;
constexpr float kVDown = 1.0f / float(1 << kVShift);
constexpr float kVUp = float(1 << kVShift);

typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
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
  const uint16_t* q;  // bf16; row (b, h, l) at b * qs_b + h * qs_h + l * qs_l
  uint16_t* out;      // bf16, same strides as q (normalized output mode)
  int64_t qs_b, qs_h, qs_l;
  int H, H_kv, G, L, gs;
  int n_blocks;   // row blocks per (batch row, KV head)
  int causal;
  float qscale;   // softmax scale * log2(e)
  Seg seg[2];
  int64_t n0, total;  // keys in segment 0; keys in all
  int64_t q_start, k_start, window;
  // Key splits: split s covers keys [s * split_len, (s + 1) * split_len).
  // With part_o set, a row's (o unnormalized, max in log2 units, sum) go to
  // slot split_base + s of n_part, row index (b * L + l) * H + h.
  int n_splits, split_len, split_base, n_part;
  float* part_o;
  float* part_m;
  float* part_l;
};

// Launch shape per head dim: wavefronts per workgroup and query rows per
// wavefront. More rows a workgroup spread the dequantization of a tile over
// more matrix-core work; the O accumulators (RW rows x D channels a
// wavefront) and two wavefronts per SIMD bound RW; D = 256 stays at 128 rows.
// Loader tasks: 64 keys x D/32 runs x {K, V}, kPer a thread.
// The f16 variant serves decode over a shared prefix, where a block holds
// only the B x G query rows of a KV head: 16 rows a wavefront there spread
// those rows' products over more SIMDs.
// D = 512 (Gemma 4's global layers): one LDS tile buffer (two would pass
// the 160 KB of LDS), so a tile costs two barriers, and four wavefronts, one
// a SIMD, so each holds its 512 O accumulators a row in the whole register
// file.
template <int D, bool H16>
struct Shape {
  static constexpr int kWaves = (D == 64 || D == 512) ? 4 : 8;
  static constexpr int kRW = (D >= 256 || H16) ? 16 : 32;
  // D = 512 with f16 operands (decode: a sequence's heads at one position)
  // splits the output channels instead of the rows: every wavefront takes
  // the block's rows, scores all of D, and accumulates a quarter of the
  // channels (its O accumulators fit the register file; one wavefront
  // holding all 512 spilled).
  static constexpr bool kChanSplit = H16 && D == 512;
  // D <= 256 with f16 operands (decode over a shared prefix: a block holds
  // a KV head's B x G query rows, 32 at config 4) splits the keys instead:
  // the wavefronts form groups of 16 rows times kKQ quarters of every 64-key
  // tile, so every wavefront carries scores and products (with whole
  // 16-row slices, two of eight did and bounded the pass); the quarters'
  // softmax states meet in LDS at the end.
  static constexpr bool kKeySplit = H16 && D <= 256;
  static constexpr int kKQ = kKeySplit ? 4 : 1;
  static constexpr int kRows = kChanSplit ? kRW : kWaves / kKQ * kRW;
  static constexpr int kThreads = kWaves * 64;
  static constexpr int kPer = 4 * D / kThreads;
  // Tiles whose raw words are in flight in registers while a tile is
  // computed. The f16 (decode) variant serves few query rows, so a tile's
  // compute is short and the loads must run further ahead to keep HBM busy
  // (one set at D = 512, where two measured slower).
  static constexpr int kSets = H16 && D <= 256 ? 2 : 1;
  static constexpr int kBufs = D == 512 ? 1 : 2;      // LDS tile buffers
  static constexpr int kWavesPerEu = D == 512 ? 1 : 2;
  // The bf16 prefill at D = 128 (two wavefronts a SIMD, 32 rows each):
  // the second wavefront of each SIMD (waves kWaves / 2..) multiplies a
  // tile's P by V one tile late, before the next tile's scores. Both
  // wavefronts of a SIMD leave each tile's barrier together; in this order
  // one's softmax (VALU) meets the other's products (matrix cores) instead
  // of both doing the same phase at once (measured on gfx950: a wavefront
  // issuing back-to-back products leaves the other on its SIMD about one
  // v_exp_f32 or two FMAs per product). A strict two-phase ping-pong (a
  // barrier between products and softmax) measured slower: a wavefront's
  // own LDS reads then stall its products with nothing to fill the gap.
  // V needs three LDS buffers (tile t - 1 read late, t read, t + 1
  // written); D = 256 has no room for them.
  static constexpr bool kDeferPV = !H16 && D == 128;
  static constexpr int kVBufs = kDeferPV ? 3 : kBufs;
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

__device__ __forceinline__ uint32_t pack_h16(float lo, float hi) {
  const f2_t f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, h2_t));
}
__device__ __forceinline__ h2_t as_h2(uint32_t x) { return __builtin_bit_cast(h2_t, x); }

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
};

// Width 16 stands for keys dequantized beforehand: rows of D bf16 values
// (mlx::dequantize's bits; bf16 caches; codebook rows). Width 17: rows of D
// f16 values already in the prefill variant's V operand form (bf16 values
// times 2^-kVShift, written once per (batch row, KV head) by
// dequantize_rows_kernel), which the loaders copy into LDS as they are.
// Width 18 (D = 128): the same V operands as transposed 64-key tiles, the
// slab padded to whole tiles (zeros past the last key). Tile t is 2 D rows
// of 32 values: row u D + c holds channel c of keys 64 t + 32 u + [0, 32)
// in the order of the P operand's k slots (slot 8 g + s: key 4 g + s for
// s < 4, 16 + 4 g + s - 4 else), so the products read V^T with one 16-byte
// LDS read where the row-major tile takes two transposing reads.
constexpr int kPreBits = 16;
constexpr int kPreF16 = 17;
constexpr int kPreF16T = 18;
template <int BITS>
constexpr bool is_rows() { return BITS == kPreBits || BITS == kPreF16 || BITS == kPreF16T; }
// The V^T variant (width 16 K rows with width 18 V^T tiles, D = 128) loads
// its tiles from HBM straight into LDS
// (global_load_lds_dwordx4: each 16-byte lane load lands at the wavefront's
// LDS base + 16 x lane, so a load instruction fills 1 KB of LDS in lane
// order, and the loader picks each lane's source). The tiles sit in LDS
// unpadded, 16-byte chunks permuted within their rows so that the operand
// reads are conflict-free under gfx950's bank rules (16-byte reads served
// 32 lanes at a time over 128 dword banks): K row r (256 bytes) keeps its
// chunk c at position c ^ (r mod 16); V^T row R (64 bytes) keeps chunk c
// at c ^ (2 x bit 3 of R).
__device__ __forceinline__ uint32_t k_chunk_pos(uint32_t r, uint32_t c) { return c ^ (r & 15u); }
__device__ __forceinline__ uint32_t vt_chunk_pos(uint32_t R, uint32_t c) { return c ^ (((R >> 3) & 1u) << 1); }
// The LDS address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}
// One global_load_lds_dwordx4: 16 bytes from each lane's src to LDS
// [lds + 16 lane, lds + 16 lane + 16). Written as assembly so that the
// compiler does not treat every later LDS read of the tile array as
// waiting on it (it cannot tell the tile buffers apart); the kernel waits
// for these loads itself (s_waitcnt vmcnt) before the barrier that
// publishes the tile. M0 carries the LDS base; the kernels that use this set nothing
// else in M0. An SALU write of M0 needs one wait state before an LDS DMA
// reads it (the s_nop; the compiler pads the same way for its own).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // M0 in the clobbers: see above
__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src),
               "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop
// 32-bit words of a loader task's run of 32 values.
template <int BITS>
constexpr int run_words() { return is_rows<BITS>() ? 16 : BITS; }
static_assert(run_words<kPreBits>() == 16 && run_words<kPreF16>() == 16 && run_words<3>() == 3,
              "a run of 32 16-bit values is 16 words; a row of D is D / 2");

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
  // Words a row: D * BITS / 32 for codes, D / 2 for rows of 16-bit values.
  constexpr int kRowWords = D * run_words<BITS>() / 32;
  return SlabPtrs{w0 + r0 * kRowWords, w1 + r1 * kRowWords, sc0 + r0 * groups,
                  sc1 + r1 * groups,         bi0 + r0 * groups,         bi1 + r1 * groups};
}

// Loads run `run` of key kk (counted across both segments) of K or V. A key
// past the end loads the last key instead, so the load is issued
// unconditionally; the tile keeps that key's (finite) values, which every
// consumer masks: its scores are -inf, so its weight is exactly 0.
template <int D, int BITS, int NW>
__device__ __forceinline__ void load_stage(Stage<NW>& st, const SlabPtrs& p, const Args& a, int kk,
                                           int run) {
  kk = min(kk, int(a.total) - 1);  // 32-bit: a cache holds fewer than 2^31 keys
  if constexpr (is_rows<BITS>()) {  // one segment of 16-bit rows, no scales
    load_words<16>(st.w, p.w0 + (uint32_t(kk) * (D / 2) + run * 16));
    st.s = st.b = 0u;
  } else {
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


// Dequantization of a run, two codes at a time; out[i] holds codes 2i (low
// half) and 2i + 1. bf16: mlx::dequantize, bf16(fma(scale, code, bias)):
// one multiply-add in f32 (the product is exact, 8-bit by at most 8-bit
// significands) and one RNE conversion, as MLX's kernel computes it.
// f16: scale * code + bias in f32 (one rounding), then to f16.
// f16 dequantization of 8- and 4-bit runs in packed f16 arithmetic, two
// codes an instruction: a byte permute puts code c under the f16 exponent of
// 1024 (bits 0x6400 | c is 1024 + c exactly; a 4-bit pair's high code lands
// as 1024 + 16 c), one packed FMA takes the offset off exactly, and one more
// gives s * c + b rounded once to f16. Scale and bias convert exactly from
// bf16 to f16 in f16's normal range.
template <int BITS>
__device__ __forceinline__ void dequant_run_h16(const uint32_t* w, uint32_t sb, uint32_t* out) {
  const _Float16 s = _Float16(__uint_as_float(sb << 16));
  const _Float16 bias = _Float16(__uint_as_float(sb & 0xffff0000u));
  const h2_t s2 = {s, s}, b2 = {bias, bias};
  constexpr uint32_t kExp = 0x64646464u;
  if constexpr (BITS == 8) {
    const h2_t one = {_Float16(1.0f), _Float16(1.0f)};
    const h2_t off = {_Float16(-1024.0f), _Float16(-1024.0f)};
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t sel = (4u + 2 * j) | ((5u + 2 * j) << 16);
        const h2_t c = __builtin_elementwise_fma(as_h2(__builtin_amdgcn_perm(w[k], kExp, sel)),
                                                 one, off);
        out[2 * k + j] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, s2, b2));
      }
  } else {
    static_assert(BITS == 4, "packed f16 dequantization takes 8- or 4-bit codes");
    const h2_t mul = {_Float16(1.0f), _Float16(0.0625f)};
    const h2_t off = {_Float16(-1024.0f), _Float16(-64.0f)};
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t sel = (4u + j) | ((4u + j) << 16);
        const uint32_t x = __builtin_amdgcn_perm(w[k], kExp, sel) & 0x64F0640Fu;
        const h2_t c = __builtin_elementwise_fma(as_h2(x), mul, off);
        out[4 * k + j] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(c, s2, b2));
      }
  }
}

template <int BITS, bool H16>
__device__ __forceinline__ void dequant_run(const uint32_t* w, uint32_t sb, uint32_t* out) {
  if constexpr (BITS == kPreBits) {  // already bf16
    static_assert(!H16, "dequantized rows are bf16");
#pragma unroll
    for (int i = 0; i < 16; ++i) out[i] = w[i];
  } else if constexpr (BITS == kPreF16) {
    static_assert(BITS != kPreF16, "f16 rows are V operands only");
  } else if constexpr (H16 && (BITS == 8 || BITS == 4)) {
    dequant_run_h16<BITS>(w, sb, out);
  } else {
    float f[32];
    run_codes<BITS>(w, f);
    const float s = __uint_as_float(sb << 16), bias = __uint_as_float(sb & 0xffff0000u);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if constexpr (H16) {
        out[i] = pack_h16(s * f[2 * i] + bias, s * f[2 * i + 1] + bias);
      } else {
        out[i] = pack_bf16(fmaf(s, f[2 * i], bias), fmaf(s, f[2 * i + 1], bias));
      }
    }
  }
}

// Writes a K task into LDS: row `key` of K at channels [32 run, 32 run + 32).
template <int D, int BITS, bool H16, int NW>
__device__ __forceinline__ void store_k(const Stage<NW>& st, uint16_t* Ks, int key, int run) {
  constexpr int KSTR = kKStride<D>;
  uint32_t v[16];
  dequant_run<BITS, H16>(st.w, st.s | (st.b << 16), v);
  u32x4_t* d = reinterpret_cast<u32x4_t*>(Ks + key * KSTR + run * 32);
#pragma unroll
  for (int i = 0; i < 4; ++i) d[i] = u32x4_t{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
}

// Writes a V task into LDS like a K task: row `key` of V, channels
// [32 run, 32 run + 32), four 16-byte stores. The products read V^T from it
// with gfx950's transposing ds_read_b64_tr_b16.
// The prefill variant's V operands of a run: mlx::dequantize's bf16 value
// times 2^-kVShift, as f16 (exact from the bf16 value wherever the product
// is an f16 normal). The scale and bias are scaled first, which scales the
// fused multiply-add's result exactly, and the bf16 rounding commutes with
// the power of two.
template <int BITS>
__device__ __forceinline__ void v_operand_run(const uint32_t* w, uint32_t sb, uint32_t* out) {
  if constexpr (BITS == kPreF16) {
#pragma unroll
    for (int i = 0; i < 16; ++i) out[i] = w[i];
  } else if constexpr (BITS == kPreBits) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      out[i] = pack_h16(__uint_as_float(w[i] << 16) * kVDown,
                        __uint_as_float(w[i] & 0xffff0000u) * kVDown);
  } else {
    float f[32];
    run_codes<BITS>(w, f);
    const float s = __uint_as_float(sb << 16) * kVDown;
    const float bias = __uint_as_float(sb & 0xffff0000u) * kVDown;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t m = pack_bf16(fmaf(s, f[2 * i], bias), fmaf(s, f[2 * i + 1], bias));
      out[i] = pack_h16(__uint_as_float(m << 16), __uint_as_float(m & 0xffff0000u));
    }
  }
}

template <int D, int BITS, bool H16, int NW>
__device__ __forceinline__ void store_v(const Stage<NW>& st, uint16_t* Vs, int key, int run) {
  if constexpr (H16) {
    store_k<D, BITS, H16>(st, Vs, key, run);
  } else {
    constexpr int KSTR = kKStride<D>;
    uint32_t v[16];
    v_operand_run<BITS>(st.w, st.s | (st.b << 16), v);
    u32x4_t* d = reinterpret_cast<u32x4_t*>(Vs + key * KSTR + run * 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) d[i] = u32x4_t{v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]};
  }
}

// The V tasks' stage registers: their own set, or the K tasks' set.
template <bool Split, typename K, typename V>
__device__ __forceinline__ decltype(auto) v_stages(K& k, V& v) {
  if constexpr (Split)
    return (v);
  else
    return (k);
}

// The 16x16x32 matrix-core product of the variant's operand type.
template <bool H16, typename V>
__device__ __forceinline__ f4_t mma(V a, V b, f4_t c) {
  if constexpr (H16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// gfx950's transposing LDS read: the 16 lanes of a group each name 4
// consecutive 16-bit values of a 4 x 16 block (lane i: row i / 4, columns
// 4 (i % 4) + [0, 4)); lane i receives column i of the block's 4 rows.
typedef short s4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2_t tr_read(const uint16_t* p) {
  const s4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s4_t*)(p));
  return __builtin_bit_cast(u32x2_t, v);
}

// Marks a block that runs on few tiles (the element mask of partially
// visible tiles, the accumulator rescale when a row's maximum moves): with
// it the compiler keeps the block behind its wave-uniform branch instead of
// turning it into selects that every tile executes (measured: ~190 of ~380
// VALU instructions a tile at head dim 128).
__device__ __forceinline__ void keep_branch() { asm volatile(""); }

// acc + both halves of a packed pair (v_dot2 against a (1, 1) splat).
template <bool H16>
__device__ __forceinline__ float sum2(uint32_t w, float acc) {
  if constexpr (H16) {
    const h2_t one = {_Float16(1.0f), _Float16(1.0f)};
    return __builtin_amdgcn_fdot2(as_h2(w), one, acc, false);
  } else {
    const bf2_t one = {__bf16(1.0f), __bf16(1.0f)};
    return __builtin_amdgcn_fdot2_f32_bf16(as_bf2(w), one, acc, false);
  }
}

// Lane l combined with lane l ^ 16 (l ^ 32): gfx950's v_permlane16_swap
// (v_permlane32_swap) of a value with itself returns the lane's and its
// partner's halves, with no LDS round trip (a ds_bpermute shuffle would sit
// on the path from the scores to the softmax).
// The maximum of two scores as one v_max_f32: fmaxf on the swapped values
// costs a v_max_f32 x, x (NaN quieting) on each first, which finite
// scores never need.
__device__ __forceinline__ float max_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return max_raw(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return max_raw(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Two wavefronts per SIMD (at most 256 registers a lane): one wavefront's
// softmax and dequantization then overlap the other's matrix-core work
// (D = 512: one, with the whole register file).
template <int D, int BK, int BV, bool H16>
__global__ __launch_bounds__((Shape<D, H16>::kThreads))
__attribute__((amdgpu_waves_per_eu(Shape<D, H16>::kWavesPerEu)))
void prefill_affine_kernel(const Args a) {
  constexpr int kWaves = Shape<D, H16>::kWaves, RW = Shape<D, H16>::kRW, kRows = Shape<D, H16>::kRows;
  constexpr int NR = RW / 16, ND = D / 32;
  constexpr bool CS = Shape<D, H16>::kChanSplit;
  // Key split: this wavefront's row group rg and key quarter kq (rows
  // rg * RW + [0, RW), keys 16 kq + [0, 16) of every tile).
  constexpr bool KS = Shape<D, H16>::kKeySplit;
  constexpr int KQ = Shape<D, H16>::kKQ, RG = kWaves / KQ;
  static_assert(!KS || RW == 16, "a key-split wavefront holds 16 rows");
  // Output channel tiles of 16 this wavefront accumulates, from t_base on;
  // RWO: rows between wavefronts (0 when they share the rows).
  constexpr int NT = CS ? D / 16 / kWaves : D / 16;
  constexpr int RWO = CS ? 0 : RW;
  // Channel-split scores: each wavefront reduces its quarter of D (NDW
  // k-steps from its own quarter of Q and K) and the four partial score
  // tiles meet in LDS, summed in wavefront order (the same bits in every
  // wavefront).
  constexpr int NDW = CS ? ND / kWaves : ND;
  constexpr int KSTR = kKStride<D>;
  constexpr int kPer = Shape<D, H16>::kPer, kThreads = Shape<D, H16>::kThreads;
  constexpr int kBufs = Shape<D, H16>::kBufs, kVBufs = Shape<D, H16>::kVBufs;
  constexpr bool kDeferPV = Shape<D, H16>::kDeferPV;
  // Two tile buffers: tile t is read from one while tile t + 1 is written
  // into the other, so a tile costs one barrier. One buffer (D = 512): tile
  // t + 1 is written after every wavefront has read tile t. Three V buffers
  // where P V runs one tile late on half the wavefronts.
  // K tiles then V tiles, one array: after the last tile the key split
  // merges its quarters' accumulators in the same memory.
  // V^T tiles (width 18; K bf16 rows with them): loaded straight into LDS,
  // unpadded, chunks permuted (k_chunk_pos, vt_chunk_pos).
  constexpr bool VT = BV == kPreF16T;
  static_assert(!VT || (D == 128 && BK == kPreBits && !H16 && !KS && !CS && kWaves == 8),
                "V^T tiles: the bf16 variant at D = 128");
  // (Buffers of one size, a two-dimensional array: with buffer offsets
  // computed from a flat array the compiler keeps more addresses live and
  // spills.)
  constexpr int kBufElems = VT ? kTile * D : kTile * KSTR;
  // The V^T variant loads two tiles ahead straight into LDS: three K and
  // four V buffers (112 KiB).
  constexpr int KBN = VT ? 3 : kBufs, VBN = VT ? 4 : kVBufs;
  __shared__ __attribute__((aligned(16))) uint16_t s_tiles[KBN + VBN][kBufElems];
  auto Ks2 = [&](int c) __attribute__((always_inline)) { return &s_tiles[c][0]; };
  auto Vt2 = [&](int c) __attribute__((always_inline)) { return &s_tiles[KBN + c][0]; };
  __shared__ float s_km[KS ? kWaves : 1][16], s_kl[KS ? kWaves : 1][16];
  __shared__ f4_t s_part[CS ? kWaves : 1][CS ? 4 : 1][kWave];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave, lr = lane % 16, lg = lane / 16;
  const int t_base = CS ? wave * NT : 0;
  const int s_base = CS ? wave * NDW : 0;
  const int kq = KS ? wave / RG : 0;
  // First row of this wavefront within the block.
  const int wrow = KS ? (wave % RG) * RW : wave * RWO;
  // Workgroup i runs on XCD i % 8 (round-robin dispatch). Consecutive
  // logical blocks, which share a (batch row, KV head) and so its keys, are
  // placed on one XCD's L2; within a unit the longest key ranges go first.
  const int n_wg = int(gridDim.x);
  int lin = int(blockIdx.x);
  if (n_wg % kXcds == 0) lin = (lin % kXcds) * (n_wg / kXcds) + lin / kXcds;
  const int per_unit = a.n_blocks * a.n_splits;
  const int blk = a.n_blocks - 1 - lin % a.n_blocks;
  const int split = (lin % per_unit) / a.n_blocks;
  const int kvh = (lin / per_unit) % a.H_kv, b = lin / (per_unit * a.H_kv);
  const int64_t rows = int64_t(a.L) * a.G;
  const int64_t row0 = int64_t(blk) * kRows;
  const int64_t row_end = row0 + kRows < rows ? row0 + kRows : rows;
  const int64_t qa_lo = a.q_start + row0 / a.G, qa_hi = a.q_start + (row_end - 1) / a.G;

  // Visible key indices of the block, within its split.
  int64_t kk_lo = int64_t(split) * a.split_len, kk_hi = a.total - 1;
  if (kk_lo + a.split_len - 1 < kk_hi) kk_hi = kk_lo + a.split_len - 1;
  if (a.causal) {
    if (qa_hi - a.k_start < kk_hi) kk_hi = qa_hi - a.k_start;
    if (a.window >= 0 && qa_lo - a.window + 1 - a.k_start > kk_lo)
      kk_lo = qa_lo - a.window + 1 - a.k_start;
  }

  using op8_t = std::conditional_t<H16, h8_t, bf8_t>;
  op8_t qf[NR][NDW];
  // Row slot j of this lane: row r of the block's (query, head) rows, held
  // as its query index within the chunk (ql, 32-bit; the Q and output row
  // offsets are recomputed where they are used, off the tile loop).
  int ql[NR];
  auto row_of = [&](int j) __attribute__((always_inline)) { return row0 + wrow + 16 * j + lr; };
  auto orow_of = [&](int64_t r) __attribute__((always_inline)) {
    const int64_t rr = r < rows ? r : rows - 1;
    const int64_t l = rr / a.G, g = rr % a.G;
    return int64_t(b) * a.qs_b + (int64_t(kvh) * a.G + g) * a.qs_h + l * a.qs_l;
  };
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    const int64_t r = row_of(j);
    const int64_t rr = r < rows ? r : rows - 1;
    ql[j] = int(rr / a.G);
    const int64_t orow = orow_of(r);
#pragma unroll
    for (int s = 0; s < NDW; ++s)
    {
      const bf8_t x =
          *reinterpret_cast<const bf8_t*>(a.q + orow + 32 * (s_base + s) + 8 * lg);
      if constexpr (H16) {
        // bf16 -> f16 is exact for |q| in f16's normal range.
#pragma unroll
        for (int e = 0; e < 8; ++e) qf[j][s][e] = _Float16(float(x[e]));
      } else {
        qf[j][s] = x;
      }
    }
  }

  // Per row slot: the running maximum m (log2 units), nm = -m (0 while no
  // key is visible) and thr, the raw score above which m must move (a tile
  // compares its raw maximum with it; all three change only on a rescale).
  float m[NR], nm[NR], thr[NR], lsum[NR];
  f4_t o[NT][NR];
  const float iqs = 1.0f / a.qscale;
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    m[j] = -INFINITY;
    nm[j] = 0.0f;
    thr[j] = -INFINITY;
    lsum[j] = 0.0f;
#pragma unroll
    for (int t = 0; t < NT; ++t) o[t][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }
  // A rescale of row slot j to the tile maximum mx (raw), on the lanes with
  // up set: the accumulators and sum scale by 2^(m - m'), then the state
  // moves. qscale > 0, so mx * qscale is the maximum of the scaled scores.
  auto rescale = [&](int j, bool up, float mx) __attribute__((always_inline)) {
    const float mn = up ? mx * a.qscale : m[j];
    const float alpha = up ? __builtin_amdgcn_exp2f(m[j] - mn) : 1.0f;
    lsum[j] *= alpha;
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2) o[t2][j] *= alpha;
    m[j] = mn;
    nm[j] = mn == -INFINITY ? 0.0f : -mn;
    thr[j] = (mn + kTau) * iqs;
  };

  if (kk_lo <= kk_hi) {
    const int64_t t_lo = kk_lo / kTile, t_hi = kk_hi / kTile;
    const SlabPtrs kp = slabs_for<D, BK>(a.seg[0], a.seg[1], a.seg[0].kw, a.seg[1].kw,
                                         a.seg[0].ks, a.seg[1].ks, a.seg[0].kb, a.seg[1].kb,
                                         a.gs, b, kvh);
    const SlabPtrs vp = slabs_for<D, BV>(a.seg[0], a.seg[1], a.seg[0].vw, a.seg[1].vw,
                                         a.seg[0].vs, a.seg[1].vs, a.seg[0].vb, a.seg[1].vb,
                                         a.gs, b, kvh);
    // Task i of this thread: tid + i * kThreads; the first 2D tasks are K
    // runs, the rest V runs.
    constexpr int NS = Shape<D, H16>::kSets;
    // K and V tasks keep their words in separate registers: with one shared
    // set the two load paths meet in register copies that must wait for the
    // loads to land, which would expose the full memory latency at issue.
    // (The bf16 prefill variant shares one set: it has no registers to
    // spare, and its long tiles hide the wait behind the other wavefront.)
    constexpr bool kSplit = H16;
    constexpr int WK = run_words<BK>(), WV = run_words<BV>();
    constexpr int NW = WK > WV ? WK : WV;
    Stage<kSplit ? WK : NW> stk[NS][kPer];
    Stage<kSplit ? WV : NW> stv_own[kSplit ? NS : 1][kPer];
    auto& stv = v_stages<kSplit>(stk, stv_own);
    // A task's kind (K or V run) goes by its index where 2D is a multiple of
    // the workgroup (the compiler then folds each task's pointers to K's or
    // V's: D = 512 holds 8 tasks a thread), else by wavefront, with one task
    // a thread.
    constexpr bool kKindByTask = (2 * D) % kThreads == 0;
    static_assert(kKindByTask || kPer == 1, "a kind by wavefront means one task a thread");
    int tkey[kPer], trun[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int task = tid + i * kThreads, r = task % (2 * D);
      tkey[i] = r % kTile;
      trun[i] = r / kTile;
    }
    // The two wavefronts on a SIMD (w and w + kWaves / 2) take the tile's
    // work in opposite orders, so one's dequantization (VALU) runs while the
    // other's products (MFMA) do.
    const bool dequant_first = wave >= kWaves / 2;
    const bool live = row0 + wrow < rows;
    // A key-split wavefront's share of tile t (buffer cur): S^T of its 16
    // keys by its 16 rows (D / 32 products), the online softmax over them,
    // and O^T += V^T P^T as D / 16 products of 16 x 16 x 16 whose k slots are
    // the 16 keys: the score registers are exactly the B operand, and one
    // transposing read gives the A operand of 4 keys x 16 channels a lane
    // group.
    auto ks_tile = [&](int64_t t, int cur, int vc) __attribute__((always_inline)) {
      if constexpr (KS) {
        const uint16_t* Ks = Ks2(cur);
        const uint16_t* Vt = Vt2(vc);
        f4_t sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s = 0; s < NDW; ++s) {
          const op8_t ka =
              *reinterpret_cast<const op8_t*>(Ks + (16 * kq + lr) * KSTR + 32 * s + 8 * lg);
          sc = mma<H16>(ka, qf[0][s], sc);
        }
        const int64_t kbase = a.k_start + int64_t(t) * kTile;
        const int rem = a.total - int64_t(t) * kTile < kTile ? int(a.total - int64_t(t) * kTile) : kTile;
        const bool full = rem == kTile &&
                          (!a.causal || (kbase + kTile - 1 <= qa_lo &&
                                         (a.window < 0 || qa_hi < kbase + a.window)));
        if (!full) {
          keep_branch();
          int hi = rem - 1, lo = 0;
          if (a.causal) {
            const int64_t dq = a.q_start + ql[0] - kbase;
            if (dq < hi) hi = dq < -1 ? -1 : int(dq);
            if (a.window >= 0) {
              const int64_t first = dq - a.window + 1;
              lo = first < 0 ? 0 : (first > kTile ? kTile : int(first));
            }
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int o2 = 16 * kq + 4 * lg + r;
            if (o2 < lo || o2 > hi) sc[r] = -INFINITY;
          }
        }
        float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
        mx = xor32_max(xor16_max(mx));
        // The running maximum may lag the true one by up to kTau: it moves
        // only when some row's raw maximum passes its threshold.
        const bool up = mx > thr[0];
        if (__any(up)) {
          keep_branch();
          rescale(0, up, mx);
        }
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], a.qscale, nm[0]));
        const uint32_t w0 = pack_h16(p[0], p[1]), w1 = pack_h16(p[2], p[3]);
        lsum[0] = sum2<true>(w1, sum2<true>(w0, lsum[0]));
        const h4_t pb = __builtin_bit_cast(h4_t, u32x2_t{w0, w1});
#pragma unroll
        for (int t2 = 0; t2 < NT; ++t2) {
          const h4_t va = __builtin_bit_cast(
              h4_t, tr_read(Vt + (16 * kq + 4 * lg + lr / 4) * KSTR + 16 * t2 + 4 * (lr % 4)));
          o[t2][0] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pb, o[t2][0], 0, 0, 0);
        }
      }
    };
    // The tile loop, compiled once per kind of this wavefront's tasks (VW:
    // V runs) where the kind goes by wavefront. Every load in it is
    // unconditional: a key past the end re-reads the last key (load_stage)
    // and a tile past the last re-reads the last tile (into a set that is
    // never dequantized for use), and the loop runs whole rounds of NS tiles
    // with the past-the-end ones computing nothing. The compiler's wait
    // counts then know exactly which loads are outstanding, and NS tiles of
    // words stay in flight: a branch around a load makes it wait for all of
    // them.
    auto run = [&](auto vw, auto dqf) __attribute__((always_inline)) {
      constexpr bool VW = decltype(vw)::value;
      constexpr bool DQF = decltype(dqf)::value;  // this wavefront dequantizes first
      auto load_tile = [&](auto set, int64_t tt) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        const int tc = int(tt < t_hi ? tt : t_hi);
        static_for<kPer>([&](auto I) {
          constexpr int i = decltype(I)::value;
          constexpr bool KV = kKindByTask ? i * kThreads >= 2 * D : VW;
          if constexpr (KV)
            load_stage<D, BV>(stv[S][i], vp, a, tc * kTile + tkey[i], trun[i]);
          else
            load_stage<D, BK>(stk[S][i], kp, a, tc * kTile + tkey[i], trun[i]);
        });
      };
      auto store_tile = [&](auto set, int kbuf, int vbuf) __attribute__((always_inline)) {
        constexpr int S = decltype(set)::value;
        static_for<kPer>([&](auto I) {
          constexpr int i = decltype(I)::value;
          constexpr bool KV = kKindByTask ? i * kThreads >= 2 * D : VW;
          if constexpr (KV)
            store_v<D, BV, H16>(stv[S][i], Vt2(vbuf), tkey[i], trun[i]);
          else
            store_k<D, BK, H16>(stk[S][i], Ks2(kbuf), tkey[i], trun[i]);
        });
      };
      // V^T tiles: tile tt's K and V^T straight into LDS buffers kb and vb,
      // this wavefront's four 1 KB pieces (K chunks 2 w and 2 w + 1 of the
      // tile's 16, the same of V^T). Lane l of K chunk j
      // fills row r = 4 j + l / 16 at position l % 16 with the row's chunk
      // k_chunk_pos(r, l % 16) (rows past the last key re-read it: their
      // scores are masked); of V^T chunk j, row R = 16 j + l / 4 at position
      // l % 4 (V^T tiles are whole, zeros past the last key).
      uint32_t dma_kr[2], dma_kc[2], dma_v[2];
      if constexpr (VT) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const uint32_t j = uint32_t(2 * wave + i);
          dma_kr[i] = 4 * j + uint32_t(lane) / 16;
          dma_kc[i] = 16 * k_chunk_pos(dma_kr[i], uint32_t(lane) % 16);
          const uint32_t R = 16 * j + uint32_t(lane) / 4;
          dma_v[i] = R * 64 + 16 * vt_chunk_pos(R, uint32_t(lane) % 4);
        }
      }
      auto dma_tile = [&](int64_t tt, int kb, int vb) __attribute__((always_inline)) {
        if constexpr (VT) {
          const uint32_t tc = uint32_t(tt < t_hi ? tt : t_hi);
          const uint32_t klds = __builtin_amdgcn_readfirstlane(lds_addr(Ks2(kb)));
          const uint32_t vlds = __builtin_amdgcn_readfirstlane(lds_addr(Vt2(vb)));
          const char* kbase = reinterpret_cast<const char*>(kp.w0);
          const char* vbase = reinterpret_cast<const char*>(vp.w0) + size_t(tc) * (kTile * D * 2);
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const uint32_t row = min(tc * kTile + dma_kr[i], uint32_t(a.total) - 1);
            lds_dma16(kbase + size_t(row) * (D * 2) + dma_kc[i], klds + uint32_t(2 * wave + i) * 1024);
          }
#pragma unroll
          for (int i = 0; i < 2; ++i)
            lds_dma16(vbase + dma_v[i], vlds + uint32_t(2 * wave + i) * 1024);
        }
      };
      // Operand read offsets in the V^T variant's unpadded tiles (elements):
      // K chunk 4 s + lg of row lr (+ 16 i rows), V^T chunk lg of row lr
      // (+ u D + 16 t2 rows: bit 3 of the row is bit 3 of lr).
      int kco[NDW], vco = 0;
      if constexpr (VT) {
#pragma unroll
        for (int s2 = 0; s2 < NDW; ++s2)
          kco[s2] = lr * D + 8 * int(k_chunk_pos(uint32_t(lr), uint32_t(4 * s2 + lg)));
        vco = lr * 32 + 8 * int(vt_chunk_pos(uint32_t(lr), uint32_t(lg)));
      }
      if constexpr (VT) {
        // The Q fragments and the first tile have landed before the loop;
        // the second tile is in flight.
        __builtin_amdgcn_s_waitcnt(0x0F70);
        dma_tile(t_lo, 0, 0);
        dma_tile(t_lo + 1, 1, 1);
        __builtin_amdgcn_s_waitcnt(0x0F74);
      } else {
        load_tile(std::integral_constant<int, 0>{}, t_lo);
        // Everything loaded so far (the Q fragments, the first tile) has
        // landed: without this the compiler's loop-carried wait analysis
        // keeps the Q loads pending and makes every tile's MFMAs wait for
        // the next tile's prefetch. (vmcnt(0); expcnt and lgkmcnt
        // unchanged.)
        __builtin_amdgcn_s_waitcnt(0x0F70);
        store_tile(std::integral_constant<int, 0>{}, 0, 0);
        // Tile t_lo + 1 + k into set (k + 1) % NS: tile x sits in set
        // (x - t_lo) % NS until it is dequantized.
        static_for<NS>([&](auto k) {
          load_tile(std::integral_constant<int, (decltype(k)::value + 1) % NS>{},
                    t_lo + 1 + decltype(k)::value);
        });
      }
      __syncthreads();
      // P V of one tile: the packed weights pp[u][j] (keys 32u + [0, 32) of
      // rows 16j + [0, 16)) times V^T from buffer Vt.
      auto pv_tile = [&](const h8_t (&pp)[2][NR], const uint16_t* Vt) __attribute__((always_inline)) {
        if constexpr (VT) {
          // Four operands read ahead of their products: one 16-byte read
          // feeds two products, too little to cover the read's latency.
  #pragma unroll
          for (int u = 0; u < 2; ++u)
  #pragma unroll
            for (int t0 = 0; t0 < NT; t0 += 4) {
              h8_t va[4];
  #pragma unroll
              for (int k = 0; k < 4; ++k)
                va[k] = *reinterpret_cast<const h8_t*>(
                    Vt + (u * D + 16 * (t_base + t0 + k)) * 32 + vco);
  #pragma unroll
              for (int k = 0; k < 4; ++k)
  #pragma unroll
                for (int j = 0; j < NR; ++j)
                  o[t0 + k][j] = mma<true>(va[k], pp[u][j], o[t0 + k][j]);
            }
          // The order for the scheduler: four reads, then a read after
          // every two products, so four stay in flight.
          __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
  #pragma unroll
          for (int k = 0; k < 2 * NT - 4; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
          __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
          return;
        }
  #pragma unroll
        for (int u = 0; u < 2; ++u)
  #pragma unroll
          for (int t2 = 0; t2 < NT; ++t2) {
            // Lane lr of group lg supplies row 32u + 4lg + lr/4 and channels
            // 16 tt + 4(lr % 4) + [0, 4); the transposing read hands it
            // channel 16 tt + lr of keys 32u + 4lg + [0, 4) (and + 16 for
            // the second read): the A operand of V^T for the k slots the
            // score registers fill.
            const uint16_t* vrow = Vt + (32 * u + 4 * lg + lr / 4) * KSTR +
                                   16 * (t_base + t2) + 4 * (lr % 4);
            const u32x2_t lo = tr_read(vrow);
            const u32x2_t hi = tr_read(vrow + 16 * KSTR);
            const h8_t va = __builtin_bit_cast(h8_t, u32x4_t{lo.x, lo.y, hi.x, hi.y});
  #pragma unroll
            for (int j = 0; j < NR; ++j)
              o[t2][j] = mma<true>(va, pp[u][j], o[t2][j]);
          }
      };
      // S^T of one tile: the K operand from buffer Ks against the
      // wavefront's Q fragments (channel split: the partial tiles of the
      // wavefronts summed through LDS).
      auto score_tile = [&](const uint16_t* Ks, f4_t (&sc)[4][NR]) __attribute__((always_inline)) {
  #pragma unroll
        for (int i = 0; i < 4; ++i)
  #pragma unroll
          for (int j = 0; j < NR; ++j) sc[i][j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
  #pragma unroll
        for (int s = 0; s < NDW; ++s)
  #pragma unroll
          for (int i = 0; i < 4; ++i) {
            // (V^T tiles: K rows unpadded, chunk 4 s + lg of row 16 i + lr
            // at its permuted position.)
            const op8_t ka = *reinterpret_cast<const op8_t*>(
                VT ? Ks + 16 * i * D + kco[s]
                   : Ks + (16 * i + lr) * KSTR + 32 * (s_base + s) + 8 * lg);
  #pragma unroll
            for (int j = 0; j < NR; ++j)
              sc[i][j] = mma<H16>(ka, qf[j][s], sc[i][j]);
          }
        if constexpr (VT) {
          // Eight K reads first, then one after every two products (eight
          // in flight; left to itself the scheduler keeps two).
          __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
  #pragma unroll
          for (int k = 0; k < 4 * NDW - 8; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          }
          __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
        }
        if constexpr (CS) {
          // Every wavefront of the block is live here (they share the rows).
  #pragma unroll
          for (int i = 0; i < 4; ++i) s_part[wave][i][lane] = sc[i][0];
          __syncthreads();
  #pragma unroll
          for (int i = 0; i < 4; ++i) {
            f4_t tot = s_part[0][i][lane];
  #pragma unroll
            for (int w = 1; w < kWaves; ++w) tot += s_part[w][i][lane];
            sc[i][0] = tot;
          }
        }
      };
      // The weights of tile t: exp2 of each scaled score less its row's
      // running maximum, rounded to f16 into pp, their sums added to acc.
      auto weigh = [&](f4_t (&sc)[4][NR], h8_t (&pp)[2][NR], float (&acc)[NR]) __attribute__((always_inline)) {
  #pragma unroll
        for (int j = 0; j < NR; ++j)
  #pragma unroll
          for (int i = 0; i < 4; ++i)
  #pragma unroll
            for (int r = 0; r < 4; ++r)
              sc[i][j][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[i][j][r], a.qscale, nm[j]));
  #pragma unroll
        for (int u = 0; u < 2; ++u)
  #pragma unroll
          for (int j = 0; j < NR; ++j) {
            const f4_t p0 = sc[2 * u][j], p1 = sc[2 * u + 1][j];
            const u32x4_t w = {pack_h16(p0[0], p0[1]), pack_h16(p0[2], p0[3]),
                               pack_h16(p1[0], p1[1]), pack_h16(p1[2], p1[3])};
            pp[u][j] = __builtin_bit_cast(h8_t, w);
            // The row sum counts the weights as rounded for the matrix cores,
            // so the output stays an exact convex combination of them.
  #pragma unroll
            for (int e = 0; e < 4; ++e)
              acc[j] = sum2<true>(w[e], acc[j]);
          }
      };
      // The online softmax of tile t's scores: the mask, the running
      // maximum (and the rescale when it moves), then the weights.
      auto softmax_tile = [&](int64_t t, f4_t (&sc)[4][NR], h8_t (&pp)[2][NR]) __attribute__((always_inline)) {
        // Mask: only on tiles some row of the block sees in part. Key offset
        // o in the tile is visible to a row iff lo <= o <= hi.
        const int64_t kbase = a.k_start + int64_t(t) * kTile;
        const int rem = a.total - int64_t(t) * kTile < kTile ? int(a.total - int64_t(t) * kTile) : kTile;
        const bool full = rem == kTile &&
                          (!a.causal || (kbase + kTile - 1 <= qa_lo &&
                                         (a.window < 0 || qa_hi < kbase + a.window)));
        if (!full) {
          keep_branch();
  #pragma unroll
          for (int j = 0; j < NR; ++j) {
            int hi = rem - 1, lo = 0;
            if (a.causal) {
              const int64_t dq = a.q_start + ql[j] - kbase;  // the row's own offset
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
          // The lane's maximum over its 16 keys of the row. The running
          // maximum may lag the true one by up to kTau: it moves only when
          // the row's raw maximum passes its threshold, which needs some
          // lane's to pass it; only then are the row's four lanes combined.
          float mx = -INFINITY;
  #pragma unroll
          for (int i = 0; i < 4; ++i)
  #pragma unroll
            for (int r = 0; r < 4; ++r) mx = fmaxf(mx, sc[i][j][r]);
          if (__any(mx > thr[j])) {
            keep_branch();
            mx = xor32_max(xor16_max(mx));
            rescale(j, mx > thr[j], mx);
          }
        }
        weigh(sc, pp, lsum);
      };
      auto vnext = [](int c) { return VBN >= 3 ? (c == VBN - 1 ? 0 : c + 1) : (c ^ (VBN - 1)); };
      auto vprev = [](int c) { return c == 0 ? VBN - 1 : c - 1; };
      auto knext = [](int c) { return KBN == 3 ? (c == 2 ? 0 : c + 1) : (c ^ (KBN - 1)); };
      // The second wavefront of each SIMD multiplies by V one tile late:
      // pprev then carries the previous tile's packed weights.
      constexpr bool DEFER = kDeferPV && DQF;
      static_assert(!kDeferPV || NS == 1, "one tile a round where P V runs late");
      h8_t pprev[2][NR];
      // One tile: set S holds tile t + 1's words, which go into the next
      // LDS buffers (last read in an earlier tile, before the barrier that
      // ended it); S then fetches tile t + 1 + NS.
      auto tile = [&](int64_t t, int cur, int vc, auto set) __attribute__((always_inline)) {
        if constexpr (VT) {
          // Tile t + 2 into the buffers after the next (K: tile t - 1's, read
          // before the barrier that ended it; V: tile t - 2's, whose late
          // P V ran at the start of tile t - 1), in flight for two tiles.
          dma_tile(t + 2, knext(knext(cur)), vnext(vnext(vc)));
        } else if constexpr (kBufs == 2 && DQF) {
          store_tile(set, cur ^ 1, vnext(vc));
          load_tile(set, t + 1 + NS);
        }
        if (t <= t_hi) {
          // A wavefront whose rows are all past the end (a short block)
          // only dequantizes.
          if (live) {
            if constexpr (KS) {
              ks_tile(t, cur, vc);
            } else {
              // The products run at the higher wave priority where the two
              // wavefronts of a SIMD alternate phases, so the matrix cores
              // are fed first.
              if constexpr (kDeferPV) __builtin_amdgcn_s_setprio(1);
              if constexpr (DEFER) {
                if (t > t_lo) pv_tile(pprev, Vt2(vprev(vc)));
              }
              f4_t sc[4][NR];
              score_tile(Ks2(cur), sc);
              if constexpr (kDeferPV) __builtin_amdgcn_s_setprio(0);
              softmax_tile(t, sc, pprev);
              if constexpr (!DEFER) {
                if constexpr (kDeferPV) __builtin_amdgcn_s_setprio(1);
                pv_tile(pprev, Vt2(vc));
                if constexpr (kDeferPV) __builtin_amdgcn_s_setprio(0);
              }
            }
          }
        }
        if constexpr (VT) {
          // This wavefront's part of tile t + 1 is in LDS (the four newest
          // loads are tile t + 2's). (vmcnt(4); expcnt and lgkmcnt unchanged.)
          __builtin_amdgcn_s_waitcnt(0x0F74);
        } else if constexpr (kBufs == 2) {
          if constexpr (!DQF) {
            store_tile(set, cur ^ 1, vnext(vc));
            load_tile(set, t + 1 + NS);
          }
        } else {
          __syncthreads();  // every wavefront is done with this tile's LDS
          store_tile(set, 0, 0);
          load_tile(set, t + 1 + NS);
        }
        __syncthreads();
      };
      // Whole rounds of NS tiles, unrolled over the stage sets so each one
      // stays in named registers.
      const int64_t rounds = (t_hi - t_lo + NS) / NS;
      int cur = 0, vc = 0;
      for (int64_t it = 0; it < rounds; ++it) {
        static_for<NS>([&](auto k) {
          tile(t_lo + it * NS + decltype(k)::value, cur, vc,
               std::integral_constant<int, (decltype(k)::value + 1) % NS>{});
          cur = knext(cur);
          vc = vnext(vc);
        });
      }
      // The last tile's P V: its V buffer is not written again (the loader's
      // last store went to the buffer after it).
      if constexpr (DEFER) {
        if (live) pv_tile(pprev, Vt2(vprev(vc)));
      }
      // The re-loads of the last tile past the end land before the
      // workgroup's LDS is released.
      if constexpr (VT) __builtin_amdgcn_s_waitcnt(0x0F70);
    };
    // One copy of the loop per (task kind, order) a wavefront can have: the
    // two arms of a runtime branch would load into the same registers, and
    // the copies where they meet would wait for every load in flight.
    auto by_order = [&](auto vw) __attribute__((always_inline)) {
      if (kBufs == 2 && dequant_first)
        run(vw, std::true_type{});
      else
        run(vw, std::false_type{});
    };
    if constexpr (kKindByTask) {
      by_order(std::false_type{});
    } else {
      if (wave * kWave >= 2 * D)
        by_order(std::true_type{});
      else
        by_order(std::false_type{});
    }
  }
  if constexpr (KS) {
    // The key quarters' (m, l, O) of each row meet in LDS (the tile memory,
    // free after the last tile's barrier); wavefront (row group, kq) then
    // combines its group's rows over channels [kq D / KQ, (kq + 1) D / KQ):
    // lane i takes row i / 4 and D / 16 consecutive channels.
    const float tot = xor32_sum(xor16_sum(lsum[0]));
    float* so = reinterpret_cast<float*>(&s_tiles[0][0]);  // [kWaves][16][D]
    static_assert(sizeof(s_tiles) >= sizeof(float) * kWaves * 16 * D, "merge space");
    __syncthreads();
#pragma unroll
    for (int t2 = 0; t2 < NT; ++t2)
      *reinterpret_cast<f4_t*>(so + (wave * 16 + lr) * D + 16 * t2 + 4 * lg) = o[t2][0];
    if (lg == 0) {
      s_km[wave][lr] = m[0];
      s_kl[wave][lr] = tot;
    }
    __syncthreads();
    constexpr int CPL = D / 16;  // channels a lane
    const int rr = lane / 4, c0 = kq * (D / KQ) + (lane % 4) * CPL;
    const int rgp = wave % RG;
    const int64_t r = row0 + rgp * RW + rr;
    if (r < rows) {
      float mk[KQ], mx = -INFINITY;
#pragma unroll
      for (int q = 0; q < KQ; ++q) {
        mk[q] = s_km[q * RG + rgp][rr];
        mx = fmaxf(mx, mk[q]);
      }
      float fk[KQ], lt = 0.0f;
#pragma unroll
      for (int q = 0; q < KQ; ++q) {
        fk[q] = mk[q] == -INFINITY ? 0.0f : exp2f(mk[q] - mx);
        lt += fk[q] * s_kl[q * RG + rgp][rr];
      }
      float ov[CPL];
#pragma unroll
      for (int c = 0; c < CPL; ++c) {
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < KQ; ++q) acc += fk[q] * so[((q * RG + rgp) * 16 + rr) * D + c0 + c];
        ov[c] = acc;
      }
      const int64_t l = r / a.G, g = r % a.G;
      if (a.part_o) {
        const int64_t slot =
            ((int64_t(b) * a.L + l) * a.H + int64_t(kvh) * a.G + g) * a.n_part + a.split_base + split;
        float* po = a.part_o + slot * D + c0;
#pragma unroll
        for (int c = 0; c < CPL; c += 4)
          *reinterpret_cast<f4_t*>(po + c) = f4_t{ov[c], ov[c + 1], ov[c + 2], ov[c + 3]};
        if (kq == 0 && lane % 4 == 0) {
          a.part_m[slot] = mx;
          a.part_l[slot] = lt;
        }
      } else {
        const float inv = lt > 0.0f ? 1.0f / lt : 0.0f;
        uint16_t* dst = a.out + int64_t(b) * a.qs_b + (int64_t(kvh) * a.G + g) * a.qs_h + l * a.qs_l + c0;
#pragma unroll
        for (int c = 0; c < CPL; c += 4)
          *reinterpret_cast<u32x2_t*>(dst + c) =
              u32x2_t{pack_bf16(ov[c] * inv, ov[c + 1] * inv), pack_bf16(ov[c + 2] * inv, ov[c + 3] * inv)};
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    float tot = lsum[j];
    tot = xor32_sum(xor16_sum(tot));
    if (row_of(j) >= rows) continue;
    // The prefill variant's V operands were scaled by 2^-kVShift.
    const float vup = H16 ? 1.0f : kVUp;
    if (a.part_o) {
      const int64_t r = row0 + wrow + 16 * j + lr;
      const int64_t l = r / a.G, h = int64_t(kvh) * a.G + r % a.G;
      const int64_t slot = ((int64_t(b) * a.L + l) * a.H + h) * a.n_part + a.split_base + split;
      float* po = a.part_o + slot * D;
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2)
        *reinterpret_cast<f4_t*>(po + 16 * (t_base + t2) + 4 * lg) = o[t2][j] * vup;
      if (lg == 0 && (!CS || wave == 0)) {
        a.part_m[slot] = m[j];
        a.part_l[slot] = tot;
      }
    } else {
      const float inv = tot > 0.0f ? vup / tot : 0.0f;
#pragma unroll
      for (int t2 = 0; t2 < NT; ++t2) {
        const f4_t v = o[t2][j] * inv;
        *reinterpret_cast<u32x2_t*>(a.out + orow_of(row_of(j)) + 16 * (t_base + t2) + 4 * lg) =
            u32x2_t{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])};
      }
    }
  }
}

typedef void (*KernelFn)(Args);

// The kernel for (D, bits_k, bits_v), bits in {2, 3, 4, 5, 6, 8}, or
// (kPreBits, kPreBits) / (kPreBits, kPreF16) for rows dequantized
// beforehand; null if unsupported. h16: the f16-operand variant.
KernelFn pick_d64(int bk, int bv, bool h16);
KernelFn pick_d128(int bk, int bv, bool h16);
KernelFn pick_d256(int bk, int bv, bool h16);
KernelFn pick_d512(int bk, int bv, bool h16);

template <int D, int BK, bool H16>
KernelFn pick_bv(int bv) {
  switch (bv) {
    case 2: return prefill_affine_kernel<D, BK, 2, H16>;
    case 3: return prefill_affine_kernel<D, BK, 3, H16>;
    case 4: return prefill_affine_kernel<D, BK, 4, H16>;
    case 5: return prefill_affine_kernel<D, BK, 5, H16>;
    case 6: return prefill_affine_kernel<D, BK, 6, H16>;
    case 8: return prefill_affine_kernel<D, BK, 8, H16>;
  }
  return nullptr;
}

template <int D, bool H16>
KernelFn pick_for(int bk, int bv) {
  if constexpr (!H16) {
    if (bk == kPreBits && bv == kPreBits) return prefill_affine_kernel<D, kPreBits, kPreBits, false>;
    if (bk == kPreBits && bv == kPreF16) return prefill_affine_kernel<D, kPreBits, kPreF16, false>;
    if constexpr (D == 128)
      if (bk == kPreBits && bv == kPreF16T) return prefill_affine_kernel<D, kPreBits, kPreF16T, false>;
  }
  switch (bk) {
    case 2: return pick_bv<D, 2, H16>(bv);
    case 3: return pick_bv<D, 3, H16>(bv);
    case 4: return pick_bv<D, 4, H16>(bv);
    case 5: return pick_bv<D, 5, H16>(bv);
    case 6: return pick_bv<D, 6, H16>(bv);
    case 8: return pick_bv<D, 8, H16>(bv);
  }
  return nullptr;
}

}  // namespace prefill
}  // namespace tqkv
