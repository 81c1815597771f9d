// Fused decode attention over affine-packed K/V (the headline hot path).
//
// Work split: one workgroup per (token split, KV head, batch row); its four
// wavefronts take contiguous quarters of the split. Inside a wavefront, LPT =
// D / EPL lanes (a lane group) own one token pair at a time, each lane EPL
// consecutive channels, all in one quantization group; a wavefront walks
// 2 * 64 / LPT consecutive tokens per step with coalesced row loads. All
// G = H / H_kv query heads of the KV head share the codes (GQA broadcast).
//
// Arithmetic is v_dot2_f32_f16 on codes that are never converted: a code ANDed
// into the low mantissa bits of an f16 half is the exact subnormal
// c * 2^(o - 24) (o = its bit offset there), so one AND turns a window of the
// packed stream into an f16x2 operand (plans in pair_plans.hpp).
//   Keys: pairs of channels of one token against f16 query pairs pre-scaled by
//   2^(E - o); the score is scale * sum(q * c) + bias * sum(q) per group (the
//   affine terms factor out), summed over the lane group by a butterfly.
//   Values: one channel of the token pair against the two tokens' weights
//   p * scale rounded to f16; the bias term p * bias accumulates apart in
//   f32. A wave-uniform power of two per head (folded into the softmax
//   reference) keeps the f16 weights finite whatever the value scales.
// The online softmax keeps its running maximum up to kTau (log2 units) behind
// the true one, so accumulators are rescaled only when it moves by more.
// Lane groups, then wavefronts (through LDS), merge their (max, sum, acc)
// states. When one workgroup owns all keys of its (batch row, KV head) it
// writes the normalized bf16 output itself: the decode is one launch. Else
// each workgroup writes its split's unnormalized partial and a small second
// kernel merges the splits, as native_quant_attention.rs:190-207 does in its
// pass 2.
//
// Decode is HBM-bound (~1 dot2 per 2 codes per head), so the kernel uses VALU
// dot products, not MFMA. f16 denormals must be preserved (the default mode).
#pragma once

#include <cmath>
#include <type_traits>
#include <utility>

#include "common.hpp"
#include "pair_plans.hpp"

namespace tqkv {
namespace decode {

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

struct Seg {
  const uint32_t* kw;
  const uint16_t* ks;
  const uint16_t* kb;
  const uint32_t* vw;
  const uint16_t* vs;
  const uint16_t* vb;
  int64_t cap;
  int64_t n;
  int64_t b_stride;  // rows between batch rows: H_kv * cap, or 0 when shared
};

struct Args {
  const uint16_t* q;
  int H, H_kv, gs;
  // Query heads of a KV head: the kernel serves G of the group's Gt heads,
  // from h_off on (Gt = G, h_off = 0 unless the group is split over
  // launches; the dot2 kernels only).
  int Gt, h_off;
  float qscale;  // softmax scale * log2(e)
  Seg seg[2];
  int64_t n0, total;
  int64_t split_len;
  int n_splits;
  // Partial slots per (batch row, query head): split s writes slot
  // split_base + s of n_part (other slots belong to other launches).
  int split_base, n_part;
  uint16_t* out;  // [B, H, 1, D], written directly when n_part == 1
  // Page-sparse decode (the paged kernels only): segment 0 is a whole cache
  // slab read through this page table, rows [0, n0) standing for pages
  // pages[(b * H_kv + kvh) * n_pages + i] (64 rows each, ascending).
  const int32_t* pages;
  int n_pages;
  // Append fused into the decode (the MFMA kernels; app_k null: none): the
  // new token's bf16 K and V rows ([B, H_kv, D] each) are quantized by the
  // last wavefront of each unit's last split, written into the cache buffers
  // at row app_row of the unit's slab (app_cap rows a slab), and attended as
  // one more key read back from LDS. The segments do not hold that row.
  const uint16_t* app_k;
  const uint16_t* app_v;
  uint32_t* app_kw;
  uint16_t* app_ks;
  uint16_t* app_kb;
  uint32_t* app_vw;
  uint16_t* app_vs;
  uint16_t* app_vb;
  int64_t app_cap, app_row;
  float* part_o;  // [B, H, n_part, D]
  float* part_m;  // [B, H, n_part]
  float* part_l;  // [B, H, n_part]
};

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2_t as_h2(uint32_t x) { return __builtin_bit_cast(h2_t, x); }
__device__ __forceinline__ uint32_t h2_bits(h2_t h) { return __builtin_bit_cast(uint32_t, h); }

// f(std::integral_constant<int, I>) for I = 0 .. N-1, fully unrolled, so plan
// lookups and register-array indices are compile-time constants.
template <typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// The 32 bits starting at bit BIT of a lane's chunk of NW words (bits past
// the chunk read as zero): a word, or one funnel shift of two.
template <int NW, int BIT>
__device__ __forceinline__ uint32_t window(const uint32_t* w) {
  constexpr int k = BIT / 32, r = BIT % 32;
  const uint32_t lo = k < NW ? w[k] : 0u;
  if constexpr (r == 0) {
    return lo;
  } else {
    const uint32_t hi = k + 1 < NW ? w[k + 1] : 0u;
    if constexpr (r % 8 == 0)
      return __builtin_amdgcn_alignbyte(hi, lo, r / 8);
    else
      return __builtin_amdgcn_alignbit(hi, lo, r);
  }
}

// Bits [BIT, BIT + 16) of token 0's chunk in the low half, the same bits of
// token 1's chunk in the high half: one byte permute when BIT is a byte
// inside a word's first three, else the two windows then the permute.
template <int NW, int BIT>
__device__ __forceinline__ uint32_t merge_pair(const uint32_t* w0, const uint32_t* w1) {
  constexpr int k = BIT / 32, r = (BIT % 32) / 8;
  if constexpr (BIT % 8 == 0 && r < 3) {
    constexpr uint32_t sel = uint32_t(r) | uint32_t(r + 1) << 8 | uint32_t(4 + r) << 16 |
                             uint32_t(5 + r) << 24;
    return __builtin_amdgcn_perm(w1[k], w0[k], sel);
  } else {
    return __builtin_amdgcn_perm(window<NW, BIT>(w1), window<NW, BIT>(w0), 0x05040100u);
  }
}

// N consecutive words of the packed stream, read once and never again:
// non-temporal vector loads (the cache is streamed, not reused), widest first.
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
template <int N>
__device__ __forceinline__ void load_words(uint32_t* dst, const uint32_t* src) {
  if constexpr (N >= 4) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src));
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
    dst[3] = v.w;
    if constexpr (N > 4) load_words<N - 4>(dst + 4, src + 4);
  } else if constexpr (N == 3) {
    const u32x3_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x3_t*>(src));
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
  } else if constexpr (N == 2) {
    const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(src));
    dst[0] = v.x;
    dst[1] = v.y;
  } else if constexpr (N == 1) {
    dst[0] = __builtin_nontemporal_load(src);
  }
}

// Score partial sum of one token: sum over the K plan of dot2(codes, q pair).
template <int BK, int EPL, int KW>
__device__ __forceinline__ float k_dot(const uint32_t* w, const uint32_t* qp) {
  using KP = Plan<BK, EPL>;
  float acc = 0.0f;
  static_for<KP::kN>([&](auto J) {
    constexpr KOp op = KP::k[J];
    const uint32_t c = window<KW, op.bit>(w) & op.mask;
    acc = __builtin_amdgcn_fdot2(as_h2(c), as_h2(qp[J]), acc, false);
  });
  return acc;
}

// Values of a token pair: acc[e] += c_t0,e * w0 + c_t1,e * w1 with the two
// tokens' weights as one f16 pair, over every window of the V plan.
template <int BV, int EPL, int VW, int G>
__device__ __forceinline__ void v_accumulate(const uint32_t* w0, const uint32_t* w1,
                                             const uint32_t* wp, float (*acc)[EPL]) {
  using VP = Plan<BV, EPL>;
  static_for<VP::vN>([&](auto I) {
    constexpr VWin win = VP::vw[I];
    const uint32_t m = merge_pair<VW, win.bit>(w0, w1);
    static_for<win.count>([&](auto C) {
      constexpr VCode vc = VP::vc[win.first + C];
      const uint32_t codes = m & vc.mask;
#pragma unroll
      for (int h = 0; h < G; ++h) {
        acc[h][vc.e] = __builtin_amdgcn_fdot2(as_h2(codes), as_h2(wp[h]), acc[h][vc.e], false);
      }
    });
  });
}

// Sum over the N lanes of an aligned lane group (N a power of two <= 64),
// every lane getting the total: quad permutes, then half-row and row
// mirrors, then cross-row shuffles.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  // Every source lane of these patterns exists, so bound_ctrl changes
  // nothing but lets the compiler fold the move into the add (v_add_f32_dpp).
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x),
                                                      decltype(ctrl)::value, 0xf, 0xf, true));
  };
  if constexpr (N >= 2) v += dpp(v, std::integral_constant<int, 0xb1>{});   // quad [1,0,3,2]
  if constexpr (N >= 4) v += dpp(v, std::integral_constant<int, 0x4e>{});   // quad [2,3,0,1]
  if constexpr (N >= 8) v += dpp(v, std::integral_constant<int, 0x141>{});  // half-row mirror
  if constexpr (N >= 16) v += dpp(v, std::integral_constant<int, 0x140>{}); // row mirror
  if constexpr (N >= 32) v += __shfl_xor(v, 16, kWave);
  if constexpr (N >= 64) v += __shfl_xor(v, 32, kWave);
  return v;
}

// Max over the whole wavefront, every lane getting it.
__device__ __forceinline__ float wave_max_all(float v) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Running maxima may lag the true maximum by up to kTau (log2 units) before
// the accumulators are rescaled: weights stay <= 2^kTau, and rescales become
// rare after the first keys.
constexpr float kTau = 8.0f;

// Value weights p * scale travel as f16 (finite below 65,504). With p <=
// 2^kTau, scales up to kScaleSafe keep every weight <= kWeightMax; a step
// with a larger scale checks its products and, where one passes kWeightMax,
// moves the head's softmax reference up by a power of two.
constexpr float kScaleSafe = 128.0f;  // 2^(15 - kTau)
constexpr float kWeightMax = 32768.0f;

template <int D, int BK, int BV, int G, int EPL, int kWaves>
__global__ __launch_bounds__(kWave* kWaves) void decode_affine_kernel(Args a) {
  using KP = Plan<BK, EPL>;
  using VP = Plan<BV, EPL>;
  constexpr int LPT = D / EPL;
  constexpr int TPW = kWave / LPT;  // lane groups per wavefront
  constexpr int KW = EPL * BK / 32;
  constexpr int VW = EPL * BV / 32;
  constexpr int KROW = D * BK / 32;
  constexpr int VROW = D * BV / 32;
  static_assert(LPT >= 1 && LPT <= kWave && (kWave % LPT) == 0, "lanes per token");
  static_assert((EPL * BK) % 32 == 0 && (EPL * BV) % 32 == 0, "whole words per lane");

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int lane_tok = lane / LPT, lane_sub = lane % LPT;
  const int e0 = lane_sub * EPL;
  const int ngroups = D / a.gs;
  const int grp = e0 / a.gs;

  // Query: f16 pairs matching the K plan, each channel scaled by
  // 2^(E - o) so every product with a code subnormal carries 2^(E - 24);
  // E per head keeps the largest |q| 2^E below 2^15.
  uint32_t qp[G][KP::kN];
  float kfac[G], qbias[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const uint16_t* qrow = a.q + (int64_t(b) * a.H + kvh * a.Gt + a.h_off + h) * D + e0;
    float qr[EPL];
    float qsum = 0.0f, qmax = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      qr[e] = bf16_to_f32(qrow[e]);
      qsum += qr[e];
      qmax = fmaxf(qmax, fabsf(qr[e]));
    }
#pragma unroll
    for (int off = 1; off < LPT; off <<= 1) qmax = fmaxf(qmax, __shfl_xor(qmax, off, kWave));
    int ex = 0;
    if (qmax > 0.0f) frexpf(qmax, &ex);
    const int E = 15 - ex;
    static_for<KP::kN>([&](auto J) {
      constexpr KOp op = KP::k[J];
      const float lo = __builtin_ldexpf(qr[op.lo_e], E - op.lo_o);
      float hi = 0.0f;
      if constexpr (op.hi_e >= 0) hi = __builtin_ldexpf(qr[op.hi_e], E - op.hi_o);
      qp[h][J] = h2_bits(h2_t{_Float16(lo), _Float16(hi)});
    });
    kfac[h] = a.qscale * __builtin_ldexpf(1.0f, 24 - E);
    qbias[h] = a.qscale * qsum;
  }

  const int64_t t_begin = int64_t(split) * a.split_len;
  const int64_t t_end = t_begin + a.split_len < a.total ? t_begin + a.split_len : a.total;
  int64_t chunk = (t_end - t_begin + kWaves - 1) / kWaves;
  chunk = (chunk + 2 * TPW - 1) / (2 * TPW) * (2 * TPW);
  const int64_t w_begin = t_begin + wave * chunk;
  const int64_t w_end = w_begin + chunk < t_end ? w_begin + chunk : t_end;

  // m: the lane group's running maximum; ev: a wave-uniform exponent raised
  // only when an f16 value weight would overflow; mr = m + ev, the reference
  // the weights 2^(s - mr), l and acc are taken against.
  float m[G], mr[G], ev[G], l[G], bacc[G];
  float acc[G][EPL];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    mr[h] = -INFINITY;
    ev[h] = 0.0f;
    l[h] = 0.0f;
    bacc[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[h][e] = 0.0f;
  }

  // One step: every lane group takes the token pair (2j, 2j+1) of the next
  // 2 * TPW keys. Loads of step n+1 are issued before step n computes.
  struct Buf {
    uint32_t k[2][KW], v[2][VW];
    uint16_t ks[2], kb[2], vs[2], vb[2];
  };
  auto load = [&](Buf& f, const Seg& s, int64_t row0, int64_t row1) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t r = i == 0 ? row0 : row1;
      load_words<KW>(f.k[i], s.kw + r * KROW + lane_sub * KW);
      load_words<VW>(f.v[i], s.vw + r * VROW + lane_sub * VW);
      f.ks[i] = __builtin_nontemporal_load(s.ks + r * ngroups + grp);
      f.kb[i] = __builtin_nontemporal_load(s.kb + r * ngroups + grp);
      f.vs[i] = __builtin_nontemporal_load(s.vs + r * ngroups + grp);
      f.vb[i] = __builtin_nontemporal_load(s.vb + r * ngroups + grp);
    }
  };
  // kMasked: some keys of the step are past the range (score -inf); only the
  // last step of a range can have them. Full steps skip those guards and use
  // the bare v_exp_f32: there every score is finite and, after the first
  // step, so is every running maximum (the first step always moves it).
  auto compute = [&](const Buf& f, const bool* valid, auto masked) {
    constexpr bool kMasked = decltype(masked)::value;
    auto ex2 = [](float x) { return kMasked ? exp2f(x) : __builtin_amdgcn_exp2f(x); };
    float sc[2][G];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float ks = bf16_to_f32(f.ks[i]), kb = bf16_to_f32(f.kb[i]);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float dot = k_dot<BK, EPL, KW>(f.k[i], qp[h]);
        const float ps = group_sum<LPT>(fmaf(kfac[h] * ks, dot, qbias[h] * kb));
        sc[i][h] = (!kMasked || valid[i]) ? ps : -INFINITY;
      }
    }
    uint32_t wp[G];
    const float vs0 = bf16_to_f32(f.vs[0]), vs1 = bf16_to_f32(f.vs[1]);
    const float vb0 = bf16_to_f32(f.vb[0]), vb1 = bf16_to_f32(f.vb[1]);
    const bool big = __builtin_expect(__any(fmaxf(fabsf(vs0), fabsf(vs1)) > kScaleSafe), 0);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      // Online softmax with a lazily moved maximum.
      const float mx = fmaxf(sc[0][h], sc[1][h]);
      const bool need = mx > m[h] + kTau;
      if (__any(need)) {
        const float mnew = need ? mx : m[h];
        const float fct = (kMasked && mnew == -INFINITY) ? 1.0f : ex2(m[h] - mnew);
        l[h] *= fct;
        bacc[h] *= fct;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[h][e] *= fct;
        m[h] = mnew;
        mr[h] = mnew + ev[h];
      }
      float p0 = (kMasked && sc[0][h] == -INFINITY) ? 0.0f : ex2(sc[0][h] - mr[h]);
      float p1 = (kMasked && sc[1][h] == -INFINITY) ? 0.0f : ex2(sc[1][h] - mr[h]);
      if (big) {
        // p <= 2^kTau and a scale past kScaleSafe: check the products.
        const float pm = wave_max_all(fmaxf(fabsf(p0 * vs0), fabsf(p1 * vs1)));
        if (pm > kWeightMax) {
          int e = 0;
          frexpf(pm * (1.0f / kWeightMax), &e);  // pm * 2^-e < kWeightMax
          const float fct = __builtin_ldexpf(1.0f, -e);
          ev[h] += float(e);
          mr[h] = m[h] + ev[h];
          l[h] *= fct;
          bacc[h] *= fct;
#pragma unroll
          for (int e2 = 0; e2 < EPL; ++e2) acc[h][e2] *= fct;
          p0 *= fct;
          p1 *= fct;
        }
      }
      l[h] += p0 + p1;
      bacc[h] = fmaf(p0, vb0, fmaf(p1, vb1, bacc[h]));
      wp[h] = h2_bits(h2_t{_Float16(p0 * vs0), _Float16(p1 * vs1)});
    }
    v_accumulate<BV, EPL, VW, G>(f.v[0], f.v[1], wp, acc);
  };

  // The wavefront's keys, one segment at a time; full steps first, then a
  // last step whose idle lanes read an in-bounds row and are masked.
  for (int sg = 0; sg < 2; ++sg) {
    const Seg& s = a.seg[sg];
    const int64_t lo = sg == 0 ? w_begin : (w_begin > a.n0 ? w_begin : a.n0);
    const int64_t hi = sg == 0 ? (w_end < a.n0 ? w_end : a.n0) : w_end;
    if (lo >= hi) continue;
    const int64_t off = sg == 0 ? 0 : a.n0;
    const int64_t slab = int64_t(b) * s.b_stride + int64_t(kvh) * s.cap - off;
    const int64_t mine = 2 * lane_tok;
    constexpr int kStep = 2 * TPW;
    const int64_t n_full = (hi - lo) / kStep;
    const bool both[2] = {true, true};
    const std::integral_constant<bool, false> full{};
    const std::integral_constant<bool, true> masked{};
    if (n_full > 0) {
      // Two buffers in turn: the loads of the next step are in flight while
      // this one computes, with no register copies between steps.
      Buf b0, b1;
      int64_t row = slab + lo + mine;
      load(b0, s, row, row + 1);
      int64_t it = 0;
      for (; it + 2 <= n_full; it += 2) {
        load(b1, s, row + kStep, row + kStep + 1);
        compute(b0, both, full);
        row += 2 * kStep;
        if (it + 2 < n_full) load(b0, s, row, row + 1);
        compute(b1, both, full);
      }
      if (it < n_full) compute(b0, both, full);
    }
    const int64_t tail = lo + n_full * kStep;
    if (tail < hi) {
      Buf f;  // idle lanes re-read the last key of the range, masked out
      const int64_t t = tail + mine;
      const bool valid[2] = {t < hi, t + 1 < hi};
      const int64_t r0 = valid[0] ? t : hi - 1;
      const int64_t r1 = valid[1] ? t + 1 : hi - 1;
      load(f, s, slab + r0, slab + r1);
      compute(f, valid, masked);
    }
  }

  // Undo the code subnormal scale 2^(o - 24) per channel, add the bias term,
  // then merge the lane groups of this wavefront.
  static_for<VP::cN>([&](auto C) {
    constexpr VCode vc = VP::vc[C];
    constexpr float unscale = float(1 << (24 - vc.o));
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h][vc.e] = fmaf(acc[h][vc.e], unscale, bacc[h]);
  });
  // From here m is the reference of l and acc (the running maximum + ev).
#pragma unroll
  for (int h = 0; h < G; ++h) m[h] = mr[h];
#pragma unroll
  for (int off = LPT; off < kWave; off <<= 1) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float mo = __shfl_xor(m[h], off, kWave);
      const float lo = __shfl_xor(l[h], off, kWave);
      const float mx = fmaxf(m[h], mo);
      const float fa = mx == -INFINITY ? 0.0f : exp2f(m[h] - mx);
      const float fb = mx == -INFINITY ? 0.0f : exp2f(mo - mx);
      l[h] = l[h] * fa + lo * fb;
      m[h] = mx;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float ao = __shfl_xor(acc[h][e], off, kWave);
        acc[h][e] = acc[h][e] * fa + ao * fb;
      }
    }
  }

  // Merge the wavefronts through LDS and write this split's partial.
  __shared__ float s_m[kWaves][G], s_l[kWaves][G];
  __shared__ float s_acc[kWaves][G][D];
  if (lane_tok == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      if (lane_sub == 0) {
        s_m[wave][h] = m[h];
        s_l[wave][h] = l[h];
      }
#pragma unroll
      for (int e = 0; e < EPL; ++e) s_acc[wave][h][e0 + e] = acc[h][e];
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < G * D; i += kWave * kWaves) {
    const int h = i / D, d = i % D;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, s_m[w][h]);
    float ls = 0.0f, os = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = mx == -INFINITY ? 0.0f : exp2f(s_m[w][h] - mx);
      ls += s_l[w][h] * f;
      os += s_acc[w][h][d] * f;
    }
    const int64_t bh = int64_t(b) * a.H + kvh * a.Gt + a.h_off + h;
    if (a.n_part == 1) {
      a.out[bh * D + d] = f32_to_bf16(ls > 0.0f ? os / ls : 0.0f);
    } else {
      const int64_t row = bh * a.n_part + a.split_base + split;
      a.part_o[row * D + d] = os;
      if (d == 0) {
        a.part_m[row] = mx;
        a.part_l[row] = ls;
      }
    }
  }
}

using KernelFn = void (*)(Args);

// Channels a lane holds in the dot2 kernel: a width every plan of both
// widths has (3 and 5 bits pack whole words only from 32 codes, 2 and 6
// bits from 16), 8 for 4/8-bit caches of 6+ heads a KV head, else 16.
constexpr int epl_of(int bk, int bv, int G) {
  return (bk == 3 || bv == 3 || bk == 5 || bv == 5)   ? 32
         : (bk == 2 || bv == 2 || bk == 6 || bv == 6) ? 16
         : G >= 6                                     ? 8
                                                      : 16;
}
template <int BK, int BV, int G>
constexpr int epl_for() {
  return epl_of(BK, BV, G);
}

// Wavefronts per workgroup of a decode kernel (the host launches with the
// same function): 8, two a SIMD with at most 256 registers each, or 4 (one
// a SIMD, up to 512) where the cross-wave merge buffer (waves x G x D
// floats) would pass 32 KB of LDS, or where a wavefront's accumulators
// outgrow 256 registers by far: the MFMA kernel's G x D/gs = 16 A rows,
// G x D = 1024 value accumulators or 8 heads (30-600 registers spilled at
// 8 wavefronts; 4 measured 1.2-1.5x faster) and
// the dot2 kernel's G heads x EPL channels above 64 (200-700 spilled; 4
// measured 2.7-3.2x faster). At G x EPL = 64 the few spills of 8
// wavefronts cost less than the lost occupancy (8 measured 10-25% faster).
constexpr int decode_waves(int D, int bk, int bv, int G, int gs, bool mfma) {
  return G * D > 1024 ? 4
         : mfma       ? (G * (D / gs) >= 16 || G * D >= 1024 || G >= 8 ? 4 : 8)
                      : (G * epl_of(bk, bv, G) > 64 ? 4 : 8);
}

// The dot2 kernel serves 6 or 8 heads a KV head in one launch only with 8
// channels a lane (registers); wider lanes take the group in two launches of
// half the heads each (split_heads).
template <int BK, int BV>
constexpr bool split_heads(int G) {
  return G >= 6 && epl_for<BK, BV, 8>() > 8;
}

template <int D, int BK, int BV, int G>
KernelFn pick_kernel() {
  constexpr int EPL = epl_for<BK, BV, G>();
  return decode_affine_kernel<D, BK, BV, G, EPL, decode_waves(D, BK, BV, G, 64, false)>;
}

// G heads in one launch, or (split_heads) the G / 2 kernel for each half.
template <int D, int BK, int BV>
KernelFn pick_g(int G) {
  if (split_heads<BK, BV>(G)) G /= 2;
  switch (G) {
    case 1: return pick_kernel<D, BK, BV, 1>();
    case 2: return pick_kernel<D, BK, BV, 2>();
    case 3: return pick_kernel<D, BK, BV, 3>();
    case 4: return pick_kernel<D, BK, BV, 4>();
    case 6:
      if constexpr (split_heads<BK, BV>(6)) return nullptr;
      else return pick_kernel<D, BK, BV, 6>();
    case 8:
      if constexpr (split_heads<BK, BV>(8)) return nullptr;
      else return pick_kernel<D, BK, BV, 8>();
  }
  return nullptr;
}

// The (K, V) widths the decode kernels take: 3, 4 and 8 bits in any pair,
// and 2, 5 and 6 bits with the same width for keys and values.
#define TQKV_DECODE_PAIRS(X)                                                         \
  X(3, 3) X(4, 4) X(8, 8) X(3, 4) X(4, 3) X(3, 8) X(8, 3) X(4, 8) X(8, 4) X(2, 2) \
  X(5, 5) X(6, 6)

template <int D>
KernelFn pick_bits(int bk, int bv, int G) {
#define TQKV_PAIR(K, V) \
  if (bk == K && bv == V) return pick_g<D, K, V>(G);
  TQKV_DECODE_PAIRS(TQKV_PAIR)
#undef TQKV_PAIR
  return nullptr;
}

// Whether the dot2 kernel takes this (K, V, G) in two launches of G / 2.
inline bool split_heads_rt(int bk, int bv, int G) {
#define TQKV_PAIR(K, V) \
  if (bk == K && bv == V) return split_heads<K, V>(G);
  TQKV_DECODE_PAIRS(TQKV_PAIR)
#undef TQKV_PAIR
  return false;
}

// Channels a lane holds in the dot2 kernel for these widths and heads.
inline int epl_rt(int bk, int bv, int G) {
  if (bk == 3 || bv == 3 || bk == 5 || bv == 5) return 32;
  if (bk == 2 || bv == 2 || bk == 6 || bv == 6) return 16;
  return G >= 6 ? 8 : 16;
}

// One translation unit per head_dim instantiates its kernels.
KernelFn pick_d64(int bk, int bv, int G);
KernelFn pick_d128(int bk, int bv, int G);
KernelFn pick_d256(int bk, int bv, int G);
KernelFn pick_d512(int bk, int bv, int G);

}  // namespace decode
}  // namespace tqkv
