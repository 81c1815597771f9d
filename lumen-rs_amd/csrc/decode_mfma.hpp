// Fused decode attention over affine-packed K/V with scores on the matrix
// cores (MFMA) and values on VALU dot2.
//
// Why MFMA for a bandwidth-bound kernel: at 3 bits the dot2 kernel spends one
// v_dot2 per two codes per query head on the keys alone, which keeps VALU
// busy enough to cap the stream well below HBM speed. Here the keys cost one
// AND per two codes whatever the number of heads, and the matrix cores do the
// multiply-adds beside the VALU work.
//
// Step = 16 consecutive tokens of one (batch row, KV head).
//   Keys: lane l takes token l % 16 and the channel quarter l / 16 of its row
//   (D/4 channels), turns the packed codes into f16 subnormals with one AND
//   per pair (plans in pair_plans.hpp) and feeds them as the B operand
//   (K = channels, N = 16 tokens) of v_mfma_f32_16x16x32_f16. The A operand
//   holds the queries, one row per (query head, quantization group): row
//   (h, g) keeps q_h on the channels of group g and zero elsewhere, so the
//   16x16 result holds per-group partial dots q_h . c_g for every token and
//   the per-(token, group) affine scale and bias apply afterwards:
//     score = sum_g scale_g * dot_g + bias_g * sum(q_h over g).
//   Queries are pre-scaled per channel by 2^(E_h - o) (o = the code's bit
//   offset in its f16 half) as in the dot2 kernel, so every product carries
//   the same 2^(E_h - 24).
//   Values: lanes take the token pair (j, j + 8) of the step per 8-lane
//   group j (D/8 channels a lane; each load instruction then reads 8 whole
//   consecutive rows)
//   and accumulate c_t0 * w_t0 + c_t1 * w_t1 with v_dot2 on codes merged from
//   the two tokens' rows, w = softmax weight * scale as an f16 pair; the
//   weights come from the score lanes by ds_bpermute.
// The softmax maximum is uniform across the wavefront and lags the true one
// by up to kTau (log2 units); it is recomputed (a 16-lane reduction plus one
// readlane per head) only on steps where some score passes it by more.
// Requirements: D in {64, 128, 256}; H/H_kv * D/group <= 16 (the A rows);
// group a multiple of D/8; plans for (bits_k, D/4) and (bits_v, D/8).
#pragma once

#include "affine_quantize.hpp"
#include "decode_affine.hpp"

namespace tqkv {
namespace decode {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// The lane widths gen_pair_plans.py writes plans for.
template <int BITS, int EPL>
constexpr bool has_plan() {
  return ((BITS == 3 || BITS == 5) && (EPL == 32 || EPL == 64)) ||
         ((BITS == 2 || BITS == 6) && (EPL == 16 || EPL == 32 || EPL == 64)) ||
         ((BITS == 4 || BITS == 8) && (EPL == 8 || EPL == 16 || EPL == 32 || EPL == 64));
}

template <int D, int BK, int BV, int G, int NG>
constexpr bool mfma_layout_ok() {
  // G * D <= 1024: the value accumulators (G x D/8 a lane) fit a
  // wavefront's registers (at 2048, 700+ spilled even with four wavefronts).
  return (D == 64 || D == 128 || D == 256) && has_plan<BK, D / 4>() && has_plan<BV, D / 8>() &&
         G * NG <= 16 && G * D <= 1024 && (D / NG) % (D / 8) == 0;
}

typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bf2_t as_bf2(uint32_t x) { return __builtin_bit_cast(bf2_t, x); }

// Cache policy of the streamed cache reads: non-temporal.
constexpr int kNonTemporal = 2;

// A raw buffer descriptor over `bytes` bytes at `base` (32-bit data, no
// swizzle; the size must fit 32 bits, which the host checks).
__device__ __forceinline__ rsrc_t buffer_rsrc(const void* base, uint64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), short(0), int(uint32_t(bytes)),
                                           0x00020000);
}

// N consecutive words at byte offset voff + soff of a buffer, widest first.
template <int N>
__device__ __forceinline__ void buffer_words(uint32_t* dst, rsrc_t r, uint32_t voff,
                                             uint32_t soff) {
  if constexpr (N >= 4) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kNonTemporal);
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
    dst[3] = v.w;
    if constexpr (N > 4) buffer_words<N - 4>(dst + 4, r, voff + 16, soff);
  } else if constexpr (N == 3) {
    const u32x3_t v = __builtin_amdgcn_raw_buffer_load_b96(r, voff, soff, kNonTemporal);
    dst[0] = v.x;
    dst[1] = v.y;
    dst[2] = v.z;
  } else if constexpr (N == 2) {
    const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kNonTemporal);
    dst[0] = v.x;
    dst[1] = v.y;
  } else if constexpr (N == 1) {
    dst[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, kNonTemporal);
  }
}

// Max over the 16 lanes of a DPP row, every lane getting it.
__device__ __forceinline__ float row_max16(float v) {
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x),
                                                      decltype(ctrl)::value, 0xf, 0xf, true));
  };
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0xb1>{}));   // quad [1,0,3,2]
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x4e>{}));   // quad [2,3,0,1]
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x141>{}));  // half-row mirror
  v = fmaxf(v, dpp(v, std::integral_constant<int, 0x140>{}));  // row mirror
  return v;
}

// Sum over the 16 lanes of a DPP row, every lane getting it (the pairings
// of row_max16).
__device__ __forceinline__ float row_sum16(float v) {
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x),
                                                      decltype(ctrl)::value, 0xf, 0xf, true));
  };
  v += dpp(v, std::integral_constant<int, 0xb1>{});
  v += dpp(v, std::integral_constant<int, 0x4e>{});
  v += dpp(v, std::integral_constant<int, 0x141>{});
  v += dpp(v, std::integral_constant<int, 0x140>{});
  return v;
}

// The wavefront's max / sum from row-reduced values (every lane of a row
// holding its row's result), as a wave-uniform value: one readlane a row.
__device__ __forceinline__ float rl(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ float rows_max(float v) {
  return fmaxf(fmaxf(rl(v, 0), rl(v, 16)), fmaxf(rl(v, 32), rl(v, 48)));
}
__device__ __forceinline__ float rows_sum(float v) {
  return (rl(v, 0) + rl(v, 16)) + (rl(v, 32) + rl(v, 48));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Rows of a page of the page-sparse decode, and the most pages one
// wavefront may cover (one page number a lane).
constexpr int kPageRows = 64;
constexpr int kMaxWavePages = 64;

// PAGED: segment 0's rows [0, n0) are the chosen 64-row pages of the slab
// (Args::pages). Wavefront ranges are whole pages; a wavefront reads its
// page numbers once (lane j holds its j-th page), and each 16-token step
// takes its page's physical row with a readlane, so the pipeline runs
// across pages as over contiguous rows.
template <int D, int BK, int BV, int G, int NG, int kWaves, bool PAGED = false>
__global__ __launch_bounds__(kWave* kWaves) void decode_mfma_kernel(Args a) {
  constexpr int EK = D / 4, EV = D / 8;
  constexpr int KW = EK * BK / 32, VW = EV * BV / 32;
  constexpr int KROW = D * BK / 32, VROW = D * BV / 32;
  constexpr int GS = D / NG;
  constexpr int M = G * NG;
  constexpr int HPL = NG >= 4 ? 1 : 4 / NG;  // query heads per key lane
  constexpr int RPH = NG >= 4 ? 4 : NG;      // result rows per head in a lane
  constexpr int NSC = NG >= 4 ? 4 : NG;      // key scales a lane reads per token
  constexpr int NSW = (NSC + 1) / 2;         // ... as words of bf16 pairs
  constexpr int kStep = 16;
  using KP = Plan<BK, EK>;
  using VP = Plan<BV, EV>;
  constexpr int NM = (KP::kN + 3) / 4;
  static_assert(mfma_layout_ok<D, BK, BV, G, NG>(), "layout");

  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  // readfirstlane: the compiler then knows the wave index (and every range
  // and buffer descriptor derived from it) is uniform.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int kt = lane & 15, kj = lane >> 4;  // key lane: token, channel quarter
  const int vp = lane >> 3, vc = lane & 7;   // value lane: token pair, channel chunk
  const int ve0 = vc * EV;
  const int vgrp = ve0 / GS;

  // ---- queries: f32 in LDS, then per-head exponents and group sums. Lane
  // l reads channel l of every 64-channel chunk, and the G * (D/64 + 1)
  // reductions run side by side (DPP within rows of 16 lanes, then one
  // readlane a row): their results are wave-uniform and no reduction waits
  // on another. A group of 64 channels is a chunk's four rows; of 32, two
  // rows; of 128, two chunks.
  static_assert(GS == 32 || GS == 64 || GS == 128, "group size");
  constexpr int NCH = D / kWave;
  __shared__ float s_q[G][D];
  for (int i = threadIdx.x; i < G * D; i += kWave * kWaves) {
    const int h = i / D, d = i % D;
    s_q[h][d] = bf16_to_f32(a.q[(int64_t(b) * a.H + kvh * a.Gt + a.h_off + h) * D + d]);
  }
  __syncthreads();
  int E[G];
  float qsum[G][NG];
  {
    float mx[G], rs[G][NCH];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      mx[h] = 0.0f;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        const float x = s_q[h][c * kWave + lane];
        mx[h] = fmaxf(mx[h], fabsf(x));
        rs[h][c] = row_sum16(x);
      }
      mx[h] = row_max16(mx[h]);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float m = rows_max(mx[h]);
      int ex = 0;
      if (m > 0.0f) frexpf(m, &ex);
      E[h] = 15 - ex;
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if constexpr (GS == 64) {
          qsum[h][c] = rows_sum(rs[h][c]);
        } else if constexpr (GS == 32) {
          qsum[h][2 * c] = rl(rs[h][c], 0) + rl(rs[h][c], 16);
          qsum[h][2 * c + 1] = rl(rs[h][c], 32) + rl(rs[h][c], 48);
        } else {
          if (c % 2 == 0)
            qsum[h][c / 2] = rows_sum(rs[h][c]);
          else
            qsum[h][c / 2] += rows_sum(rs[h][c]);
        }
      }
    }
  }

  // A operand: row kt = (head, group); this lane supplies the k slots of
  // channel quarter kj.
  h8_t aq[NM];
  {
    const int m = kt;
    const int h = m / NG, g = m % NG;
    const bool row_ok = m < M;
    const int hq = row_ok ? h : 0;  // padding rows read a real row, then drop it
    int Eh = 0;
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
      if (hh == h) Eh = E[hh];
    static_for<NM>([&](auto I) {
      h8_t v;
      static_for<8>([&](auto S) {
        constexpr int J = 4 * decltype(I)::value + decltype(S)::value / 2;
        float val = 0.0f;
        if constexpr (J < KP::kN) {
          constexpr KOp op = KP::k[J];
          constexpr bool lo = decltype(S)::value % 2 == 0;
          constexpr int e = lo ? op.lo_e : op.hi_e;
          constexpr int o = lo ? op.lo_o : op.hi_o;
          if constexpr (e >= 0) {
            // An unconditional read times 0 or 1 (a select would be turned
            // back into a branch around the read): the reads issue back to
            // back instead of one wait each.
            const int ch = kj * EK + e;
            const float x = s_q[hq][ch];
            val = __builtin_ldexpf(x, Eh - o) * ((row_ok && ch / GS == g) ? 1.0f : 0.0f);
          }
        }
        v[decltype(S)::value] = _Float16(val);
      });
      aq[decltype(I)::value] = v;
    });
  }

  // Score constants of this lane's four result rows 4 * kj + r.
  float kf[4], qb[4];
  int hl[HPL];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * kj + r;
    const int h = m / NG, g = m % NG;
    kf[r] = 0.0f;
    qb[r] = 0.0f;
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
#pragma unroll
      for (int gg = 0; gg < NG; ++gg) {
        if (m < M && hh == h && gg == g) {
          kf[r] = a.qscale * __builtin_ldexpf(1.0f, 24 - E[hh]);
          qb[r] = a.qscale * qsum[hh][gg];
        }
      }
    }
  }
#pragma unroll
  for (int hh = 0; hh < HPL; ++hh) hl[hh] = (4 * kj + hh * RPH) / NG;

  // ---- fused append: the last wavefront of the unit's last split quantizes
  // the new K row (lanes [0, 32)) and V row (lanes [32, 64)), D / 16 lanes a
  // row, writes both into the cache and keeps them in LDS for one more key
  // step after its range. LDS accesses of one wavefront complete in order,
  // so its lanes read what its lanes wrote without a workgroup barrier.
  __shared__ uint64_t s_ach[2][D / 8];
  __shared__ uint32_t s_akw[KROW], s_avw[VROW];
  __shared__ uint16_t s_aks[NG], s_akb[NG], s_avs[NG], s_avb[NG];
  const bool app = a.app_k != nullptr && split == int(gridDim.x) - 1 && wave == kWaves - 1;
  if (app) {
    constexpr int LPR = D / aq::kLaneElems;
    const int tv = lane >> 5, lir = lane & 31;
    const int li = lir < LPR ? lir : LPR - 1;  // idle lanes repeat a live one
    const int64_t slab = int64_t(b) * a.H_kv + kvh;
    float x[aq::kLaneElems];
    aq::load_lane((tv ? a.app_v : a.app_k) + slab * D + li * aq::kLaneElems, x);
    const aq::LaneCodes qc = aq::quantize_lane(x, a.gs, tv ? BV : BK);
    const int lpg = a.gs / aq::kLaneElems;
    const int64_t dst = slab * a.app_cap + a.app_row;
    if (lir < LPR) {
      if (lir % lpg == 0) {
        const int g = lir / lpg;
        const uint16_t sc = f32_to_bf16(qc.scale), bi = f32_to_bf16(qc.bias);
        (tv ? a.app_vs : a.app_ks)[dst * NG + g] = sc;
        (tv ? a.app_vb : a.app_kb)[dst * NG + g] = bi;
        (tv ? s_avs : s_aks)[g] = sc;
        (tv ? s_avb : s_akb)[g] = bi;
      }
      s_ach[tv][2 * lir] = qc.chunk[0];
      s_ach[tv][2 * lir + 1] = qc.chunk[1];
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    for (int w = lane; w < KROW; w += kWave) {
      const uint32_t word = aq::packed_word(s_ach[0], w, BK);
      a.app_kw[dst * KROW + w] = word;
      s_akw[w] = word;
    }
    for (int w = lane; w < VROW; w += kWave) {
      const uint32_t word = aq::packed_word(s_ach[1], w, BV);
      a.app_vw[dst * VROW + w] = word;
      s_avw[w] = word;
    }
  }

  // ---- this wavefront's keys
  const int64_t t_begin = int64_t(split) * a.split_len;
  const int64_t t_end = t_begin + a.split_len < a.total ? t_begin + a.split_len : a.total;
  int64_t chunk = (t_end - t_begin + kWaves - 1) / kWaves;
  constexpr int kChunkAlign = PAGED ? kPageRows : kStep;  // paged: whole pages
  chunk = (chunk + kChunkAlign - 1) / kChunkAlign * kChunkAlign;
  const int64_t w_begin = t_begin + wave * chunk;
  const int64_t w_end = w_begin + chunk < t_end ? w_begin + chunk : t_end;

  // ev[h]: a wave-uniform exponent folded into head h's softmax reference
  // (weights are 2^(s - m - ev)), raised only when a value weight p * scale
  // would leave the f16 range (see values()).
  float m[G], l[G], bacc[G], mlane[HPL], ev[G];
  float acc[G][EV];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    ev[h] = 0.0f;
    m[h] = -INFINITY;
    l[h] = 0.0f;
    bacc[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < EV; ++e) acc[h][e] = 0.0f;
  }
#pragma unroll
  for (int hh = 0; hh < HPL; ++hh) mlane[hh] = hl[hh] < G ? -INFINITY : 0.0f;

  // Loads: one buffer descriptor per array over the rows of the range being
  // walked (base and size wave-uniform, in SGPRs), the lane's offset in a
  // VGPR and the step's offset in an SGPR, so stepping costs no VALU work.
  // Every access is in range by construction; the descriptors' size checks
  // (reads past them return zeros) are a second line of defence.
  // Keys and values of a step load into separate buffers: the pipeline below
  // scores step i + 1 while it accumulates the values of step i.
  struct KBuf {
    uint32_t kw[KW];
    uint32_t ks[NSW], kb[NSW];
  };
  struct VBuf {
    uint32_t vw[2][VW];
    uint32_t vs[2], vb[2];  // bf16 in the low half
  };
  // A scored step's weights, as this value lane needs them: tokens j and
  // j + 8 of the step for every head.
  struct Pend {
    float p0[G], p1[G];
  };
  struct Rsrc {
    rsrc_t kw, ks, kb, vw, vs, vb;
  };
  auto make = [&](const Seg& s, int64_t row0, uint32_t nrows) {
    Rsrc r;
    r.kw = buffer_rsrc(s.kw + row0 * KROW, uint64_t(nrows) * KROW * 4);
    r.ks = buffer_rsrc(s.ks + row0 * NG, uint64_t(nrows) * NG * 2);
    r.kb = buffer_rsrc(s.kb + row0 * NG, uint64_t(nrows) * NG * 2);
    r.vw = buffer_rsrc(s.vw + row0 * VROW, uint64_t(nrows) * VROW * 4);
    r.vs = buffer_rsrc(s.vs + row0 * NG, uint64_t(nrows) * NG * 2);
    r.vb = buffer_rsrc(s.vb + row0 * NG, uint64_t(nrows) * NG * 2);
    return r;
  };
  // Loads of step `step`; rows are relative to the step's first token.
  auto load_k = [&](KBuf& f, const Rsrc& r, uint32_t step, uint32_t krow) {
    const uint32_t k_so = step * uint32_t(kStep * KROW * 4);
    const uint32_t s_so = step * uint32_t(kStep * NG * 2);
    buffer_words<KW>(f.kw, r.kw, (krow * KROW + kj * KW) * 4, k_so);
    const uint32_t ks_off = (krow * NG + (4 * kj) % NG) * 2;
    if constexpr (NSC == 1) {
      f.ks[0] = __builtin_amdgcn_raw_buffer_load_b16(r.ks, ks_off, s_so, kNonTemporal);
      f.kb[0] = __builtin_amdgcn_raw_buffer_load_b16(r.kb, ks_off, s_so, kNonTemporal);
    } else {
      buffer_words<NSW>(f.ks, r.ks, ks_off, s_so);
      buffer_words<NSW>(f.kb, r.kb, ks_off, s_so);
    }
  };
  auto load_v = [&](VBuf& f, const Rsrc& r, uint32_t step, uint32_t vrow0, uint32_t vrow1) {
    const uint32_t s_so = step * uint32_t(kStep * NG * 2);
    const uint32_t v_so = step * uint32_t(kStep * VROW * 4);
    buffer_words<VW>(f.vw[0], r.vw, (vrow0 * VROW + vc * VW) * 4, v_so);
    buffer_words<VW>(f.vw[1], r.vw, (vrow1 * VROW + vc * VW) * 4, v_so);
    f.vs[0] = __builtin_amdgcn_raw_buffer_load_b16(r.vs, (vrow0 * NG + vgrp) * 2, s_so, kNonTemporal);
    f.vs[1] = __builtin_amdgcn_raw_buffer_load_b16(r.vs, (vrow1 * NG + vgrp) * 2, s_so, kNonTemporal);
    f.vb[0] = __builtin_amdgcn_raw_buffer_load_b16(r.vb, (vrow0 * NG + vgrp) * 2, s_so, kNonTemporal);
    f.vb[1] = __builtin_amdgcn_raw_buffer_load_b16(r.vb, (vrow1 * NG + vgrp) * 2, s_so, kNonTemporal);
  };
  auto scale_of = [](const uint32_t* w, int i) {
    const uint32_t x = w[i / 2];
    return __uint_as_float((i % 2) == 0 ? (x << 16) : (x & 0xffff0000u));
  };
  // The bias term sum_g bias_g * qsum_g runs as bf16 dot2 against the query
  // sums split in a bf16 high and low part (~16 significant bits).
  constexpr int QP = RPH >= 2 ? RPH / 2 : 1;
  uint32_t qbh[HPL][QP], qbl[HPL][QP];
#pragma unroll
  for (int hh = 0; hh < HPL; ++hh) {
#pragma unroll
    for (int w = 0; w < QP; ++w) {
      float x0 = qb[hh * RPH + 2 * w], x1 = RPH >= 2 ? qb[hh * RPH + 2 * w + 1] : 0.0f;
      const uint16_t h0 = f32_to_bf16(x0), h1 = f32_to_bf16(x1);
      const uint16_t l0 = f32_to_bf16(x0 - bf16_to_f32(h0)), l1 = f32_to_bf16(x1 - bf16_to_f32(h1));
      qbh[hh][w] = uint32_t(h0) | uint32_t(h1) << 16;
      qbl[hh][w] = uint32_t(l0) | uint32_t(l1) << 16;
    }
  }
  // mtau: the lane's running maximum plus kTau (+inf on padding rows, which
  // never move it).
  float mtau[HPL];
#pragma unroll
  for (int hh = 0; hh < HPL; ++hh) mtau[hh] = hl[hh] < G ? -INFINITY : INFINITY;

  // Scores of a step and their softmax weights, handed to the value lanes.
  // When the (uniform) maximum moves, everything accumulated so far and the
  // weights `prev` of the step still waiting for its values are rescaled.
  // kMasked: keys past the range are in this step (scores -inf).
  auto score = [&](const KBuf& f, bool kvalid, auto masked, Pend& prev, Pend& out) {
    constexpr bool kMasked = decltype(masked)::value;
    // Per-group partial dots of the 16 tokens on the matrix cores.
    f4_t c = {0.0f, 0.0f, 0.0f, 0.0f};
    static_for<NM>([&](auto I) {
      uint32_t bw[4];
      static_for<4>([&](auto S) {
        constexpr int J = 4 * decltype(I)::value + decltype(S)::value;
        if constexpr (J < KP::kN) {
          constexpr KOp op = KP::k[J];
          bw[decltype(S)::value] = window<KW, op.bit>(f.kw) & op.mask;
        } else {
          bw[decltype(S)::value] = 0u;
        }
      });
      const h8_t bv = __builtin_bit_cast(h8_t, (u32x4_t{bw[0], bw[1], bw[2], bw[3]}));
      c = __builtin_amdgcn_mfma_f32_16x16x32_f16(aq[decltype(I)::value], bv, c, 0, 0, 0);
    });
    float s[HPL];
#pragma unroll
    for (int hh = 0; hh < HPL; ++hh) {
      float sd = 0.0f;
#pragma unroll
      for (int rr = 0; rr < RPH; ++rr) {
        const int r = hh * RPH + rr;
        sd = fmaf(scale_of(f.ks, r % NSC), c[r], sd);
      }
      float sb = 0.0f;
      if constexpr (RPH == 1) {
        sb = scale_of(f.kb, 0) * qb[hh];
      } else {
#pragma unroll
        for (int w = 0; w < QP; ++w) {
          const uint32_t kbw = f.kb[((hh * RPH) % NSC) / 2 + w];
          sb = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(kbw), as_bf2(qbh[hh][w]), sb, false);
          sb = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(kbw), as_bf2(qbl[hh][w]), sb, false);
        }
      }
      float acc_s = fmaf(kf[hh * RPH], sd, sb);
      if constexpr (NG >= 8) acc_s += __shfl_xor(acc_s, 16, kWave);
      if constexpr (NG >= 16) acc_s += __shfl_xor(acc_s, 32, kWave);
      s[hh] = (!kMasked || kvalid) ? acc_s : -INFINITY;
    }

    bool need = false;
#pragma unroll
    for (int hh = 0; hh < HPL; ++hh) need |= s[hh] > mtau[hh];
    if (__any(need)) {
      float smax[HPL];
#pragma unroll
      for (int hh = 0; hh < HPL; ++hh) smax[hh] = row_max16(s[hh]);
      static_for<G>([&](auto Hc) {
        constexpr int h = decltype(Hc)::value;
        constexpr int src = NG >= 4 ? 16 * (h * NG / 4) : 16 * (h / HPL);
        constexpr int reg = NG >= 4 ? 0 : h % HPL;
        const float smf = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(smax[reg]), src));
        if (smf > m[h] + kTau) {
          const float fct = m[h] == -INFINITY ? 0.0f : exp2f(m[h] - smf);
          m[h] = smf;
          l[h] *= fct;
          bacc[h] *= fct;
          prev.p0[h] *= fct;
          prev.p1[h] *= fct;
#pragma unroll
          for (int e = 0; e < EV; ++e) acc[h][e] *= fct;
        }
      });
#pragma unroll
      for (int hh = 0; hh < HPL; ++hh) {
#pragma unroll
        for (int h = 0; h < G; ++h)
          if (hl[hh] == h) {
            mlane[hh] = m[h] + ev[h];
            mtau[hh] = m[h] + kTau;
          }
      }
    }
    float p[HPL];
#pragma unroll
    for (int hh = 0; hh < HPL; ++hh) p[hh] = __builtin_amdgcn_exp2f(s[hh] - mlane[hh]);
    static_for<G>([&](auto Hc) {
      constexpr int h = decltype(Hc)::value;
      constexpr int grp_lane = NG >= 4 ? 16 * (h * NG / 4) : 16 * (h / HPL);
      constexpr int reg = NG >= 4 ? 0 : h % HPL;
      out.p0[h] = __shfl(p[reg], grp_lane + vp, kWave);
      out.p1[h] = __shfl(p[reg], grp_lane + vp + 8, kWave);
    });
  };
  // Values of a scored step; `nxt` holds the next step's weights, already
  // scored against the same reference.
  // The f16 weight p * scale must stay finite: p <= 2^kTau, so a step whose
  // |scales| are all <= 2^(15 - kTau) is safe as it stands (the common case:
  // one max and one compare). Otherwise the products are checked, and a head
  // where one passes 2^15 moves its reference up by a power of two: every
  // accumulator and pending weight of that head is scaled down by it, exactly
  // as when the running maximum moves.
  auto values = [&](const VBuf& f, Pend& w, Pend& nxt) {
    const float vs0 = bf16_to_f32(f.vs[0]), vs1 = bf16_to_f32(f.vs[1]);
    const float vb0 = bf16_to_f32(f.vb[0]), vb1 = bf16_to_f32(f.vb[1]);
    if (__builtin_expect(__any(fmaxf(fabsf(vs0), fabsf(vs1)) > kScaleSafe), 0)) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float pm = wave_max(fmaxf(fabsf(w.p0[h] * vs0), fabsf(w.p1[h] * vs1)));
        if (pm > kWeightMax) {
          int e = 0;
          frexpf(pm * (1.0f / kWeightMax), &e);  // pm * 2^-e < kWeightMax
          const float fct = __builtin_ldexpf(1.0f, -e);
          ev[h] += float(e);
          l[h] *= fct;
          bacc[h] *= fct;
#pragma unroll
          for (int c = 0; c < EV; ++c) acc[h][c] *= fct;
          w.p0[h] *= fct;
          w.p1[h] *= fct;
          nxt.p0[h] *= fct;
          nxt.p1[h] *= fct;
#pragma unroll
          for (int hh = 0; hh < HPL; ++hh)
            if (hl[hh] == h) mlane[hh] = m[h] + ev[h];
        }
      }
    }
    uint32_t wp[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float p0 = w.p0[h], p1 = w.p1[h];
      l[h] += p0 + p1;
      bacc[h] = fmaf(p0, vb0, fmaf(p1, vb1, bacc[h]));
      wp[h] = h2_bits(h2_t{_Float16(p0 * vs0), _Float16(p1 * vs1)});
    }
    v_accumulate<BV, EV, VW, G>(f.vw[0], f.vw[1], wp, acc);
  };

  for (int sg = 0; sg < 2; ++sg) {
    const Seg& s = a.seg[sg];
    const int64_t lo = sg == 0 ? w_begin : (w_begin > a.n0 ? w_begin : a.n0);
    const int64_t hi = sg == 0 ? (w_end < a.n0 ? w_end : a.n0) : w_end;
    if (lo >= hi) continue;
    const int64_t off = sg == 0 ? 0 : a.n0;
    const bool paged = PAGED && sg == 0;
    const int64_t slab0 = int64_t(b) * s.b_stride + int64_t(kvh) * s.cap;
    const int64_t row0 = paged ? slab0 : slab0 + (lo - off);
    const uint32_t nrows = uint32_t(hi - lo);
    const uint32_t n = nrows / kStep;  // full steps (a page segment has no partial one)
    const std::integral_constant<bool, false> full{};
    const std::integral_constant<bool, true> masked{};
    if (n > 0) {
      // Iteration i: load keys of step i + 2 and values of step i + 1, score
      // step i + 1, accumulate the values of step i. Loads past the last
      // step re-read it (unconditional loads keep the buffers in place).
      // Paged: the descriptors span the slab and step i maps to the physical
      // step of its page.
      const Rsrc r = make(s, row0, paged ? uint32_t(s.cap) : n * kStep);
      const uint32_t last = n - 1;
      // Paged: lo is a page boundary; lane j holds the range's j-th page.
      int my_page = 0;
      if constexpr (PAGED) {
        if (paged) {
          const int64_t first = lo / kPageRows;
          const int npg = int((hi - lo + kPageRows - 1) / kPageRows);
          if (lane < npg) my_page = a.pages[(int64_t(b) * a.H_kv + kvh) * a.n_pages + first + lane];
        }
      }
      auto cl = [&](uint32_t x) {
        const uint32_t c = x < last ? x : last;
        if constexpr (PAGED) {
          if (paged) {
            constexpr uint32_t kSteps = kPageRows / kStep;
            const int pg = __builtin_amdgcn_readlane(my_page, int(c / kSteps));
            return uint32_t(pg) * kSteps + c % kSteps;
          }
        }
        return c;
      };
      KBuf k0, k1;
      VBuf v0, v1;
      Pend p0, p1;
#pragma unroll
      for (int h = 0; h < G; ++h) p1.p0[h] = p1.p1[h] = 0.0f;
      load_k(k0, r, cl(0), kt);
      load_k(k1, r, cl(1), kt);
      load_v(v0, r, cl(0), vp, vp + 8);
      score(k0, true, full, p1, p0);
      uint32_t i = 0;
      for (; i + 2 < n; i += 2) {
        load_k(k0, r, cl(i + 2), kt);
        load_v(v1, r, cl(i + 1), vp, vp + 8);
        score(k1, true, full, p0, p1);
        values(v0, p0, p1);
        load_k(k1, r, cl(i + 3), kt);
        load_v(v0, r, cl(i + 2), vp, vp + 8);
        score(k0, true, full, p1, p0);
        values(v1, p1, p0);
      }
      if (i + 1 < n) {
        load_v(v1, r, cl(i + 1), vp, vp + 8);
        score(k1, true, full, p0, p1);
        values(v0, p0, p1);
        values(v1, p1, p0);
      } else {
        values(v0, p0, p1);
      }
    }
    const uint32_t left = nrows - n * kStep;
    if (left > 0 && !paged) {
      // Lanes past the range re-read its last row and are masked.
      const Rsrc r = make(s, row0 + n * kStep, left);
      const uint32_t lst = left - 1;
      KBuf kf_;
      VBuf vf_;
      Pend pz, pt;
#pragma unroll
      for (int h = 0; h < G; ++h) pz.p0[h] = pz.p1[h] = 0.0f;
      load_k(kf_, r, 0, kt < left ? kt : lst);
      load_v(vf_, r, 0, vp < left ? vp : lst, vp + 8 < left ? vp + 8 : lst);
      score(kf_, kt < left, masked, pz, pt);
      values(vf_, pt, pz);
    }
  }
  if (app) {
    // The appended token: a masked step whose one key (token 0) is the new
    // row, every lane reading its share from LDS.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    KBuf kf_;
    VBuf vf_;
    Pend pz, pt;
#pragma unroll
    for (int h = 0; h < G; ++h) pz.p0[h] = pz.p1[h] = 0.0f;
#pragma unroll
    for (int i = 0; i < KW; ++i) kf_.kw[i] = s_akw[kj * KW + i];
    const int si = (4 * kj) % NG;
    if constexpr (NSC == 1) {
      kf_.ks[0] = s_aks[si];
      kf_.kb[0] = s_akb[si];
    } else {
#pragma unroll
      for (int w = 0; w < NSW; ++w) {
        kf_.ks[w] = uint32_t(s_aks[si + 2 * w]) | uint32_t(s_aks[si + 2 * w + 1]) << 16;
        kf_.kb[w] = uint32_t(s_akb[si + 2 * w]) | uint32_t(s_akb[si + 2 * w + 1]) << 16;
      }
    }
#pragma unroll
    for (int i = 0; i < VW; ++i) vf_.vw[0][i] = vf_.vw[1][i] = s_avw[vc * VW + i];
    vf_.vs[0] = vf_.vs[1] = s_avs[vgrp];
    vf_.vb[0] = vf_.vb[1] = s_avb[vgrp];
    score(kf_, kt == 0, std::integral_constant<bool, true>{}, pz, pt);
    values(vf_, pt, pz);
  }

  // ---- merge: undo the code scale, add the bias term, sum the token pairs
  // of the wavefront (its maximum is uniform), then the wavefronts via LDS.
  static_for<VP::cN>([&](auto C) {
    constexpr VCode vcd = VP::vc[decltype(C)::value];
    constexpr float unscale = float(1 << (24 - vcd.o));
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h][vcd.e] = fmaf(acc[h][vcd.e], unscale, bacc[h]);
  });
  // The 8 token-pair groups (lanes vp = lane / 8) summed as a
  // reduce-scatter: each lane ends with a quarter of the wavefront's sums.
  // v_permlane16_swap of two different registers (A, B) hands even 16-lane
  // rows their own and their lane ^ 16 partner's A and odd rows the same of
  // B, so one swap and one add fold both halves of a pair of values, each
  // into the rows that keep it; v_permlane32_swap does the same for lane ^
  // 32; the NQ values left are then summed over lane ^ 8 by DPP row_ror:8.
  // Lane bits (4, 5) = (b4, b5) keep the sums of value indices
  // i + 2 NQ b4 + NQ b5, i < NQ (acc[h][e] at h * EV + e, then l[h]).
  // (A butterfly over all G * (EV + 1) values took about three times the
  // instructions.)
  constexpr int NV = G * EV + G, NQ = (NV + 3) / 4;
  float vsum[4 * NQ];
#pragma unroll
  for (int h = 0; h < G; ++h) {
#pragma unroll
    for (int e = 0; e < EV; ++e) vsum[h * EV + e] = acc[h][e];
    vsum[G * EV + h] = l[h];
  }
#pragma unroll
  for (int k = NV; k < 4 * NQ; ++k) vsum[k] = 0.0f;
  float half[2 * NQ];
#pragma unroll
  for (int i = 0; i < 2 * NQ; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(vsum[i]),
                                                    __float_as_uint(vsum[i + 2 * NQ]), false, false);
    half[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  float quarter[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(half[i]),
                                                    __float_as_uint(half[i + NQ]), false, false);
    quarter[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    quarter[i] += __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(quarter[i]), 0x128, 0xf, 0xf, true));
  }

  __shared__ float s_m[kWaves][G], s_l[kWaves][G];
  __shared__ float s_acc[kWaves][G][D];
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) s_m[wave][h] = m[h] + ev[h];  // the reference of l and acc
  }
  if ((lane & 8) == 0) {  // lanes ^ 8 hold the same sums
    const int k0 = 2 * NQ * ((lane >> 4) & 1) + NQ * ((lane >> 5) & 1);
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int k = k0 + i;
      if (k < G * EV)
        s_acc[wave][k / EV][ve0 + k % EV] = quarter[i];
      else if (k < NV && vc == 0)
        s_l[wave][k - G * EV] = quarter[i];
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

// The MFMA kernel for a layout, or nullptr where it does not apply (the dot2
// kernel serves those). Group sizes 64 (here), 32 and 128 (decode_affine_gs_d*,
// not for page segments).
template <int D, int GS, int BK, int BV, int G, bool PAGED>
KernelFn pick_mfma_g() {
  constexpr int NG = D / GS;
  if constexpr (NG >= 1 && D % GS == 0 && mfma_layout_ok<D, BK, BV, G, NG>())
    return decode_mfma_kernel<D, BK, BV, G, NG, decode_waves(D, BK, BV, G, GS, true), PAGED>;
  else
    return nullptr;
}

template <int D, int GS, int BK, int BV, bool PAGED>
KernelFn pick_mfma_bits_g(int G) {
  switch (G) {
    case 1: return pick_mfma_g<D, GS, BK, BV, 1, PAGED>();
    case 2: return pick_mfma_g<D, GS, BK, BV, 2, PAGED>();
    case 4: return pick_mfma_g<D, GS, BK, BV, 4, PAGED>();
    case 8: return pick_mfma_g<D, GS, BK, BV, 8, PAGED>();
  }
  return nullptr;
}

template <int D, int GS, bool PAGED = false>
KernelFn pick_mfma_gs(int bk, int bv, int G) {
#define TQKV_PAIR(K, V) \
  if (bk == K && bv == V) return pick_mfma_bits_g<D, GS, K, V, PAGED>(G);
  TQKV_DECODE_PAIRS(TQKV_PAIR)
#undef TQKV_PAIR
  return nullptr;
}

// Group sizes 32 and 128 (instantiated in their own units).
KernelFn pick_mfma_gs_d64(int bk, int bv, int G, int gs);
KernelFn pick_mfma_gs_d128(int bk, int bv, int G, int gs);
KernelFn pick_mfma_gs_d256(int bk, int bv, int G, int gs);

template <int D, bool PAGED = false>
KernelFn pick_mfma(int bk, int bv, int G, int gs) {
  if (gs == 64) return pick_mfma_gs<D, 64, PAGED>(bk, bv, G);
  if constexpr (PAGED) return nullptr;
  switch (D) {
    case 64: return pick_mfma_gs_d64(bk, bv, G, gs);
    case 128: return pick_mfma_gs_d128(bk, bv, G, gs);
    case 256: return pick_mfma_gs_d256(bk, bv, G, gs);
  }
  return nullptr;
}

KernelFn pick_mfma_d64(int bk, int bv, int G, int gs, bool paged = false);
KernelFn pick_mfma_d128(int bk, int bv, int G, int gs, bool paged = false);
KernelFn pick_mfma_d256(int bk, int bv, int G, int gs, bool paged = false);

}  // namespace decode
}  // namespace tqkv
