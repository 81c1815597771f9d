// Fused decode attention over affine-packed K/V (the headline hot path).
//
// Work split: one workgroup per (token split, KV head, batch row); its four
// wavefronts take contiguous quarters of the split. Inside a wavefront, LPT =
// D / EPL lanes share one token (each lane owns EPL consecutive channels, all
// in one quantization group), so a wavefront walks TPW = 64 / LPT tokens per
// step with coalesced loads of TPW whole rows. All G = H / H_kv query heads
// of the KV head are served by the same dequantized codes (GQA broadcast).
//
// Per key and query head the lane computes scale * sum(q * code) +
// bias * sum(q) over its channels (the affine terms factor out of the inner
// loop), a butterfly over the LPT lanes finishes the score, and an online
// softmax in log2 units folds U keys at a time with one rescale. Values
// accumulate as (p * scale) * code with the bias term p * bias kept apart.
// Lane groups, then wavefronts (through LDS), merge their (max, sum, acc)
// states; each workgroup writes one split's unnormalized partial, and the last
// workgroup of a (batch row, KV head) to finish merges all its splits
// (native_quant_attention.rs:190-207 does this in a second pass): the decode
// is one kernel launch. An arrival counter per (batch row, KV head) lives in
// the workspace; the merging workgroup puts it back to zero.
//
// Decode is HBM-bound (~9-14 FLOP per byte of packed cache), so the kernel
// uses VALU reductions, not MFMA.
#pragma once

#include <cmath>

#include "common.hpp"

namespace tqkv {
namespace decode {

constexpr int kWave = 64;
constexpr int kWaves = 4;  // wavefronts per workgroup
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
  float qscale;  // softmax scale * log2(e)
  Seg seg[2];
  int64_t n0, total;
  int64_t split_len;
  int n_splits;
  int* counters;  // [B, H_kv], zero between calls
  uint16_t* out;  // [B, H, 1, D]
  float* part_o;  // [B, H, n_splits, D]
  float* part_m;  // [B, H, n_splits]
  float* part_l;  // [B, H, n_splits]
};

// Code e (compile-time) of a lane's little-endian packed words.
template <int BITS, int E>
__device__ __forceinline__ uint32_t code_at(const uint32_t* w) {
  constexpr int bit = E * BITS;
  constexpr int k = bit / 32, off = bit % 32;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  if constexpr (off + BITS <= 32) {
    return (w[k] >> off) & mask;
  } else {
    return __builtin_amdgcn_alignbit(w[k + 1], w[k], off) & mask;
  }
}

template <int BITS, int EPL, int E = 0>
__device__ __forceinline__ void unpack_all(const uint32_t* w, float* c) {
  if constexpr (E < EPL) {
    c[E] = float(code_at<BITS, E>(w));
    unpack_all<BITS, EPL, E + 1>(w, c);
  }
}

template <int N>
__device__ __forceinline__ void load_words(uint32_t* dst, const uint32_t* src) {
#pragma unroll
  for (int i = 0; i < N; ++i) dst[i] = src[i];
}

template <int D, int BK, int BV, int G, int EPL, int U>
__global__ __launch_bounds__(kWave* kWaves) void decode_affine_kernel(Args a) {
  constexpr int LPT = D / EPL;
  constexpr int TPW = kWave / LPT;
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

  // Query channels of this lane for every head of the group, pre-scaled.
  float qf[G][EPL];
  float qsum[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const uint16_t* qp = a.q + (int64_t(b) * a.H + kvh * G + h) * D + e0;
    qsum[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      qf[h][e] = bf16_to_f32(qp[e]) * a.qscale;
      qsum[h] += qf[h][e];
    }
  }

  const int64_t t_begin = int64_t(split) * a.split_len;
  const int64_t t_end = t_begin + a.split_len < a.total ? t_begin + a.split_len : a.total;
  int64_t chunk = (t_end - t_begin + kWaves - 1) / kWaves;
  chunk = (chunk + TPW - 1) / TPW * TPW;
  const int64_t w_begin = t_begin + wave * chunk;
  const int64_t w_end = w_begin + chunk < t_end ? w_begin + chunk : t_end;

  float m[G], l[G], bacc[G];
  float acc[G][EPL];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
    bacc[h] = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[h][e] = 0.0f;
  }

  for (int64_t tb = w_begin; tb < w_end; tb += int64_t(TPW) * U) {
    uint32_t kwd[U][KW], vwd[U][VW];
    float ksc[U], kbi[U], vsc[U], vbi[U];
    bool valid[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t t = tb + u * TPW + lane_tok;
      valid[u] = t < w_end;
      const int64_t tt = valid[u] ? t : w_begin;  // in-bounds row for idle lanes
      const bool second = tt >= a.n0;
      const Seg& s = second ? a.seg[1] : a.seg[0];
      const int64_t row = int64_t(b) * s.b_stride + int64_t(kvh) * s.cap + (second ? tt - a.n0 : tt);
      load_words<KW>(kwd[u], s.kw + row * KROW + lane_sub * KW);
      load_words<VW>(vwd[u], s.vw + row * VROW + lane_sub * VW);
      ksc[u] = bf16_to_f32(s.ks[row * ngroups + grp]);
      kbi[u] = bf16_to_f32(s.kb[row * ngroups + grp]);
      vsc[u] = bf16_to_f32(s.vs[row * ngroups + grp]);
      vbi[u] = bf16_to_f32(s.vb[row * ngroups + grp]);
    }

    float sc[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float c[EPL];
      unpack_all<BK, EPL>(kwd[u], c);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float dot = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) dot = fmaf(qf[h][e], c[e], dot);
        float ps = fmaf(ksc[u], dot, kbi[u] * qsum[h]);
#pragma unroll
        for (int off = 1; off < LPT; off <<= 1) ps += __shfl_xor(ps, off, kWave);
        sc[u][h] = valid[u] ? ps : -INFINITY;
      }
    }

    float p[U][G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mx = m[h];
#pragma unroll
      for (int u = 0; u < U; ++u) mx = fmaxf(mx, sc[u][h]);
      const float f = mx == -INFINITY ? 1.0f : exp2f(m[h] - mx);
      float ls = 0.0f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        p[u][h] = mx == -INFINITY ? 0.0f : exp2f(sc[u][h] - mx);
        ls += p[u][h];
      }
      m[h] = mx;
      l[h] = fmaf(l[h], f, ls);
      bacc[h] *= f;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[h][e] *= f;
    }

#pragma unroll
    for (int u = 0; u < U; ++u) {
      float c[EPL];
      unpack_all<BV, EPL>(vwd[u], c);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float pv = p[u][h] * vsc[u];
        bacc[h] = fmaf(p[u][h], vbi[u], bacc[h]);
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[h][e] = fmaf(pv, c[e], acc[h][e]);
      }
    }
  }

  // Fold the bias term, then merge the TPW lane groups of this wavefront.
#pragma unroll
  for (int h = 0; h < G; ++h) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[h][e] += bacc[h];
  }
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
    const int64_t row = (int64_t(b) * a.H + kvh * G + h) * a.n_splits + split;
    a.part_o[row * D + d] = os;
    if (d == 0) {
      a.part_m[row] = mx;
      a.part_l[row] = ls;
    }
  }

  // The last workgroup of this (batch row, KV head) to arrive merges the
  // splits: out = sum_s o_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
  __shared__ int s_last;
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) {
    int* ctr = a.counters + int64_t(b) * a.H_kv + kvh;
    const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = prev == a.n_splits - 1;
    if (s_last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  for (int i = threadIdx.x; i < G * D; i += kWave * kWaves) {
    const int h = i / D, d = i % D;
    const int64_t bh = int64_t(b) * a.H + kvh * G + h;
    const float* pm = a.part_m + bh * a.n_splits;
    const float* pl = a.part_l + bh * a.n_splits;
    const float* po = a.part_o + bh * a.n_splits * D + d;
    float mx = -INFINITY;
    for (int sp = 0; sp < a.n_splits; ++sp) mx = fmaxf(mx, __builtin_nontemporal_load(pm + sp));
    float ls = 0.0f, os = 0.0f;
    for (int sp = 0; sp < a.n_splits; ++sp) {
      const float msp = __builtin_nontemporal_load(pm + sp);
      if (msp == -INFINITY) continue;
      const float f = exp2f(msp - mx);
      ls += __builtin_nontemporal_load(pl + sp) * f;
      os += __builtin_nontemporal_load(po + int64_t(sp) * D) * f;
    }
    a.out[bh * D + d] = f32_to_bf16(ls > 0.0f ? os / ls : 0.0f);
  }
}

using KernelFn = void (*)(Args);

template <int D, int BK, int BV, int G>
KernelFn pick_kernel() {
  constexpr int EPL = (BK == 3 || BV == 3) ? 32 : (G >= 6 ? 8 : 16);
  constexpr int U = G <= 2 ? 4 : 2;
  return decode_affine_kernel<D, BK, BV, G, EPL, U>;
}

template <int D, int BK, int BV>
KernelFn pick_g(int G) {
  switch (G) {
    case 1: return pick_kernel<D, BK, BV, 1>();
    case 2: return pick_kernel<D, BK, BV, 2>();
    case 3: return pick_kernel<D, BK, BV, 3>();
    case 4: return pick_kernel<D, BK, BV, 4>();
    case 6:
      if constexpr (BK == 3 || BV == 3) return nullptr;
      else return pick_kernel<D, BK, BV, 6>();
    case 8:
      if constexpr (BK == 3 || BV == 3) return nullptr;
      else return pick_kernel<D, BK, BV, 8>();
  }
  return nullptr;
}

template <int D>
KernelFn pick_bits(int bk, int bv, int G) {
#define TQKV_PAIR(K, V) \
  if (bk == K && bv == V) return pick_g<D, K, V>(G);
  TQKV_PAIR(3, 3) TQKV_PAIR(4, 4) TQKV_PAIR(8, 8)
  TQKV_PAIR(3, 4) TQKV_PAIR(4, 3) TQKV_PAIR(3, 8)
  TQKV_PAIR(8, 3) TQKV_PAIR(4, 8) TQKV_PAIR(8, 4)
#undef TQKV_PAIR
  return nullptr;
}

// One translation unit per head_dim instantiates its kernels.
KernelFn pick_d64(int bk, int bv, int G);
KernelFn pick_d128(int bk, int bv, int G);
KernelFn pick_d256(int bk, int bv, int G);
KernelFn pick_d512(int bk, int bv, int G);

}  // namespace decode
}  // namespace tqkv
