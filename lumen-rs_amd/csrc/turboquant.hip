// TurboQuant codebook format on the device: encode (rotate, normalize,
// Lloyd-Max codes, QJL residual signs), the SimpleCache estimators, rotation,
// and fused decode attention over codebook caches.
//
// The encode and the estimators are bit-exact restatements of lumen-core's
// CPU path, so codes, scales, signs and scores equal the reference's given
// the same R and Phi: every sum runs sequentially from the index the Rust
// iterates first, products and sums round separately (__fmul_rn / __fadd_rn;
// the file is also built with -ffp-contract=off), division and square root
// are correctly rounded, and codebook decisions compare in f64:
//   compress_one            compressor.rs:61-107  (tq_encode_kernel)
//   RotationMatrix::apply   rotation.rs:91-99
//   apply_inverse           rotation.rs:102-113
//   quantize (linear scan)  lloyd_max.rs:132-144
//   project_and_pack        qjl.rs:57-74
//   estimate_..._stage1     compressor.rs:165-184 (tq_scores_kernel)
//   accumulate_weighted_value / attend_values  simple.rs:40-62, 105-118
// Rust's f32 `Sum` folds from -0.0, explicit accumulators from +0.0; the
// kernels start each sum the way the corresponding Rust line does.
#include <cmath>
#include <cstdlib>
#include <cstring>

#include "common.hpp"

namespace tqkv {
namespace tq {
namespace {

constexpr int kWave = 64;

__device__ __forceinline__ float mul(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add(float a, float b) { return __fadd_rn(a, b); }
// Correctly rounded quotient and square root. (HIP's __fsqrt_rn is the
// hardware approximation unless OCML_BASIC_ROUNDED_OPERATIONS is set; the
// plain operator and __builtin_sqrtf are correctly rounded under HIP's
// default -fhip-fp32-correctly-rounded-divide-sqrt.)
__device__ __forceinline__ float div_rn(float a, float b) { return a / b; }
__device__ __forceinline__ float sqrt_rn(float a) { return __builtin_sqrtf(a); }

// Index of the codebook level of x: the first i in 1..n-1 with x < b[i],
// minus one, or n - 1 if none (lloyd_max.rs:132-144). Binary search over the
// increasing boundaries gives the linear scan's answer, NaN included.
__device__ __forceinline__ uint32_t level_of(double x, const double* __restrict__ b, int n) {
  int lo = 1, hi = n;  // answer index in [lo, hi]; hi = n means "none"
  while (lo < hi) {
    const int mid = (lo + hi) / 2;
    if (x < b[mid]) hi = mid;
    else lo = mid + 1;
  }
  return uint32_t(lo - 1);
}

// One wavefront per row. x: f32 or bf16 rows [n_slabs, s, D]; row j of slab
// i goes to row (i * dst_cap + dst_start + j) of the outputs.
template <int D>
__global__ __launch_bounds__(kWave) void tq_encode_kernel(
    const void* __restrict__ xv, int x_bf16, int64_t s, const float* __restrict__ R,
    const double* __restrict__ bnd, const float* __restrict__ cent_f32, int n_levels,
    const float* __restrict__ phi, int m, uint8_t* __restrict__ codes, float* __restrict__ sigma,
    uint32_t* __restrict__ signs, float* __restrict__ rnorm, int64_t dst_cap, int64_t dst_start) {
  constexpr int PER = D / kWave;
  __shared__ float xs[D], ys[D], rs[D];
  __shared__ float s_scale, s_rn;
  __shared__ uint8_t cs[D];
  const int lane = threadIdx.x;
  const int64_t r = blockIdx.x;
  const int64_t dst = (r / s) * dst_cap + dst_start + (r % s);
  for (int i = lane; i < D; i += kWave)
    xs[i] = x_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(xv)[r * D + i])
                   : static_cast<const float*>(xv)[r * D + i];
  __syncthreads();
  // y = R x, each y[i] a sequential sum over j from -0.0.
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int i = lane + k * kWave;
    const float* row = R + int64_t(i) * D;
    float acc = -0.0f;
    for (int j = 0; j < D; ++j) acc = add(acc, mul(row[j], xs[j]));
    ys[i] = acc;
  }
  __syncthreads();
  if (lane == 0) {
    float ss = -0.0f;
    for (int i = 0; i < D; ++i) ss = add(ss, mul(ys[i], ys[i]));
    s_scale = sqrt_rn(div_rn(ss, float(D)));
  }
  __syncthreads();
  const float scale = s_scale;
  const bool degenerate = scale < 1e-10f;
  const float inv = degenerate ? 0.0f : div_rn(1.0f, scale);
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int i = lane + k * kWave;
    const uint8_t c = degenerate ? uint8_t(0) : uint8_t(level_of(double(mul(ys[i], inv)), bnd, n_levels));
    cs[i] = c;
    codes[dst * D + i] = c;
  }
  if (lane == 0) sigma[dst] = scale;
  if (m <= 0) return;
  __syncthreads();
  // Residual against the stage-1 reconstruction R^T (centroid * scale),
  // accumulated row by row from +0.0 as apply_inverse does.
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int i = lane + k * kWave;
    float acc = 0.0f;
    for (int j = 0; j < D; ++j) acc = add(acc, mul(R[int64_t(j) * D + i], mul(cent_f32[cs[j]], scale)));
    rs[i] = __fsub_rn(xs[i], acc);
  }
  __syncthreads();
  if (lane == 0) {
    float rn = 0.0f;
    for (int i = 0; i < D; ++i) rn = add(rn, mul(rs[i], rs[i]));
    s_rn = sqrt_rn(rn);
  }
  __syncthreads();
  if (lane == 0) rnorm[dst] = s_rn;
  // QJL signs: bit `row` = (Phi[row] . r >= 0), LSB-first in u32 words.
  const int words = (m + 31) / 32;
  for (int base = 0; base < m; base += kWave) {
    const int row = base + lane;
    bool bit = false;
    if (row < m) {
      const float* p = phi + int64_t(row) * D;
      float acc = -0.0f;
      for (int j = 0; j < D; ++j) acc = add(acc, mul(p[j], rs[j]));
      bit = acc >= 0.0f;
    }
    const uint64_t ball = __ballot(bit);
    if (lane == 0) {
      const int w0 = base / 32;
      signs[dst * words + w0] = uint32_t(ball);
      if (w0 + 1 < words) signs[dst * words + w0 + 1] = uint32_t(ball >> 32);
    }
  }
}

// The same encode for D <= 128 with SUB = 4 lanes per row. Each output is
// still the sequential sum over j that compress_one forms, but the loops run
// j outermost: a lane keeps the partial sums of its D / SUB outputs in
// registers while the matrix entries of column (or row) j reach the lanes as
// LDS reads shared by every row of the block: R transposed for y = R x and R
// as stored for the reconstruction R^T (centroid * scale), each lane's
// quarter of a matrix row padded by 4 floats so the four quarters sit in
// different banks. The sums over all D outputs (sigma, the residual norm)
// run quarter after quarter, the carry passed lane to lane. For the QJL
// signs the residual goes through LDS so each lane holds all of it, and the
// SUB lanes of a row take Phi rows in turn (Phi staged 32 rows at a time).
// tq_encode_kernel spends a wavefront per row and reads R rows strided
// across lanes; here 128 rows share one copy of R in LDS.
constexpr int kLaneSub = 4;
constexpr int kLaneBlock = 512;
constexpr int kLaneRows = kLaneBlock / kLaneSub;

__device__ __forceinline__ void load8(const void* __restrict__ xv, int x_bf16, int64_t off,
                                      float (&o)[8]) {
  if (x_bf16) {
    const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(xv) + off);
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o[2 * k] = __uint_as_float(u[k] << 16);
      o[2 * k + 1] = __uint_as_float(u[k] & 0xffff0000u);
    }
  } else {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(xv) + off);
    const float4 a = p[0], b = p[1];
    o[0] = a.x, o[1] = a.y, o[2] = a.z, o[3] = a.w, o[4] = b.x, o[5] = b.y, o[6] = b.z, o[7] = b.w;
  }
}

template <int D>
struct LaneLayout {
  static constexpr int NI = D / kLaneSub;       // outputs a lane owns
  static constexpr int SEG = NI + 4;            // padded quarter of a matrix row
  static constexpr int PS = kLaneSub * SEG;     // padded matrix row stride
  static constexpr int RS = D + 4;              // residual / Phi row stride
  static constexpr int PHI_ROWS = 32;           // Phi rows staged at a time
  static constexpr int RES = kLaneRows * RS;    // residual rows of the block
  static constexpr int MAT = D * PS > RES + PHI_ROWS * RS ? D * PS : RES + PHI_ROWS * RS;
};

template <int D>
__global__ __launch_bounds__(kLaneBlock) void tq_encode_lane_kernel(
    const void* __restrict__ xv, int x_bf16, int64_t rows, int64_t s, const float* __restrict__ R,
    const double* __restrict__ bnd, const float* __restrict__ cent_f32, int n_levels,
    const float* __restrict__ phi, int m, uint8_t* __restrict__ codes, float* __restrict__ sigma,
    uint32_t* __restrict__ signs, float* __restrict__ rnorm, int64_t dst_cap, int64_t dst_start) {
  using L = LaneLayout<D>;
  constexpr int NI = L::NI;
  __shared__ __attribute__((aligned(16))) float mat[L::MAT];
  __shared__ uint32_t code_words[(D / 4) * kLaneRows];
  __shared__ float cent_s[256];
  __shared__ double bnd_s[256];
  const int tid = threadIdx.x;
  const int vec = tid / kLaneSub, sub = tid % kLaneSub;
  const int lane = tid % kWave;
  const int first = lane & ~(kLaneSub - 1);  // lane of sub 0 of this row
  const int64_t r_raw = int64_t(blockIdx.x) * kLaneRows + vec;
  const bool valid = r_raw < rows;
  const int64_t r = valid ? r_raw : rows - 1;  // idle rows recompute the last row, store nothing
  const int64_t dst = (r / s) * dst_cap + dst_start + (r % s);
  const int i0 = sub * NI;  // first output of this lane
  for (int i = tid; i < n_levels; i += kLaneBlock) cent_s[i] = cent_f32[i], bnd_s[i] = bnd[i];
  // mat[j * PS + quarter(i) * SEG + i % NI] = R[i][j]
  for (int idx = tid; idx < D * D; idx += kLaneBlock) {
    const int i = idx / D, j = idx % D;
    mat[j * L::PS + (i / NI) * L::SEG + i % NI] = R[idx];
  }
  __syncthreads();

  // y = R x: y[i] = sum_j R[i][j] x[j] from -0.0, j in order.
  float acc[NI];
#pragma unroll
  for (int l = 0; l < NI; ++l) acc[l] = -0.0f;
  for (int j0 = 0; j0 < D; j0 += 8) {
    float x8[8];
    load8(xv, x_bf16, r * D + j0, x8);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const float4* col = reinterpret_cast<const float4*>(mat + (j0 + jj) * L::PS + sub * L::SEG);
#pragma unroll
      for (int c = 0; c < NI / 4; ++c) {
        const float4 w = col[c];
        acc[4 * c + 0] = add(acc[4 * c + 0], mul(w.x, x8[jj]));
        acc[4 * c + 1] = add(acc[4 * c + 1], mul(w.y, x8[jj]));
        acc[4 * c + 2] = add(acc[4 * c + 2], mul(w.z, x8[jj]));
        acc[4 * c + 3] = add(acc[4 * c + 3], mul(w.w, x8[jj]));
      }
    }
  }
  // sum_i y[i]^2 from -0.0, quarter after quarter.
  float ss = -0.0f;
#pragma unroll
  for (int q = 0; q < kLaneSub; ++q) {
    if (sub == q) {
#pragma unroll
      for (int l = 0; l < NI; ++l) ss = add(ss, mul(acc[l], acc[l]));
    }
    ss = __shfl(ss, first + q);
  }
  const float scale = sqrt_rn(div_rn(ss, float(D)));
  const bool degenerate = scale < 1e-10f;
  const float inv = degenerate ? 0.0f : div_rn(1.0f, scale);
#pragma unroll
  for (int q = 0; q < NI / 16; ++q) {
    uint32_t w4[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t w = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int l = 16 * q + 4 * k + b;
        const uint32_t c = degenerate ? 0u : level_of(double(mul(acc[l], inv)), bnd_s, n_levels);
        w |= c << (8 * b);
      }
      w4[k] = w;
      code_words[((i0 + 16 * q + 4 * k) / 4) * kLaneRows + vec] = w;
    }
    if (valid)
      reinterpret_cast<uint4*>(codes + dst * D + i0)[q] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
  }
  if (valid && sub == 0) sigma[dst] = scale;
  if (m <= 0) return;  // uniform: the whole block leaves together

  // Residual against R^T (centroid * scale): sum_j R[j][i] * cv[j] from +0.0.
  __syncthreads();  // every lane is done with R^T; code_words are complete
  for (int idx = tid; idx < D * D; idx += kLaneBlock) {
    const int j = idx / D, i = idx % D;
    mat[j * L::PS + (i / NI) * L::SEG + i % NI] = R[idx];
  }
  __syncthreads();
#pragma unroll
  for (int l = 0; l < NI; ++l) acc[l] = 0.0f;
  for (int wid = 0; wid < D / 4; ++wid) {
    const uint32_t w = code_words[wid * kLaneRows + vec];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const float cv = mul(cent_s[(w >> (8 * b)) & 0xffu], scale);
      const float4* row = reinterpret_cast<const float4*>(mat + (4 * wid + b) * L::PS + sub * L::SEG);
#pragma unroll
      for (int c = 0; c < NI / 4; ++c) {
        const float4 e = row[c];
        acc[4 * c + 0] = add(acc[4 * c + 0], mul(e.x, cv));
        acc[4 * c + 1] = add(acc[4 * c + 1], mul(e.y, cv));
        acc[4 * c + 2] = add(acc[4 * c + 2], mul(e.z, cv));
        acc[4 * c + 3] = add(acc[4 * c + 3], mul(e.w, cv));
      }
    }
  }
#pragma unroll
  for (int l0 = 0; l0 < NI; l0 += 8) {
    float x8[8];
    load8(xv, x_bf16, r * D + i0 + l0, x8);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[l0 + e] = __fsub_rn(x8[e], acc[l0 + e]);
  }
  float rn = 0.0f;
#pragma unroll
  for (int q = 0; q < kLaneSub; ++q) {
    if (sub == q) {
#pragma unroll
      for (int l = 0; l < NI; ++l) rn = add(rn, mul(acc[l], acc[l]));
    }
    rn = __shfl(rn, first + q);
  }
  if (valid && sub == 0) rnorm[dst] = sqrt_rn(rn);

  // QJL signs: bit `row` = (Phi[row] . r >= 0) from -0.0, LSB-first u32
  // words. The residual rows go to mat[0, RES) and Phi rows to the rest.
  __syncthreads();  // every lane is done with R
  float* res = mat;
  float* phis = mat + L::RES;
#pragma unroll
  for (int c = 0; c < NI / 4; ++c)
    reinterpret_cast<float4*>(res + vec * L::RS + i0)[c] =
        make_float4(acc[4 * c], acc[4 * c + 1], acc[4 * c + 2], acc[4 * c + 3]);
  __syncthreads();
  float rf[D];
#pragma unroll
  for (int c = 0; c < D / 4; ++c) {
    const float4 e = reinterpret_cast<const float4*>(res + vec * L::RS)[c];
    rf[4 * c] = e.x, rf[4 * c + 1] = e.y, rf[4 * c + 2] = e.z, rf[4 * c + 3] = e.w;
  }
  const int words = (m + 31) / 32;
  for (int base = 0; base < m; base += L::PHI_ROWS) {
    const int nr = m - base < L::PHI_ROWS ? m - base : L::PHI_ROWS;
    __syncthreads();  // the previous rows are consumed
    for (int idx = tid; idx < nr * D; idx += kLaneBlock)
      phis[(idx / D) * L::RS + idx % D] = phi[int64_t(base) * D + idx];
    __syncthreads();
    uint32_t word = 0;
    constexpr int T = L::PHI_ROWS / kLaneSub;
    float a[T];
#pragma unroll
    for (int t = 0; t < T; ++t) a[t] = -0.0f;
#pragma unroll
    for (int c = 0; c < D / 4; ++c) {
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int rr = kLaneSub * t + sub;
        const float4 e = reinterpret_cast<const float4*>(phis + (rr < nr ? rr : 0) * L::RS)[c];
        a[t] = add(a[t], mul(e.x, rf[4 * c + 0]));
        a[t] = add(a[t], mul(e.y, rf[4 * c + 1]));
        a[t] = add(a[t], mul(e.z, rf[4 * c + 2]));
        a[t] = add(a[t], mul(e.w, rf[4 * c + 3]));
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      const int rr = kLaneSub * t + sub;
      if (rr < nr && a[t] >= 0.0f) word |= 1u << rr;
    }
    word |= __shfl_xor(word, 1);
    word |= __shfl_xor(word, 2);
    if (valid && sub == 0) signs[dst * words + base / 32] = word;
  }
}

// y = x M with M = R (transpose = 0) or R^T, the same fmaf chain over j from
// 0.0 as tq_rotate_rows_kernel, laid out as tq_encode_lane_kernel: SUB lanes
// a row, each holding D / SUB outputs, M's row j read from LDS by every row
// of the block (tq_rotate_rows_kernel reads all of R from L2 for each row).
template <int D>
__global__ __launch_bounds__(kLaneBlock) void tq_rotate_lane_kernel(const uint16_t* __restrict__ x,
                                                                    int64_t rows,
                                                                    const float* __restrict__ R,
                                                                    int transpose,
                                                                    uint16_t* __restrict__ y) {
  using L = LaneLayout<D>;
  constexpr int NI = L::NI;
  __shared__ __attribute__((aligned(16))) float mat[D * L::PS];
  const int tid = threadIdx.x;
  const int vec = tid / kLaneSub, sub = tid % kLaneSub;
  const int64_t r_raw = int64_t(blockIdx.x) * kLaneRows + vec;
  const bool valid = r_raw < rows;
  const int64_t r = valid ? r_raw : rows - 1;
  const int i0 = sub * NI;
  // mat[j * PS + quarter(i) * SEG + i % NI] = M[j][i]
  for (int idx = tid; idx < D * D; idx += kLaneBlock) {
    const int a = idx / D, b = idx % D;  // R[a][b]
    const int j = transpose ? b : a, i = transpose ? a : b;
    mat[j * L::PS + (i / NI) * L::SEG + i % NI] = R[idx];
  }
  __syncthreads();
  float acc[NI];
#pragma unroll
  for (int l = 0; l < NI; ++l) acc[l] = 0.0f;
  for (int j0 = 0; j0 < D; j0 += 8) {
    float x8[8];
    load8(x, 1, r * D + j0, x8);
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const float4* row = reinterpret_cast<const float4*>(mat + (j0 + jj) * L::PS + sub * L::SEG);
#pragma unroll
      for (int c = 0; c < NI / 4; ++c) {
        const float4 e = row[c];
        acc[4 * c + 0] = fmaf(x8[jj], e.x, acc[4 * c + 0]);
        acc[4 * c + 1] = fmaf(x8[jj], e.y, acc[4 * c + 1]);
        acc[4 * c + 2] = fmaf(x8[jj], e.z, acc[4 * c + 2]);
        acc[4 * c + 3] = fmaf(x8[jj], e.w, acc[4 * c + 3]);
      }
    }
  }
  if (!valid) return;
#pragma unroll
  for (int c = 0; c < NI / 8; ++c) {
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      w[k] = uint32_t(f32_to_bf16(acc[8 * c + 2 * k])) |
             (uint32_t(f32_to_bf16(acc[8 * c + 2 * k + 1])) << 16);
    reinterpret_cast<uint4*>(y + r * D + i0)[c] = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// rq = R q (the rotated query of compressor.rs:170), one wavefront.
__global__ __launch_bounds__(kWave) void tq_rotate_query_kernel(const float* __restrict__ R,
                                                                const float* __restrict__ q,
                                                                int D, float* __restrict__ rq) {
  for (int i = threadIdx.x; i < D; i += kWave) {
    float acc = -0.0f;
    for (int j = 0; j < D; ++j) acc = add(acc, mul(R[int64_t(i) * D + j], q[j]));
    rq[i] = acc;
  }
}

// Code j of vector t, stored one byte per code ([n, D] u8) ...
struct CodesU8 {
  const uint8_t* __restrict__ p;
  int D;
  __device__ __forceinline__ int operator()(int64_t t, int j) const { return p[t * D + j]; }
};
// ... or in CompressedVector::stage1_packed's layout (bitpack.rs:11-52):
// `per` = 64 / bits codes to a u64 word, code j of a vector at bits
// (j % per) * bits of word j / per, none straddling two words; `words` =
// ceil(D / per) words a vector.
struct CodesPacked {
  const uint64_t* __restrict__ p;
  int words, bits, per;
  __device__ __forceinline__ int operator()(int64_t t, int j) const {
    const uint64_t w = p[t * words + j / per];
    return int(w >> ((j % per) * bits)) & ((1 << bits) - 1);
  }
};

// Stage-1 scores: one thread per token, sum over channels from -0.0, times
// the token's scale (compressor.rs:165-184).
template <class Codes>
__global__ void tq_scores_kernel(const float* __restrict__ rq, Codes code,
                                 const float* __restrict__ sigma,
                                 const float* __restrict__ cent_f32, int D, int64_t n,
                                 float* __restrict__ scores) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n) return;
  float acc = -0.0f;
  for (int i = 0; i < D; ++i) acc = add(acc, mul(rq[i], cent_f32[code(t, i)]));
  scores[t] = mul(acc, sigma[t]);
}

// pack_codes (bitpack.rs:17-33) over n vectors of D u8 codes: one thread per
// output word.
__global__ void pack_codes_kernel(const uint8_t* __restrict__ codes, int64_t n, int D, int bits,
                                  int words, uint64_t* __restrict__ out) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n * words) return;
  const int64_t t = i / words;
  const int w = int(i - t * words), per = 64 / bits;
  const uint8_t* c = codes + t * D;
  uint64_t acc = 0;
  for (int k = 0; k < per; ++k) {
    const int j = w * per + k;
    if (j < D) acc |= uint64_t(c[j]) << (k * bits);
  }
  out[i] = acc;
}

// unpack_codes (bitpack.rs:36-49): one thread per code.
__global__ void unpack_codes_kernel(const uint64_t* __restrict__ words_in, int64_t n, int D,
                                    int bits, int words, uint8_t* __restrict__ codes) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n * D) return;
  const int64_t t = i / D;
  const CodesPacked code{words_in, words, bits, 64 / bits};
  codes[i] = uint8_t(code(t, int(i - t * D)));
}

// QJLProjector::project_query (qjl.rs:76-84): pq[row] = sum_j Phi[row][j] *
// q[j], folded from -0.0 in j order.
__global__ void tq_project_query_kernel(const float* __restrict__ phi, int m, int D,
                                        const float* __restrict__ q, float* __restrict__ pq) {
  for (int row = blockIdx.x * blockDim.x + threadIdx.x; row < m; row += gridDim.x * blockDim.x) {
    const float* p = phi + int64_t(row) * D;
    float acc = -0.0f;
    for (int j = 0; j < D; ++j) acc = add(acc, mul(p[j], q[j]));
    pq[row] = acc;
  }
}

// The QJL correction of estimate_correction_from_projection (qjl.rs:86-118):
// 0 when ||r|| < 1e-10, else ||r|| * sqrt(pi/2) / sqrt(m) * sum_i sign_i * pq_i
// with the sum folded from +0.0 in row order; sign bit i of a key is bit
// i % 32 of word i / 32 (the reference's u64 words, little-endian).
__device__ __forceinline__ float qjl_correction(const float* pq, int m, const uint32_t* sg,
                                                float rn) {
  if (rn < 1e-10f) return 0.0f;
  float sum = 0.0f;
  for (int row = 0; row < m; ++row) {
    const float sgn = ((sg[row / 32] >> (row % 32)) & 1u) ? 1.0f : -1.0f;
    sum = add(sum, mul(sgn, pq[row]));
  }
  const float scale = div_rn(mul(rn, sqrt_rn(1.57079632679489661923f)), sqrt_rn(float(m)));
  return mul(scale, sum);
}

// estimate_inner_products (compressor.rs:122-159): stage 1 as
// tq_scores_kernel plus the QJL correction of the stored residual signs.
__global__ void tq_scores_two_stage_kernel(const float* __restrict__ rq,
                                           const float* __restrict__ pq,
                                           const uint8_t* __restrict__ codes,
                                           const float* __restrict__ sigma,
                                           const float* __restrict__ cent_f32,
                                           const uint32_t* __restrict__ signs,
                                           const float* __restrict__ rnorm, int D, int m,
                                           int64_t n, float* __restrict__ scores) {
  const int64_t t = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (t >= n) return;
  const uint8_t* c = codes + t * D;
  float acc = -0.0f;
  for (int i = 0; i < D; ++i) acc = add(acc, mul(rq[i], cent_f32[c[i]]));
  const float s1 = mul(acc, sigma[t]);
  const int words = (m + 31) / 32;
  scores[t] = add(s1, qjl_correction(pq, m, signs + t * words, rnorm[t]));
}

// The GPU TurboQuant path's stage 2 (turboquant.rs:592-622): one wavefront
// per kQjlRows rows (each load of Phi serves them all); residual =
// f32(K_rot) - f32(K_dq), r_norm = sqrt(sum r^2) in channel order, sign bit
// i = (sum_d r_d * Phi[i][d] >= 0), sums from +0.0.
constexpr int kQjlRows = 4;
__global__ __launch_bounds__(kWave) void qjl_encode_stage2_kernel(
    const uint16_t* __restrict__ k_rot, const uint16_t* __restrict__ k_dq,
    const float* __restrict__ phi, int D, int m, int64_t rows, uint32_t* __restrict__ signs,
    float* __restrict__ rnorm) {
  extern __shared__ float s_r[];  // kQjlRows x D residuals
  const int64_t t0 = int64_t(blockIdx.x) * kQjlRows;
  const int nr = rows - t0 < kQjlRows ? int(rows - t0) : kQjlRows;
  const int lane = threadIdx.x;
  for (int q = 0; q < kQjlRows; ++q)
    for (int d = lane; d < D; d += kWave)
      s_r[q * D + d] = q < nr ? __fsub_rn(bf16_to_f32(k_rot[(t0 + q) * D + d]),
                                          bf16_to_f32(k_dq[(t0 + q) * D + d]))
                              : 0.0f;
  __syncthreads();
  if (lane < nr) {
    float ss = 0.0f;
    for (int d = 0; d < D; ++d) ss = add(ss, mul(s_r[lane * D + d], s_r[lane * D + d]));
    rnorm[t0 + lane] = sqrt_rn(ss);
  }
  const int words = (m + 31) / 32;
  for (int base = 0; base < m; base += kWave) {
    const int row = base + lane;
    float acc[kQjlRows] = {};
    if (row < m) {
      const float* p = phi + int64_t(row) * D;
      for (int d = 0; d < D; ++d) {
        const float pv = p[d];
#pragma unroll
        for (int q = 0; q < kQjlRows; ++q) acc[q] = add(acc[q], mul(s_r[q * D + d], pv));
      }
    }
#pragma unroll
    for (int q = 0; q < kQjlRows; ++q) {
      if (q >= nr) break;
      const uint64_t ball = __ballot(row < m && acc[q] >= 0.0f);
      if (lane == 0) {
        const int w0 = base / 32;
        signs[(t0 + q) * words + w0] = uint32_t(ball);
        if (w0 + 1 < words) signs[(t0 + q) * words + w0 + 1] = uint32_t(ball >> 32);
      }
    }
  }
}

// qjl_apply_correction_packed / _to_k_dq (turboquant.rs:624-691): one
// thread per (kQjlRows rows, channel), each load of Phi serving the rows;
// K_eff = bf16(K_dq + bf16((sum_i sign_i * Phi[i][d]) * (r_norm *
// sqrt(pi/2) / sqrt(m)))), the sum from +0.0 in i order.
__global__ void qjl_apply_correction_kernel(const uint16_t* __restrict__ k_dq,
                                            const uint32_t* __restrict__ signs,
                                            const float* __restrict__ rnorm,
                                            const float* __restrict__ phi, int D, int m,
                                            int64_t rows, uint16_t* __restrict__ k_eff) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t groups = (rows + kQjlRows - 1) / kQjlRows;
  if (i >= groups * D) return;
  const int64_t t0 = (i / D) * kQjlRows;
  const int d = int(i % D);
  const int nr = rows - t0 < kQjlRows ? int(rows - t0) : kQjlRows;
  const int words = (m + 31) / 32;
  float acc[kQjlRows] = {};
  for (int w0 = 0; w0 < words; ++w0) {
    // The rows' sign words for Phi rows 32 w0 .. + 31, loaded once.
    uint32_t sw[kQjlRows];
#pragma unroll
    for (int q = 0; q < kQjlRows; ++q) sw[q] = q < nr ? signs[(t0 + q) * words + w0] : 0u;
    const int row_end = m - 32 * w0 < 32 ? m : 32 * w0 + 32;
    for (int row = 32 * w0; row < row_end; ++row) {
      const float p = phi[int64_t(row) * D + d];
#pragma unroll
      for (int q = 0; q < kQjlRows; ++q)
        if (q < nr) acc[q] = add(acc[q], ((sw[q] >> (row % 32)) & 1u) ? p : -p);
    }
  }
  const float sc = div_rn(sqrt_rn(1.57079632679489661923f), sqrt_rn(float(m)));
#pragma unroll
  for (int q = 0; q < kQjlRows; ++q) {
    if (q >= nr) break;
    const int64_t t = t0 + q;
    const float corr = bf16_to_f32(f32_to_bf16(mul(acc[q], mul(rnorm[t], sc))));
    k_eff[t * D + d] = f32_to_bf16(add(bf16_to_f32(k_dq[t * D + d]), corr));
  }
}

// attend_values: output channel i sums, token by token in order and channel
// j by channel j, R[j][i] * (centroid * (scale * w)); tokens with |w| < 1e-10
// are skipped (simple.rs:40-62, 105-118).
template <class Codes>
__global__ void tq_values_kernel(const float* __restrict__ R, Codes code,
                                 const float* __restrict__ sigma,
                                 const float* __restrict__ cent_f32, const float* __restrict__ w,
                                 int D, int64_t n, float* __restrict__ out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= D) return;
  float acc = 0.0f;
  for (int64_t t = 0; t < n; ++t) {
    const float wt = w[t];
    if (fabsf(wt) < 1e-10f) continue;
    const float sc = mul(sigma[t], wt);
    for (int j = 0; j < D; ++j)
      acc = add(acc, mul(R[int64_t(j) * D + i], mul(cent_f32[code(t, j)], sc)));
  }
  out[i] = acc;
}

// The reference GPU cache's encode chain: lloyd_max_quantize_stage1
// (turboquant.rs:398-423) over y = x (mode 0), over y = bf16(x M) (mode 1:
// rotate_last_axis, then the encode) or over y = x M kept in f32 (mode 2:
// rotate_and_lloyd_max_quantize_stage1_fused, :720-745), M = R or R^T
// (transpose). sigma = sqrt(sum y^2 / D); code = the number of inner
// boundaries b (ascending, f32) with b <= bf16(y / sigma) (the level scan of
// lloyd_max_boundaries_inner, :310-331). One wavefront per kEncRows rows,
// lane l holding channels l + 64 k of each (each load of M serves them
// all): the rotation is tq_rotate_rows_kernel's fmaf chain over j from 0.0;
// the sum of squares runs over k in each lane, then over the lanes by an
// xor butterfly 32, 16, ..., 1 (MLX's own reduction order is not in the
// reference; this one is fixed, and the oracle restates it).
constexpr int kEncRows = 4;
template <int D>
__global__ __launch_bounds__(kWave) void tq_encode_gpu_kernel(
    const uint16_t* __restrict__ x, int64_t s, int64_t rows, const float* __restrict__ R,
    int mode, int transpose, const float* __restrict__ inner, int n_inner,
    uint8_t* __restrict__ codes, float* __restrict__ sigma, int64_t dst_cap, int64_t dst_start) {
  constexpr int PER = D / kWave;
  __shared__ float xs[kEncRows][D];
  __shared__ float bnd[256];
  const int64_t r0 = int64_t(blockIdx.x) * kEncRows;
  const int nr = rows - r0 < kEncRows ? int(rows - r0) : kEncRows;
  const int lane = threadIdx.x;
  for (int q = 0; q < kEncRows; ++q)
    for (int i = lane; i < D; i += kWave)
      xs[q][i] = q < nr ? bf16_to_f32(x[(r0 + q) * D + i]) : 0.0f;
  for (int i = lane; i < n_inner; i += kWave) bnd[i] = inner[i];
  __syncthreads();
  float y[kEncRows][PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int i = lane + k * kWave;
    if (mode == 0) {
#pragma unroll
      for (int q = 0; q < kEncRows; ++q) y[q][k] = xs[q][i];
    } else {
      float acc[kEncRows] = {};
      for (int j = 0; j < D; ++j) {
        const float rv = transpose ? R[int64_t(i) * D + j] : R[int64_t(j) * D + i];
#pragma unroll
        for (int q = 0; q < kEncRows; ++q) acc[q] = fmaf(xs[q][j], rv, acc[q]);
      }
#pragma unroll
      for (int q = 0; q < kEncRows; ++q)
        y[q][k] = mode == 1 ? bf16_to_f32(f32_to_bf16(acc[q])) : acc[q];
    }
  }
#pragma unroll
  for (int q = 0; q < kEncRows; ++q) {
    if (q >= nr) break;
    const int64_t r = r0 + q;
    float p = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) p = add(p, mul(y[q][k], y[q][k]));
#pragma unroll
    for (int off = kWave / 2; off >= 1; off >>= 1) p = add(p, __shfl_xor(p, off, kWave));
    const float sg = sqrt_rn(div_rn(p, float(D)));
    const int64_t dst = (r / s) * dst_cap + dst_start + r % s;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const float xn = bf16_to_f32(f32_to_bf16(div_rn(y[q][k], sg)));
      int lo = 0, hi = n_inner;
      while (lo < hi) {
        const int mid = (lo + hi) / 2;
        if (bnd[mid] <= xn)
          lo = mid + 1;
        else
          hi = mid;
      }
      codes[dst * D + lane + k * kWave] = uint8_t(lo);
    }
    if (lane == 0) sigma[dst] = sg;
  }
}

// y = x R (x bf16 [rows, D] -> bf16): the GPU path's rotate_last_axis
// (turboquant.rs:258-267), f32 accumulation. transpose = 1 applies R^T.
__global__ void tq_rotate_rows_kernel(const uint16_t* __restrict__ x, int64_t rows, int D,
                                      const float* __restrict__ R, int transpose,
                                      uint16_t* __restrict__ y) {
  const int64_t r = blockIdx.x;
  extern __shared__ float xr[];
  for (int j = threadIdx.x; j < D; j += blockDim.x) xr[j] = bf16_to_f32(x[r * D + j]);
  __syncthreads();
  for (int i = threadIdx.x; i < D; i += blockDim.x) {
    float acc = 0.0f;
    for (int j = 0; j < D; ++j)
      acc = fmaf(xr[j], transpose ? R[int64_t(i) * D + j] : R[int64_t(j) * D + i], acc);
    y[r * D + i] = f32_to_bf16(acc);
  }
}

}  // namespace
}  // namespace tq
}  // namespace tqkv

using namespace tqkv;
using namespace tqkv::tq;

extern "C" int32_t tqkv_tq_encode(const void* x, int32_t x_is_bf16, int64_t n_slabs, int64_t s,
                                  int32_t dim, const float* rotation, const double* boundaries,
                                  const float* centroids_f32, int32_t bits, const float* qjl,
                                  int32_t qjl_m, uint8_t* codes, float* sigma, uint32_t* signs,
                                  float* rnorm, int64_t dst_cap, int64_t dst_start,
                                  tqkv_stream stream) {
  if (bits < 1 || bits > 8) return fail(TQKV_EUNSUPPORTED, "codebook bits=%d", bits);
  if (!(dim == 64 || dim == 128 || dim == 256 || dim == 512))
    return fail(TQKV_EUNSUPPORTED, "encode dim=%d not in {64,128,256,512}", dim);
  if (n_slabs < 0 || s < 0 || dst_start < 0 || dst_start + s > dst_cap)
    return fail(TQKV_EINVAL_SHAPE, "rows [%lld, %lld) do not fit a buffer of %lld",
                (long long)dst_start, (long long)(dst_start + s), (long long)dst_cap);
  if (n_slabs == 0 || s == 0) return ok();
  if (!x || !rotation || !boundaries || !centroids_f32 || !codes || !sigma)
    return fail(TQKV_EINVAL_ARG, "null pointer");
  if (qjl_m < 0 || (qjl_m > 0 && (!qjl || !signs || !rnorm)))
    return fail(TQKV_EINVAL_ARG, "qjl_m=%d needs the QJL matrix, signs and rnorm", qjl_m);
  const int64_t rows = n_slabs * s;
  if (rows > 0x7fffffffLL) return fail(TQKV_EINVAL_SHAPE, "too many rows");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int n = 1 << bits;
  // The lane-per-row kernel loads x in 16-byte pieces and stores 16 code
  // bytes at a time; other alignments take the wavefront-per-row kernel.
  const bool aligned = (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(codes)) % 16 == 0;
  // TQKV_TQ_ENCODE_LANE=0 keeps the wavefront-per-row kernel (tests compare both).
  const char* lane_env = getenv("TQKV_TQ_ENCODE_LANE");
  if ((dim == 64 || dim == 128) && aligned && !(lane_env && strcmp(lane_env, "0") == 0)) {
    const unsigned blocks = unsigned((rows + kLaneRows - 1) / kLaneRows);
    if (dim == 64)
      hipLaunchKernelGGL(tq_encode_lane_kernel<64>, dim3(blocks), dim3(kLaneBlock), 0, st, x,
                         x_is_bf16, rows, s, rotation, boundaries, centroids_f32, n, qjl, qjl_m,
                         codes, sigma, signs, rnorm, dst_cap, dst_start);
    else
      hipLaunchKernelGGL(tq_encode_lane_kernel<128>, dim3(blocks), dim3(kLaneBlock), 0, st, x,
                         x_is_bf16, rows, s, rotation, boundaries, centroids_f32, n, qjl, qjl_m,
                         codes, sigma, signs, rnorm, dst_cap, dst_start);
    TQKV_LAUNCHED();
    return ok();
  }
#define TQKV_ENC(DIM)                                                                      \
  case DIM:                                                                                 \
    hipLaunchKernelGGL(tq_encode_kernel<DIM>, dim3(unsigned(rows)), dim3(kWave), 0, st, x,   \
                       x_is_bf16, s, rotation, boundaries, centroids_f32, n, qjl, qjl_m,     \
                       codes, sigma, signs, rnorm, dst_cap, dst_start);                      \
    break;
  switch (dim) {
    TQKV_ENC(64) TQKV_ENC(128) TQKV_ENC(256) TQKV_ENC(512)
  }
#undef TQKV_ENC
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_tq_encode_gpu_path(const uint16_t* x, int64_t n_slabs, int64_t s,
                                           int32_t dim, const float* rotation, int32_t mode,
                                           int32_t transpose, const float* boundaries_inner,
                                           int32_t bits, uint8_t* codes, float* sigma,
                                           int64_t dst_cap, int64_t dst_start,
                                           tqkv_stream stream) {
  if (bits < 1 || bits > 8) return fail(TQKV_EUNSUPPORTED, "codebook bits=%d", bits);
  if (!(dim == 64 || dim == 128 || dim == 256 || dim == 512))
    return fail(TQKV_EUNSUPPORTED, "encode dim=%d not in {64,128,256,512}", dim);
  if (mode < 0 || mode > 2) return fail(TQKV_EINVAL_ARG, "mode=%d not in {0, 1, 2}", mode);
  if (n_slabs < 0 || s < 0 || dst_start < 0 || dst_start + s > dst_cap)
    return fail(TQKV_EINVAL_SHAPE, "rows [%lld, %lld) do not fit a buffer of %lld",
                (long long)dst_start, (long long)(dst_start + s), (long long)dst_cap);
  if (n_slabs == 0 || s == 0) return ok();
  if (!x || !boundaries_inner || !codes || !sigma || (mode != 0 && !rotation))
    return fail(TQKV_EINVAL_ARG, "null pointer");
  const int64_t rows = n_slabs * s;
  if (rows > 0x7fffffffLL) return fail(TQKV_EINVAL_SHAPE, "too many rows");
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int n_inner = (1 << bits) - 1;
#define TQKV_ENC(DIM)                                                                       \
  case DIM:                                                                                  \
    hipLaunchKernelGGL(tq_encode_gpu_kernel<DIM>,                                            \
                       dim3(unsigned((rows + kEncRows - 1) / kEncRows)), dim3(kWave), 0, st, x,  \
                       s, rows, rotation, mode, transpose ? 1 : 0, boundaries_inner, n_inner,    \
                       codes, sigma, dst_cap, dst_start);                                       \
    break;
  switch (dim) {
    TQKV_ENC(64) TQKV_ENC(128) TQKV_ENC(256) TQKV_ENC(512)
  }
#undef TQKV_ENC
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_tq_rotate_query(const float* rotation, const float* q, int32_t dim,
                                        float* rq, tqkv_stream stream) {
  if (!rotation || !q || !rq) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (dim <= 0) return fail(TQKV_EINVAL_SHAPE, "dim=%d", dim);
  hipLaunchKernelGGL(tq_rotate_query_kernel, dim3(1), dim3(kWave), 0,
                     reinterpret_cast<hipStream_t>(stream), rotation, q, dim, rq);
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_qjl_project_query(const float* qjl, int32_t m, int32_t dim,
                                          const float* q, float* pq, tqkv_stream stream) {
  if (!qjl || !q || !pq) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (m <= 0 || dim <= 0) return fail(TQKV_EINVAL_SHAPE, "m=%d dim=%d", m, dim);
  hipLaunchKernelGGL(tq_project_query_kernel, dim3(unsigned((m + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), qjl, m, dim, q, pq);
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_tq_scores_two_stage(const float* rq, const float* pq,
                                            const uint8_t* codes, const float* sigma,
                                            const float* centroids_f32, const uint32_t* signs,
                                            const float* rnorm, int32_t dim, int32_t m, int64_t n,
                                            float* scores, tqkv_stream stream) {
  if (n == 0) return ok();
  if (!rq || !pq || !codes || !sigma || !centroids_f32 || !signs || !rnorm || !scores)
    return fail(TQKV_EINVAL_ARG, "null pointer");
  if (dim <= 0 || m <= 0 || n < 0)
    return fail(TQKV_EINVAL_SHAPE, "dim=%d m=%d n=%lld", dim, m, (long long)n);
  hipLaunchKernelGGL(tq_scores_two_stage_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), rq, pq, codes, sigma, centroids_f32,
                     signs, rnorm, dim, m, n, scores);
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_qjl_encode_stage2(const uint16_t* k_rot, const uint16_t* k_dq,
                                          const float* qjl, int64_t rows, int32_t dim, int32_t m,
                                          uint32_t* signs, float* rnorm, tqkv_stream stream) {
  if (rows == 0) return ok();
  if (!k_rot || !k_dq || !qjl || !signs || !rnorm) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (rows < 0 || rows > 0x7fffffffLL || dim <= 0 || dim > 4096 || m <= 0)
    return fail(TQKV_EINVAL_SHAPE, "rows=%lld dim=%d m=%d", (long long)rows, dim, m);
  hipLaunchKernelGGL(qjl_encode_stage2_kernel, dim3(unsigned((rows + kQjlRows - 1) / kQjlRows)),
                     dim3(kWave), size_t(kQjlRows) * size_t(dim) * sizeof(float),
                     reinterpret_cast<hipStream_t>(stream), k_rot, k_dq, qjl, dim, m, rows, signs,
                     rnorm);
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_qjl_apply_correction(const uint16_t* k_dq, const uint32_t* signs,
                                             const float* rnorm, const float* qjl, int64_t rows,
                                             int32_t dim, int32_t m, uint16_t* k_eff,
                                             tqkv_stream stream) {
  if (rows == 0) return ok();
  if (!k_dq || !signs || !rnorm || !qjl || !k_eff) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (rows < 0 || dim <= 0 || m <= 0)
    return fail(TQKV_EINVAL_SHAPE, "rows=%lld dim=%d m=%d", (long long)rows, dim, m);
  const int64_t blocks = ((rows + kQjlRows - 1) / kQjlRows * dim + 255) / 256;
  if (blocks > 0x7fffffffLL) return fail(TQKV_EINVAL_SHAPE, "too many rows");
  hipLaunchKernelGGL(qjl_apply_correction_kernel, dim3(unsigned(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), k_dq, signs, rnorm, qjl, dim, m, rows,
                     k_eff);
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_tq_scores(const float* rq, const uint8_t* codes, const float* sigma,
                                  const float* centroids_f32, int32_t dim, int64_t n,
                                  float* scores, tqkv_stream stream) {
  if (n == 0) return ok();
  if (!rq || !codes || !sigma || !centroids_f32 || !scores) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (dim <= 0 || n < 0) return fail(TQKV_EINVAL_SHAPE, "dim=%d n=%lld", dim, (long long)n);
  if ((n + 255) / 256 > 0x7fffffffLL) return fail(TQKV_EINVAL_SHAPE, "n=%lld", (long long)n);
  hipLaunchKernelGGL(tq_scores_kernel<CodesU8>, dim3(unsigned((n + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), rq, CodesU8{codes, dim}, sigma,
                     centroids_f32, dim, n, scores);
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_tq_values(const float* rotation, const uint8_t* codes, const float* sigma,
                                  const float* centroids_f32, const float* weights, int32_t dim,
                                  int64_t n, float* out, tqkv_stream stream) {
  if (!rotation || !centroids_f32 || !out || (n > 0 && (!codes || !sigma || !weights)))
    return fail(TQKV_EINVAL_ARG, "null pointer");
  if (dim <= 0 || n < 0) return fail(TQKV_EINVAL_SHAPE, "dim=%d n=%lld", dim, (long long)n);
  hipLaunchKernelGGL(tq_values_kernel<CodesU8>, dim3(unsigned((dim + 63) / 64)), dim3(64), 0,
                     reinterpret_cast<hipStream_t>(stream), rotation, CodesU8{codes, dim}, sigma,
                     centroids_f32, weights, dim, n, out);
  TQKV_LAUNCHED();
  return ok();
}

namespace {

// The packed layout's shape for (dim, bits), or an error status.
int32_t packed_shape(int32_t dim, int32_t bits, int64_t n, CodesPacked* out) {
  if (bits < 1 || bits > 8) return fail(TQKV_EUNSUPPORTED, "bits=%d not in 1..8", bits);
  if (dim <= 0 || dim > 65536 || n < 0)
    return fail(TQKV_EINVAL_SHAPE, "dim=%d n=%lld", dim, (long long)n);
  const int per = 64 / bits;
  *out = CodesPacked{nullptr, (dim + per - 1) / per, bits, per};
  return ok();
}

}  // namespace

extern "C" int64_t tqkv_packed_words(int32_t dim, int32_t bits) {
  CodesPacked c{};
  if (bits < 1 || bits > 8 || dim <= 0) return -1;
  if (packed_shape(dim, bits, 0, &c)) return -1;
  return c.words;
}

extern "C" int32_t tqkv_pack_codes(const uint8_t* codes, int64_t n, int32_t dim, int32_t bits,
                                   uint64_t* words, tqkv_stream stream) {
  CodesPacked c{};
  if (int32_t rc = packed_shape(dim, bits, n, &c)) return rc;
  if (n == 0) return ok();
  if (!codes || !words) return fail(TQKV_EINVAL_ARG, "null pointer");
  const int64_t blocks = (n * c.words + 255) / 256;
  if (blocks > 0x7fffffffLL) return fail(TQKV_EINVAL_SHAPE, "n=%lld", (long long)n);
  hipLaunchKernelGGL(pack_codes_kernel, dim3(unsigned(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), codes, n, dim, bits, c.words, words);
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_unpack_codes(const uint64_t* words, int64_t n, int32_t dim, int32_t bits,
                                     uint8_t* codes, tqkv_stream stream) {
  CodesPacked c{};
  if (int32_t rc = packed_shape(dim, bits, n, &c)) return rc;
  if (n == 0) return ok();
  if (!codes || !words) return fail(TQKV_EINVAL_ARG, "null pointer");
  const int64_t blocks = (n * dim + 255) / 256;
  if (blocks > 0x7fffffffLL) return fail(TQKV_EINVAL_SHAPE, "n=%lld", (long long)n);
  hipLaunchKernelGGL(unpack_codes_kernel, dim3(unsigned(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), words, n, dim, bits, c.words, codes);
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_tq_scores_packed(const float* rq, const uint64_t* words,
                                         const float* sigma, const float* centroids_f32,
                                         int32_t bits, int32_t dim, int64_t n, float* scores,
                                         tqkv_stream stream) {
  CodesPacked c{};
  if (int32_t rc = packed_shape(dim, bits, n, &c)) return rc;
  if (n == 0) return ok();
  if (!rq || !words || !sigma || !centroids_f32 || !scores)
    return fail(TQKV_EINVAL_ARG, "null pointer");
  if ((n + 255) / 256 > 0x7fffffffLL) return fail(TQKV_EINVAL_SHAPE, "n=%lld", (long long)n);
  c.p = words;
  hipLaunchKernelGGL(tq_scores_kernel<CodesPacked>, dim3(unsigned((n + 255) / 256)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), rq, c, sigma, centroids_f32, dim, n,
                     scores);
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_tq_values_packed(const float* rotation, const uint64_t* words,
                                         const float* sigma, const float* centroids_f32,
                                         const float* weights, int32_t bits, int32_t dim,
                                         int64_t n, float* out, tqkv_stream stream) {
  CodesPacked c{};
  if (int32_t rc = packed_shape(dim, bits, n, &c)) return rc;
  if (!rotation || !centroids_f32 || !out || (n > 0 && (!words || !sigma || !weights)))
    return fail(TQKV_EINVAL_ARG, "null pointer");
  c.p = words;
  hipLaunchKernelGGL(tq_values_kernel<CodesPacked>, dim3(unsigned((dim + 63) / 64)), dim3(64), 0,
                     reinterpret_cast<hipStream_t>(stream), rotation, c, sigma, centroids_f32,
                     weights, dim, n, out);
  TQKV_LAUNCHED();
  return ok();
}

extern "C" int32_t tqkv_rotate_bf16(const uint16_t* x, int64_t rows, int32_t dim,
                                    const float* rotation, int32_t transpose, uint16_t* y,
                                    tqkv_stream stream) {
  if (rows == 0) return ok();
  if (!x || !rotation || !y) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (dim <= 0 || dim > 4096 || rows < 0 || rows > 0x7fffffffLL)
    return fail(TQKV_EINVAL_SHAPE, "rows=%lld dim=%d", (long long)rows, dim);
  // TQKV_TQ_ENCODE_LANE=0 also keeps the block-per-row rotation.
  const char* lane_env = getenv("TQKV_TQ_ENCODE_LANE");
  if ((dim == 64 || dim == 128) &&
      (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) % 16 == 0 &&
      !(lane_env && strcmp(lane_env, "0") == 0)) {
    const unsigned blocks = unsigned((rows + kLaneRows - 1) / kLaneRows);
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (dim == 64)
      hipLaunchKernelGGL(tq_rotate_lane_kernel<64>, dim3(blocks), dim3(kLaneBlock), 0, st, x, rows,
                         rotation, transpose, y);
    else
      hipLaunchKernelGGL(tq_rotate_lane_kernel<128>, dim3(blocks), dim3(kLaneBlock), 0, st, x,
                         rows, rotation, transpose, y);
    TQKV_LAUNCHED();
    return ok();
  }
  hipLaunchKernelGGL(tq_rotate_rows_kernel, dim3(unsigned(rows)), dim3(dim < 256 ? dim : 256),
                     size_t(dim) * sizeof(float), reinterpret_cast<hipStream_t>(stream), x, rows,
                     dim, rotation, transpose, y);
  TQKV_LAUNCHED();
  return ok();
}

// ---------------------------------------------------------------------------
// Decode attention over a codebook cache (the GPU TurboQuant caches'
// fused attention, turboquant.rs:763-923, for one query position): keys and
// values are stored rotated (y = R x) as codes + sigma, so the query is
// rotated the same way, attention runs in the rotated basis over
// centroid[c] * sigma, and the output goes back through R^T.
namespace tqkv {
namespace tq {
namespace {

constexpr int kCbTile = 64;  // tokens per step of a wavefront

// q_rot[b, h, :] = R q[b, h, :] in f32, and qs = q_rot * qscale (the
// scores' query). A workgroup takes kRotRows (batch row, head) rows and 64
// outputs (blockIdx.y); a wavefront takes four outputs at a time for all
// its rows: its lanes read rows i of R (coalesced) against the queries,
// then sum across the lanes. Each load of R serves kRotRows rows (a
// workgroup a row, reading all of R, made 128 MiB of L2 reads at config
// 2's shape). Every output's sum runs in the same order either way.
// blockDim: 256 (4 wavefronts x 4 outputs x 4 steps = 64 outputs).
constexpr int kRotRows = 4;
__global__ __launch_bounds__(256) void cb_rotate_q_kernel(const uint16_t* __restrict__ q,
                                                          const float* __restrict__ R, int D,
                                                          int64_t rows, float qscale,
                                                          float* __restrict__ qr,
                                                          float* __restrict__ qs) {
  const int64_t r0 = int64_t(blockIdx.x) * kRotRows;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const uint16_t* qrow[kRotRows];
#pragma unroll
  for (int k = 0; k < kRotRows; ++k)
    qrow[k] = q + (r0 + k < rows ? r0 + k : rows - 1) * D;  // rows past the end repeat one
  for (int i0 = int(blockIdx.y) * kWave + 4 * wave; i0 < (int(blockIdx.y) + 1) * kWave;
       i0 += 16) {
    float acc[kRotRows][4] = {};
    for (int j = lane; j < D; j += kWave) {
      float x[kRotRows];
#pragma unroll
      for (int k = 0; k < kRotRows; ++k) x[k] = bf16_to_f32(qrow[k][j]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float rv = R[int64_t(i0 + r) * D + j];
#pragma unroll
        for (int k = 0; k < kRotRows; ++k) acc[k][r] = fmaf(rv, x[k], acc[k][r]);
      }
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1)
#pragma unroll
      for (int k = 0; k < kRotRows; ++k)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[k][r] += __shfl_xor(acc[k][r], off, kWave);
#pragma unroll
    for (int k = 0; k < kRotRows; ++k) {
      if (lane < 4 && r0 + k < rows) {
        const float v =
            lane == 0 ? acc[k][0] : lane == 1 ? acc[k][1] : lane == 2 ? acc[k][2] : acc[k][3];
        qr[(r0 + k) * D + i0 + lane] = v;
        qs[(r0 + k) * D + i0 + lane] = v * qscale;
      }
    }
  }
}

// pq = Phi q for every (batch row, head): the query's QJL projection
// (QJLProjector::project_query, qjl.rs:76-84) for the score correction.
__global__ void cb_project_q_kernel(const uint16_t* __restrict__ q, const float* __restrict__ phi,
                                    int D, int m, float* __restrict__ pq) {
  const int64_t bh = blockIdx.x;
  for (int row = threadIdx.x; row < m; row += blockDim.x) {
    float acc = 0.0f;
    for (int j = 0; j < D; ++j) acc = fmaf(phi[int64_t(row) * D + j], bf16_to_f32(q[bh * D + j]), acc);
    pq[bh * m + row] = acc;
  }
}

// pq = Phi (R_eff q) from the rotated f32 query: the QJL projection of a
// cache whose signs are of the rotated-basis residual (the GPU-path encode).
__global__ void cb_project_qr_kernel(const float* __restrict__ qr, const float* __restrict__ phi,
                                     int D, int m, float* __restrict__ pq) {
  const int64_t bh = blockIdx.x;
  for (int row = threadIdx.x; row < m; row += blockDim.x) {
    float acc = 0.0f;
    for (int j = 0; j < D; ++j) acc = fmaf(phi[int64_t(row) * D + j], qr[bh * D + j], acc);
    pq[bh * m + row] = acc;
  }
}

// Most QJL rows the fused decode takes (m = 32 * qjl_words).
constexpr int kMaxQjl = 1024;

// One workgroup of one wavefront per (split, KV head, batch row): partial
// softmax state over its tokens for the G query heads. Scores: lane = token;
// values: lane = D / 64 consecutive channels. QJL: each key's score gains the
// QJL estimate of q . r from its residual signs (estimate_correction,
// qjl.rs:86-118; the two-stage scores of compressor.rs:122-159), with the
// query's projection in LDS.
template <int D, int G, bool QJL>
__global__ __launch_bounds__(kWave) void cb_decode_kernel(
    const float* __restrict__ qs, int H, const uint8_t* __restrict__ kc,
    const float* __restrict__ ks, const uint8_t* __restrict__ vc, const float* __restrict__ vs,
    int64_t cap, int64_t n, int H_kv, const float* __restrict__ cent_k,
    const float* __restrict__ cent_v, int n_k, int n_v, float qscale, int64_t split_len,
    int n_splits, float* __restrict__ part_o, float* __restrict__ part_m,
    float* __restrict__ part_l, const uint32_t* __restrict__ ksg, const float* __restrict__ krn,
    const float* __restrict__ pq, int qm, int hg) {
  constexpr int PER = D / kWave;
  __shared__ float s_ck[256], s_cv[256];
  __shared__ float s_p[G][kCbTile];
  __shared__ float s_pq[QJL ? G : 1][QJL ? kMaxQjl : 1];
  // blockIdx.y: KV head x head group (hg groups of G query heads each).
  const int split = blockIdx.x, b = blockIdx.z;
  const int kvh = int(blockIdx.y) / hg;
  const int h0 = kvh * G * hg + (int(blockIdx.y) % hg) * G;  // first query head
  const int lane = threadIdx.x;
  // The scaled query of the G heads: every lane reads the same values, so
  // the compiler loads them into scalar registers (s_load) as the scores
  // need them, where copies in LDS took a vector LDS read per four values
  // (measured at config 2's shape: 1.026 -> 0.960 ms a call).
  const float* qg = qs + (int64_t(b) * H + h0) * D;
  if constexpr (QJL) {
    for (int i = lane; i < G * qm; i += kWave) {
      const int h = i / qm, r = i % qm;
      s_pq[h][r] = pq[(int64_t(b) * H + h0 + h) * qm + r];
    }
  }
  for (int i = lane; i < 256; i += kWave) {
    s_ck[i] = i < n_k ? cent_k[i] : 0.0f;
    s_cv[i] = i < n_v ? cent_v[i] : 0.0f;
  }
  __syncthreads();
  const int64_t slab = (int64_t(b) * H_kv + kvh) * cap;
  const int64_t t0 = int64_t(split) * split_len;
  const int64_t t1 = t0 + split_len < n ? t0 + split_len : n;
  float m[G], l[G], acc[G][PER];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) acc[h][k] = 0.0f;
  }
  // D <= 256: the lane's key row of the next tile loads while this tile's
  // softmax and values run (16 B a load, D / 16 registers of 4 words).
  // D = 256 (kVRegs): once a tile's keys are scored, their 64 registers take
  // the tile's 64 value words (one 4-byte load a token, all issued at once,
  // landing under the softmax), and the next tile's key row loads a quarter
  // at a time as the value words are used up. A value loop that loaded
  // words as it went waited for memory every four tokens.
  constexpr bool kAhead = D <= 256;
  constexpr bool kVRegs = D == 256;
  constexpr int KW = kAhead ? D / 16 : 1;
  // The scores' loop over a key row: whole at D <= 256 (the row is in
  // registers); at D = 512, eight 16-byte loads in flight (unrolled by one,
  // each load had waited for the last).
  constexpr int KU = kAhead ? KW : 8;
  uint4 kn[KW];
  // Unconditional loads (a lane past the range re-reads the range's last
  // row, whose scores it masks): a lane that kept its old row instead would
  // hold both rows' registers live at once.
  auto load_keys_part = [&](int64_t at, int i0, int i1) {
    const uint8_t* row = kc + (slab + (at < t1 ? at : t1 - 1)) * D;
#pragma unroll
    for (int i = i0; i < i1; ++i) kn[i] = *reinterpret_cast<const uint4*>(row + 16 * i);
  };
  auto load_keys = [&](int64_t at) { load_keys_part(at, 0, KW); };
  if constexpr (kAhead) load_keys(t0 + lane);
  for (int64_t base = t0; base < t1; base += kCbTile) {
    const int64_t t = base + lane;
    const bool valid = t < t1;
    float sc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) sc[h] = 0.0f;
    if (valid) {
      const uint8_t* row = kc + (slab + t) * D;
#pragma unroll KU
      for (int d = 0; d < D; d += 16) {
        const uint4 w = kAhead ? kn[d / 16] : *reinterpret_cast<const uint4*>(row + d);
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const float c = s_ck[(ws[k / 4] >> (8 * (k % 4))) & 0xffu];
#pragma unroll
          for (int h = 0; h < G; ++h) sc[h] = fmaf(qg[h * D + d + k], c, sc[h]);
        }
      }
      const float sg = ks[slab + t];
#pragma unroll
      for (int h = 0; h < G; ++h) sc[h] *= sg;
      if constexpr (QJL) {
        const float rn = krn[slab + t];
        if (rn >= 1e-10f) {
          const int words = (qm + 31) / 32;
          const uint32_t* sw = ksg + (slab + t) * words;
          float corr[G];
#pragma unroll
          for (int h = 0; h < G; ++h) corr[h] = 0.0f;
          for (int w = 0; w < words; ++w) {
            const uint32_t bits = sw[w];
            const int nb = qm - 32 * w < 32 ? qm - 32 * w : 32;
            for (int j = 0; j < nb; ++j) {
              const bool pos = (bits >> j) & 1u;
#pragma unroll
              for (int h = 0; h < G; ++h) {
                const float p = s_pq[h][32 * w + j];
                corr[h] += pos ? p : -p;
              }
            }
          }
          const float cm = rn * (1.2533141373155001f / sqrtf(float(qm)));  // sqrt(pi/2) / sqrt(m)
#pragma unroll
          for (int h = 0; h < G; ++h) sc[h] = fmaf(corr[h] * cm, qscale, sc[h]);
        }
      }
    }
    const int cnt = int(t1 - base < kCbTile ? t1 - base : kCbTile);
    uint32_t vw[kVRegs ? kCbTile : 1];
    const uint8_t* vrow = vc + (slab + base) * D + PER * lane;
    if constexpr (kVRegs) {
      // Tokens past the range re-read the last row; their weights are 0.
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < kCbTile; ++j)
        vw[j] = *reinterpret_cast<const uint32_t*>(vrow + int64_t(j < cnt ? j : cnt - 1) * D);
    } else if constexpr (kAhead) {
      load_keys(t + kCbTile);  // this tile's keys are scored
    }
    // D < 256: the values' codes go through registers 16 tokens at a time,
    // two groups in flight (the first two load under the softmax), in
    // place of a loop that loaded each token's codes as it went.
    constexpr bool kVGroups = D < 256;
    constexpr int VWD = (PER + 3) / 4;  // words of a lane's codes a token
    constexpr int NGT = 16;             // tokens a group
    uint32_t va[kVGroups ? NGT : 1][VWD], vb[kVGroups ? NGT : 1][VWD];
    auto load_group = [&](uint32_t (&dst)[kVGroups ? NGT : 1][VWD], int g) {
#pragma unroll
      for (int u = 0; u < NGT; ++u) {
        const int j = g * NGT + u;
        const uint8_t* src = vrow + int64_t(j < cnt ? j : cnt - 1) * D;
        if constexpr (PER == 1) {
          dst[u][0] = *src;
        } else if constexpr (PER == 2) {
          dst[u][0] = *reinterpret_cast<const uint16_t*>(src);
        } else {
#pragma unroll
          for (int w = 0; w < VWD; ++w) dst[u][w] = *reinterpret_cast<const uint32_t*>(src + 4 * w);
        }
      }
    };
    auto use_group = [&](const uint32_t (&src)[kVGroups ? NGT : 1][VWD], int g) {
#pragma unroll
      for (int u = 0; u < NGT; ++u) {
        const int j = g * NGT + u;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
          const float c = s_cv[(src[u][k / 4] >> (8 * (k % 4))) & 0xffu];
#pragma unroll
          for (int h = 0; h < G; ++h) acc[h][k] = fmaf(s_p[h][j], c, acc[h][k]);
        }
      }
    };
    if constexpr (kVGroups) {
      load_group(va, 0);
      load_group(vb, 1);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float mx = valid ? sc[h] : -INFINITY;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
      const float mn = fmaxf(m[h], mx);
      const float f = m[h] == -INFINITY ? 0.0f : exp2f(m[h] - mn);
      l[h] *= f;
#pragma unroll
      for (int k = 0; k < PER; ++k) acc[h][k] *= f;
      m[h] = mn;
      const float p = valid ? exp2f(sc[h] - mn) : 0.0f;
      float ps = p;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) ps += __shfl_xor(ps, off, kWave);
      l[h] += ps;
      s_p[h][lane] = valid ? p * vs[slab + t] : 0.0f;
    }
    __syncthreads();
    // Values: lane takes channels PER * lane .. + PER - 1 (one PER-byte load
    // of each token's row; the wavefront reads the row whole).
    if constexpr (kVRegs) {
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
#pragma unroll
        for (int j = 16 * qq; j < 16 * qq + 16; ++j) {
#pragma unroll
          for (int k = 0; k < PER; ++k) {
            const float c = s_cv[(vw[j] >> (8 * k)) & 0xffu];
#pragma unroll
            for (int h = 0; h < G; ++h) acc[h][k] = fmaf(s_p[h][j], c, acc[h][k]);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        load_keys_part(t + kCbTile, qq * (KW / 4), (qq + 1) * (KW / 4));
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (kVGroups) {
      // Tokens past the range re-read the last row; their weights are 0.
      use_group(va, 0);
      load_group(va, 2);
      use_group(vb, 1);
      load_group(vb, 3);
      use_group(va, 2);
      use_group(vb, 3);
    }
    // D = 512: one token's codes at a time (two words a lane; staged
    // groups measured slower at Gemma 4's global shape).
    for (int j = 0; j < (D > 256 ? cnt : 0); ++j) {
      uint32_t cw[VWD];
#pragma unroll
      for (int w = 0; w < VWD; ++w)
        cw[w] = *reinterpret_cast<const uint32_t*>(vrow + int64_t(j) * D + 4 * w);
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const float c = s_cv[(cw[k / 4] >> (8 * (k % 4))) & 0xffu];
#pragma unroll
        for (int h = 0; h < G; ++h) acc[h][k] = fmaf(s_p[h][j], c, acc[h][k]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const int64_t row = (int64_t(b) * H + h0 + h) * n_splits + split;
#pragma unroll
    for (int k = 0; k < PER; ++k) part_o[row * D + PER * lane + k] = acc[h][k];
    if (lane == 0) {
      part_m[row] = m[h];
      part_l[row] = l[h];
    }
  }
}

// Merge the splits of one (batch row, head) in the rotated basis, then
// o = R^T o_rot, as bf16.
__global__ void cb_merge_kernel(const float* __restrict__ part_o, const float* __restrict__ part_m,
                                const float* __restrict__ part_l, int n_splits, int D,
                                const float* __restrict__ R, uint16_t* __restrict__ out) {
  extern __shared__ float s_o[];
  const int64_t bh = blockIdx.x;
  const float* pm = part_m + bh * n_splits;
  const float* pl = part_l + bh * n_splits;
  float mx = -INFINITY;
  for (int s = 0; s < n_splits; ++s) mx = fmaxf(mx, pm[s]);
  // Each split's weight once (the same exp2f of the same argument as a
  // per-element evaluation; empty splits are skipped by their max).
  float* s_w = s_o + D;
  for (int s = threadIdx.x; s < n_splits; s += blockDim.x)
    s_w[s] = pm[s] != -INFINITY ? exp2f(pm[s] - mx) : 0.0f;
  __syncthreads();
  // No branch per split (an empty split's weight is 0, and the decode
  // writes its partial as zeros), so the unrolled loads issue together: a
  // test per split had them wait one at a time.
  float ls = 0.0f;
  for (int s = 0; s < n_splits; ++s) ls += pl[s] * s_w[s];
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float os = 0.0f;
#pragma unroll 16
    for (int s = 0; s < n_splits; ++s) os += part_o[(bh * n_splits + s) * D + d] * s_w[s];
    s_o[d] = ls > 0.0f ? os / ls : 0.0f;
  }
  __syncthreads();
  // o = R^T o_rot: a thread's outputs (one, or two at D = 512) in one loop,
  // sixteen steps of loads of R in flight (the sums' order per output is
  // the sequence j = 0 .. D-1 either way).
  const int i0 = threadIdx.x, i1 = threadIdx.x + blockDim.x;
  const bool two = i1 < D;
  float a0 = 0.0f, a1 = 0.0f;
  if (two) {
#pragma unroll 16
    for (int j = 0; j < D; ++j) {
      const float o = s_o[j];
      a0 = fmaf(R[int64_t(j) * D + i0], o, a0);
      a1 = fmaf(R[int64_t(j) * D + i1], o, a1);
    }
  } else {
#pragma unroll 16
    for (int j = 0; j < D; ++j) a0 = fmaf(R[int64_t(j) * D + i0], s_o[j], a0);
  }
  if (i0 < D) out[bh * D + i0] = f32_to_bf16(a0);
  if (two) out[bh * D + i1] = f32_to_bf16(a1);
}

template <int D>
int32_t launch_cb(int G, dim3 grid, hipStream_t st, const float* qs, int H, const uint8_t* kc,
                  const float* ks, const uint8_t* vc, const float* vs, int64_t cap, int64_t n,
                  int H_kv, const float* ck, const float* cv, int nk, int nv, float qscale,
                  int64_t split_len, int n_splits, float* po, float* pm, float* pl,
                  const uint32_t* ksg, const float* krn, const float* pq, int m, int hg) {
#define TQKV_CB(GG)                                                                           \
  case GG:                                                                                   \
    if (ksg)                                                                                 \
      hipLaunchKernelGGL((cb_decode_kernel<D, GG, true>), grid, dim3(kWave), 0, st, qs, H, kc, \
                         ks, vc, vs, cap, n, H_kv, ck, cv, nk, nv, qscale, split_len, n_splits, \
                         po, pm, pl, ksg, krn, pq, m, hg);                                    \
    else                                                                                     \
      hipLaunchKernelGGL((cb_decode_kernel<D, GG, false>), grid, dim3(kWave), 0, st, qs, H, kc,\
                         ks, vc, vs, cap, n, H_kv, ck, cv, nk, nv, qscale, split_len, n_splits, \
                         po, pm, pl, ksg, krn, pq, m, hg);                                    \
    break;
  switch (G) {
    TQKV_CB(1) TQKV_CB(2) TQKV_CB(4) TQKV_CB(8) TQKV_CB(16)
    default: return fail(TQKV_EUNSUPPORTED, "codebook decode with %d query heads a wavefront", G);
  }
#undef TQKV_CB
  TQKV_LAUNCHED();
  return TQKV_OK;
}

}  // namespace
}  // namespace tq
}  // namespace tqkv

namespace tqkv {
namespace tq {
namespace {
// lloyd_max_dequantize_scaled (turboquant.rs:428-439): bf16(centroid[c] *
// sigma) for rows [0, rows) of each slab of codes [slabs, cap, D] and sigma
// [slabs, cap], into out [slabs, rows, D]. A thread writes 8 values (one
// 16-byte store) from 8 codes (one 8-byte load); the centroids sit in LDS.
__global__ __launch_bounds__(256) void cb_dequant_kernel(const uint8_t* __restrict__ codes,
                                                         const float* __restrict__ sigma,
                                                         const float* __restrict__ cent,
                                                         int n_cent, int64_t rows, int64_t cap,
                                                         int D, int64_t slabs,
                                                         uint16_t* __restrict__ out) {
  __shared__ float s_c[256];
  for (int i = threadIdx.x; i < 256; i += blockDim.x) s_c[i] = i < n_cent ? cent[i] : 0.0f;
  __syncthreads();
  const int per_row = D / 8;
  const int64_t total = slabs * rows * per_row;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t j = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; j < total; j += stride) {
    const int64_t r = j / per_row, slab = r / rows, t = r % rows;
    const int e0 = int(j % per_row) * 8;
    const int64_t src = slab * cap + t;
    const uint2 c8 = *reinterpret_cast<const uint2*>(codes + src * D + e0);
    const float sg = sigma[src];
    uint32_t w[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t word = k < 2 ? c8.x : c8.y;
      const int sh = 16 * (k % 2);
      const uint32_t lo = f32_to_bf16(s_c[(word >> sh) & 0xffu] * sg);
      const uint32_t hi = f32_to_bf16(s_c[(word >> (sh + 8)) & 0xffu] * sg);
      w[k] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(out + (slab * rows + t) * D + e0) = uint4{w[0], w[1], w[2], w[3]};
  }
}
}  // namespace
}  // namespace tq

// Codes rows [0, rows) of each slab of a [slabs, cap, D] codebook slot,
// dequantized to bf16 into out [slabs, rows, D].
int32_t codebook_dequantize_slabs(const uint8_t* codes, const float* sigma, const float* cent,
                                  int bits, int64_t slabs, int64_t cap, int64_t rows, int D,
                                  uint16_t* out, hipStream_t st) {
  if (rows == 0 || slabs == 0) return TQKV_OK;
  if (!codes || !sigma || !cent || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (bits < 1 || bits > 8 || D <= 0 || D % 8 != 0 || slabs < 0 || rows < 0 || rows > cap)
    return fail(TQKV_EINVAL_SHAPE, "bits=%d D=%d slabs=%lld rows=%lld cap=%lld", bits, D,
                (long long)slabs, (long long)rows, (long long)cap);
  if ((reinterpret_cast<uintptr_t>(codes) | reinterpret_cast<uintptr_t>(out)) % 16 != 0)
    return fail(TQKV_EINVAL_ARG, "codes and output must be 16-byte aligned");
  int64_t blocks = (slabs * rows * (D / 8) + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(tq::cb_dequant_kernel, dim3(unsigned(blocks)), dim3(256), 0, st, codes,
                     sigma, cent, 1 << bits, rows, cap, D, slabs, out);
  TQKV_LAUNCHED();
  return TQKV_OK;
}
}  // namespace tqkv

extern "C" int32_t tqkv_codebook_dequantize(const uint8_t* codes, const float* sigma,
                                            const float* centroids, int32_t bits, int64_t rows,
                                            int32_t dim, uint16_t* out, tqkv_stream stream) {
  if (rows < 0) return fail(TQKV_EINVAL_SHAPE, "rows=%lld", (long long)rows);
  if (int32_t rc = tqkv::codebook_dequantize_slabs(codes, sigma, centroids, bits, 1, rows, rows,
                                                   dim, out, reinterpret_cast<hipStream_t>(stream)))
    return rc;
  return ok();
}

extern "C" size_t tqkv_decode_codebook_workspace_size(int32_t B, int32_t H, int32_t D,
                                                       int64_t total_tokens) {
  if (B <= 0 || H <= 0 || D <= 0 || total_tokens <= 0) return 0;
  // The most splits decode_codebook plans for any context up to total_tokens.
  const int64_t splits = (total_tokens + 255) / 256 < 64 ? (total_tokens + 255) / 256 : 64;
  return size_t(B) * H *
         (2 * size_t(D) + size_t(tq::kMaxQjl) + size_t(splits) * (size_t(D) + 2)) * sizeof(float);
}

namespace {
int32_t decode_codebook(const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t D,
                        float scale, const float* rotation, const float* centroids_k,
                        int32_t bits_k, const float* centroids_v, int32_t bits_v,
                        const uint8_t* k_codes, const float* k_sigma, const uint32_t* k_signs,
                        const float* k_rnorm, const float* qjl, int32_t qjl_m,
                        const uint8_t* v_codes, const float* v_sigma, int64_t cap, int64_t n,
                        uint16_t* out, void* workspace, size_t workspace_bytes,
                        tqkv_stream stream, bool qjl_rotated = false) {
  if (!q || !rotation || !centroids_k || !centroids_v || !k_codes || !k_sigma || !v_codes ||
      !v_sigma || !out)
    return fail(TQKV_EINVAL_ARG, "null pointer");
  if (qjl_m != 0 && (!k_signs || !k_rnorm || !qjl || qjl_m < 0 || qjl_m > tq::kMaxQjl))
    return fail(TQKV_EINVAL_ARG, "qjl_m=%d needs signs, residual norms and the QJL matrix "
                "(m <= %d)", qjl_m, tq::kMaxQjl);
  if (B <= 0 || H <= 0 || H_kv <= 0 || H % H_kv != 0 || n <= 0 || n > cap)
    return fail(TQKV_EINVAL_SHAPE, "B=%d H=%d H_kv=%d n=%lld cap=%lld", B, H, H_kv, (long long)n,
                (long long)cap);
  if (bits_k < 1 || bits_k > 8 || bits_v < 1 || bits_v > 8)
    return fail(TQKV_EUNSUPPORTED, "bits %d/%d", bits_k, bits_v);
  // A lane loads D / 64 value codes at once (up to 4-byte words); key rows
  // are read 16 bytes a load (rows of D >= 64 bytes keep that alignment).
  const int v_align = D >= 256 ? 4 : D >= 128 ? 2 : 1;
  if (reinterpret_cast<uintptr_t>(v_codes) % v_align != 0)
    return fail(TQKV_EINVAL_ARG, "v_codes must be %d-byte aligned", v_align);
  if (reinterpret_cast<uintptr_t>(k_codes) % 16 != 0)
    return fail(TQKV_EINVAL_ARG, "k_codes must be 16-byte aligned");
  const int G = H / H_kv;
  if (G > 16 || (G & (G - 1)) != 0)
    return fail(TQKV_EUNSUPPORTED, "codebook decode with %d query heads per KV head (1, 2, 4, "
                "8 or 16)", G);
  // A wavefront takes Gw = G / hg of a KV head's query heads, Gw x D <= 1024
  // (each head group re-reads the keys and values, mostly from L2): at D =
  // 512 with 16 heads a KV head (Gemma 4's global layers) one wavefront of
  // all 16 heads held 251 registers and the few (batch row, KV head) units
  // left most SIMDs idle.
  int hg = 1;
  while (G / hg > 1 && (G / hg) * D > 1024) hg *= 2;
  const int Gw = G / hg;
  // Splits: with 128 or more (batch row, KV head, head group) units the grid
  // fills the chip with splits of 1024 tokens (at most 32), which pay the
  // first key load and the merge half as often (config 2's shape: 1.061
  // against 1.094 ms); fewer units take enough splits for ~4,096
  // wavefronts, never under 256 tokens a split, at most 64 (the workspace
  // size assumes no more).
  const int64_t units = int64_t(B) * H_kv * hg;
  int64_t n_splits64;
  if (units >= 128) {
    n_splits64 = (n + 1023) / 1024 < 32 ? (n + 1023) / 1024 : 32;
  } else {
    n_splits64 = (4096 + units - 1) / units;
    if (n_splits64 > (n + 255) / 256) n_splits64 = (n + 255) / 256;
    if (n_splits64 > 64) n_splits64 = 64;
  }
  const int n_splits = int(n_splits64);
  const int64_t split_len = (n + n_splits - 1) / n_splits;
  const size_t need = tqkv_decode_codebook_workspace_size(B, H, D, n);
  void* ws = workspace;
  if (!ws) {
    if (int32_t rc = scratch_for_current_device(need, &ws)) return rc;
  } else if (workspace_bytes < need) {
    return fail(TQKV_EINVAL_ARG, "workspace of %zu bytes, need %zu", workspace_bytes, need);
  }
  float* qr = static_cast<float*>(ws);
  float* qsc = qr + size_t(B) * H * D;
  float* pq = qsc + size_t(B) * H * D;
  float* po = pq + size_t(B) * H * tq::kMaxQjl;
  float* pm = po + size_t(B) * H * n_splits * D;
  float* pl = pm + size_t(B) * H * n_splits;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const float qscale = scale * 1.4426950408889634f;
  const int64_t qrows = int64_t(B) * H;
  hipLaunchKernelGGL(tq::cb_rotate_q_kernel,
                     dim3(unsigned((qrows + tq::kRotRows - 1) / tq::kRotRows), unsigned(D / 64)),
                     dim3(256), 0, st, q, rotation, D, qrows, qscale, qr, qsc);
  TQKV_LAUNCHED();
  if (qjl_m > 0) {
    if (qjl_rotated)
      hipLaunchKernelGGL(tq::cb_project_qr_kernel, dim3(unsigned(B * H)), dim3(256), 0, st, qr,
                         qjl, D, qjl_m, pq);
    else
      hipLaunchKernelGGL(tq::cb_project_q_kernel, dim3(unsigned(B * H)), dim3(256), 0, st, q,
                         qjl, D, qjl_m, pq);
    TQKV_LAUNCHED();
  }
  const uint32_t* sg = qjl_m > 0 ? k_signs : nullptr;
  const dim3 grid{unsigned(n_splits), unsigned(H_kv * hg), unsigned(B)};
  int32_t rc = TQKV_OK;
  switch (D) {
    case 64: rc = tq::launch_cb<64>(Gw, grid, st, qsc, H, k_codes, k_sigma, v_codes, v_sigma, cap, n, H_kv, centroids_k, centroids_v, 1 << bits_k, 1 << bits_v, qscale, split_len, n_splits, po, pm, pl, sg, k_rnorm, pq, qjl_m, hg); break;
    case 128: rc = tq::launch_cb<128>(Gw, grid, st, qsc, H, k_codes, k_sigma, v_codes, v_sigma, cap, n, H_kv, centroids_k, centroids_v, 1 << bits_k, 1 << bits_v, qscale, split_len, n_splits, po, pm, pl, sg, k_rnorm, pq, qjl_m, hg); break;
    case 256: rc = tq::launch_cb<256>(Gw, grid, st, qsc, H, k_codes, k_sigma, v_codes, v_sigma, cap, n, H_kv, centroids_k, centroids_v, 1 << bits_k, 1 << bits_v, qscale, split_len, n_splits, po, pm, pl, sg, k_rnorm, pq, qjl_m, hg); break;
    case 512: rc = tq::launch_cb<512>(Gw, grid, st, qsc, H, k_codes, k_sigma, v_codes, v_sigma, cap, n, H_kv, centroids_k, centroids_v, 1 << bits_k, 1 << bits_v, qscale, split_len, n_splits, po, pm, pl, sg, k_rnorm, pq, qjl_m, hg); break;
    default: return fail(TQKV_EUNSUPPORTED, "codebook decode D=%d not in {64,128,256,512}", D);
  }
  if (rc) return rc;
  hipLaunchKernelGGL(tq::cb_merge_kernel, dim3(unsigned(B * H)), dim3(D < 256 ? D : 256),
                     size_t(D + n_splits) * sizeof(float), st, po, pm, pl, n_splits, D, rotation,
                     out);
  TQKV_LAUNCHED();
  return ok();
}
}  // namespace

extern "C" int32_t tqkv_decode_attend_codebook(
    const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t D, float scale,
    const float* rotation, const float* centroids_k, int32_t bits_k, const float* centroids_v,
    int32_t bits_v, const uint8_t* k_codes, const float* k_sigma, const uint8_t* v_codes,
    const float* v_sigma, int64_t cap, int64_t n, uint16_t* out, void* workspace,
    size_t workspace_bytes, tqkv_stream stream) {
  return decode_codebook(q, B, H, H_kv, D, scale, rotation, centroids_k, bits_k, centroids_v,
                         bits_v, k_codes, k_sigma, nullptr, nullptr, nullptr, 0, v_codes, v_sigma,
                         cap, n, out, workspace, workspace_bytes, stream);
}

namespace tqkv {
// Codebook decode with QJL signs of the rotated-basis residual (a GPU-path
// cache): the score correction projects the rotated query.
int32_t decode_codebook_qjl_rotated(
    const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t D, float scale,
    const float* rotation, const float* centroids_k, int32_t bits_k, const float* centroids_v,
    int32_t bits_v, const uint8_t* k_codes, const float* k_sigma, const uint32_t* k_signs,
    const float* k_rnorm, const float* qjl, int32_t qjl_m, const uint8_t* v_codes,
    const float* v_sigma, int64_t cap, int64_t n, uint16_t* out, void* workspace,
    size_t workspace_bytes, tqkv_stream stream) {
  if (qjl_m <= 0) return fail(TQKV_EINVAL_ARG, "qjl_m=%d", qjl_m);
  return decode_codebook(q, B, H, H_kv, D, scale, rotation, centroids_k, bits_k, centroids_v,
                         bits_v, k_codes, k_sigma, k_signs, k_rnorm, qjl, qjl_m, v_codes, v_sigma,
                         cap, n, out, workspace, workspace_bytes, stream, true);
}
}  // namespace tqkv

extern "C" int32_t tqkv_decode_attend_codebook_qjl(
    const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t D, float scale,
    const float* rotation, const float* centroids_k, int32_t bits_k, const float* centroids_v,
    int32_t bits_v, const uint8_t* k_codes, const float* k_sigma, const uint32_t* k_signs,
    const float* k_rnorm, const float* qjl, int32_t qjl_m, const uint8_t* v_codes,
    const float* v_sigma, int64_t cap, int64_t n, uint16_t* out, void* workspace,
    size_t workspace_bytes, tqkv_stream stream) {
  if (qjl_m <= 0) return fail(TQKV_EINVAL_ARG, "qjl_m=%d", qjl_m);
  return decode_codebook(q, B, H, H_kv, D, scale, rotation, centroids_k, bits_k, centroids_v,
                         bits_v, k_codes, k_sigma, k_signs, k_rnorm, qjl, qjl_m, v_codes, v_sigma,
                         cap, n, out, workspace, workspace_bytes, stream);
}
