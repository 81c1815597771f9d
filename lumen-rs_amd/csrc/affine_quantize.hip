// Quantize-on-append in MLX's affine format, bit-exact with its Metal kernel,
// and the matching dequantize.
//
// Layout of the work: each lane owns 16 consecutive elements of a row, read
// as two 16-byte loads, so a row takes dim / 16 lanes and a wavefront holds
// several rows (8 at dim 128); a 256-thread workgroup takes a block of rows
// of one tensor, and the grid covers K and V in one launch. A group's lanes
// are adjacent, so its min and max are a butterfly over gs / 16 lanes. Each
// lane packs every 8 codes into a 64-bit chunk (8 x bits bits), the chunks go
// through LDS, and each output word is cut from the one or two chunks it
// overlaps: LSB-first u32 words for every width, including those whose codes
// straddle words (3, 5, 6 bits). The per-lane arithmetic (affine_quantize.hpp)
// is MLX's exactly.
#include "affine_quantize.hpp"

namespace tqkv {
namespace {

constexpr int kWave = 64;
constexpr int kQThreads = 256;
constexpr int kQWaves = kQThreads / kWave;

// One tensor of a quantize launch: rows [n_slabs * s] of bf16 x into a
// cache buffer at rows slab * dst_cap + dst_start + j.
struct QTensor {
  const uint16_t* x;
  uint32_t* packed;
  uint16_t* scales;
  uint16_t* biases;
  int bits;
};

struct QArgs {
  QTensor t[2];
  int64_t s, rows, dst_cap, dst_start;
  int gs;
  int blocks_per_tensor;  // row blocks of one tensor
  int n_blocks;           // over all tensors
};

template <int D, int WAVES = kQWaves>
struct QShape {
  static constexpr int kEpl = 16;                 // elements a lane
  static constexpr int kLpr = D / kEpl;           // lanes a row
  static constexpr int kRpw = kWave / kLpr;       // rows a wavefront
  static constexpr int kRows = WAVES * kRpw;      // rows a block
  static constexpr int kUnits = kEpl / 8;         // 8-code chunks a lane
};

// Destination row of input row r (rows of n_slabs slabs of s rows, written
// at slab * dst_cap + dst_start + j). 32-bit division: the host keeps rows
// (and so s) below 2^31.
__device__ __forceinline__ int64_t dst_row(int64_t r, int64_t s, int64_t dst_cap,
                                           int64_t dst_start) {
  const uint32_t slab = uint32_t(r) / uint32_t(s), j = uint32_t(r) - slab * uint32_t(s);
  return int64_t(slab) * dst_cap + dst_start + j;
}

// One block of rows (row block `blk` of the tensor, WAVES wavefronts) of the
// plain quantize. chunks: WAVES x (kWave * kUnits) u64 of LDS. Every thread
// of the workgroup calls it (it synchronizes the workgroup).
template <int D, int WAVES>
__device__ __forceinline__ void quantize_rows_block(const QTensor& t, int64_t blk, int64_t rows,
                                                    int64_t s, int64_t dst_cap, int64_t dst_start,
                                                    int gs, uint64_t* chunks) {
  using S = QShape<D, WAVES>;
  constexpr int EPL = S::kEpl, LPR = S::kLpr;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int lir = lane % LPR;                // lane in its row
  const int rw = lane / LPR;                 // row in the wavefront
  uint64_t* ch = chunks + wave * (kWave * S::kUnits) + rw * (D / 8);

  const int64_t r = blk * S::kRows + wave * S::kRpw + rw;
  const bool live = r < rows;
  const int64_t rr = live ? r : rows - 1;  // dead rows recompute the last one
  const int64_t dst = dst_row(rr, s, dst_cap, dst_start);

  float v[EPL];
  aq::load_lane(t.x + rr * D + lir * EPL, v);
  const int bits = t.bits;
  const aq::LaneCodes qc = aq::quantize_lane(v, gs, bits);
  const int lpg = gs / EPL;  // lanes a group: a power of two, <= LPR
  const int groups = D / gs;
  if (live && lir % lpg == 0) {
    const int g = lir / lpg;
    t.scales[dst * groups + g] = f32_to_bf16(qc.scale);
    t.biases[dst * groups + g] = f32_to_bf16(qc.bias);
  }
#pragma unroll
  for (int h = 0; h < S::kUnits; ++h) ch[lir * S::kUnits + h] = qc.chunk[h];
  __syncthreads();

  const int words = D * bits / 32;
  if (live) {
    uint32_t* out = t.packed + dst * words;
    for (int w = lir; w < words; w += LPR) out[w] = aq::packed_word(ch, w, bits);
  }
  __syncthreads();  // the chunks are reused by the next block
}

template <int D>
__global__ __launch_bounds__(kQThreads) void affine_quantize_kernel(const QArgs a) {
  using S = QShape<D>;
  __shared__ uint64_t chunks[kQWaves * kWave * S::kUnits];
  for (int blk = blockIdx.x; blk < a.n_blocks; blk += gridDim.x) {
    const int ti = blk / a.blocks_per_tensor;  // uniform: K then V
    quantize_rows_block<D, kQWaves>(a.t[ti], blk % a.blocks_per_tensor, a.rows, a.s, a.dst_cap,
                                    a.dst_start, a.gs, chunks);
  }
}

// ---------------------------------------------------------------------------
// Rotate, then quantize, in one pass (the affine + rotation cache mode,
// gemma4_moe.rs:4154-4173: k_to_cache = rotate_last_axis(k, R), then the
// cache's mlx::quantize). rotate_last_axis (turboquant.rs:258-267) is an
// f32 x f32 matmul rounded to bf16; here the product runs on the matrix
// cores with f32 accumulation (MLX's summation order is its own), is rounded
// to bf16 in registers, and the quantize reads it from there: no rotated
// copy goes through HBM.
//
// A wavefront takes 16 rows. In either product the output tile n (0..7) of
// lane l = 16 q + c holds column c0 + 8 c + n, so after the k-steps lane l
// holds rows 4 q + i (i < 4), columns c0 + 8 c .. + 7 of the product: eight
// consecutive elements of four rows, which is what the quantizer takes (a
// 64-element group is 8 adjacent lanes).
//  - D = 128 (three bf16 products, RShape::kSplit): k-step ks covers k in
//    [32 ks, 32 ks + 32); lane l supplies x[row c][32 ks + 8 q .. + 7] and
//    the R part's column 8 c + n at those k, from LDS.
//  - D = 256 (v_mfma_f32_16x16x4_f32): k-step kk supplies
//    A[c][q] = x[row c][q * D/4 + kk], so a lane reads one contiguous quarter
//    of its row, and B[q][c] = R[q * D/4 + kk][c0 + 8 c + n]; two workgroups
//    split a row's columns, each holding its 128 columns of R in LDS.
// ---------------------------------------------------------------------------
constexpr int kRW = 8;                 // wavefronts a rotate workgroup
constexpr int kRT = kRW * kWave;
constexpr int kTileRows = 16;

typedef float floatx4 __attribute__((ext_vector_type(4)));

typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
typedef float f2_t __attribute__((ext_vector_type(2)));

template <int D>
struct RShape {
  static constexpr int kNC = 128;                 // output columns a workgroup takes
  static constexpr int kHalves = D / kNC;         // column blocks of a row
  static constexpr int kKq = D / 4;               // k values a lane supplies (f32 path)
  static constexpr int kQS = kKq * kNC + 16;      // floats between k-quarters in LDS
  // D = 128: the product as three bf16 matrix-core products, R = R_hi +
  // R_lo + R_lo2 split exactly into bf16 parts (x is bf16, so every product
  // is exact in f32 and only the f32 accumulation rounds): 96 products of
  // 16x16x32 a tile instead of 256 of 16x16x4 f32, at 16x the rate. R's
  // parts stay in LDS as rows of k: row n * 16 + c holds output column
  // 8 c + n, kCS bf16 apart (32 bytes of padding: rows 8 dwords apart in
  // the banks; 16 bytes of padding measured 4% slower, 48 and 80 no faster).
  static constexpr bool kSplit = D == 128;
  static constexpr int kCS = D + 16;
  static constexpr int kPart = kNC * kCS;         // bf16 a part
  static constexpr int kLdsBytes = kSplit ? 3 * kPart * 2 : 4 * kQS * 4;
  // LDS chunk area: the plain path's kWave x 2 a wavefront (the rotate
  // path's 4 rows x 16 chunks a wavefront fit in it).
  static constexpr int kChunks = kRW * kWave * 2;
};

struct RArgs {
  QTensor rot;             // rotated, then quantized
  QTensor plain;           // quantized as it is (x null: none)
  const float* R;          // [D, D] f32, row-major: y = x R
  uint16_t* rotated;       // optional: the rotated bf16 rows, input order
  int64_t s, rows, dst_cap, dst_start;
  int gs;
  int tiles;               // 16-row tiles of the rotated tensor
  int groups;              // workgroups a column block
  int rot_blocks;          // groups x column blocks
  int plain_blocks;        // row blocks of the plain tensor
};

// The rotate phase of a workgroup: its R columns into LDS, then its tiles.
template <int D>
__device__ __forceinline__ void rotate_quantize_tiles(const RArgs& a, unsigned char* lds_r,
                                                      uint64_t* chunks) {
  using S = RShape<D>;
  constexpr int NC = S::kNC, KQ = S::kKq, QS = S::kQS, CS = S::kCS, PART = S::kPart;
  float* Rl = reinterpret_cast<float*>(lds_r);
  uint16_t* Rb = reinterpret_cast<uint16_t*>(lds_r);

  const int half = int(blockIdx.x) % S::kHalves, g = int(blockIdx.x) / S::kHalves;
  const int c0 = half * NC;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int q = lane / 16, c = lane % 16;
  const int stride = a.groups * kRW;

  // A wavefront's tile t: lane l reads 8 elements of row 16 t + c for each
  // k-step (split path: x[32 ks + 8 q .. + 7]; f32 path: the contiguous
  // quarter q). Dead rows read the last row.
  uint4 xa[KQ / 8];
  auto load_x = [&](int t) {
    const int64_t ra = int64_t(t) * kTileRows + c;
    const int64_t rr = ra < a.rows ? ra : a.rows - 1;
#pragma unroll
    for (int i = 0; i < KQ / 8; ++i) {
      const int k0 = S::kSplit ? 32 * i + 8 * q : q * KQ + 8 * i;
      xa[i] = *reinterpret_cast<const uint4*>(a.rot.x + rr * D + k0);
    }
  };
  int t = g * kRW + wave;
  if (t < a.tiles) load_x(t);  // in flight with R's loads

  if constexpr (S::kSplit) {
    // Thread -> a block of 8 k x 4 columns of R (float4 loads of 8 rows;
    // 32 threads read a whole row); each element splits exactly into three
    // bf16 parts by truncation (hi = the top 16 bits, lo = those of the
    // remainder, lo2 = what is left, at most 8 significant bits), and each
    // column's 8 k of a part go to LDS as one 16-byte row piece.
    static_assert(D * NC / 32 == kRT, "one 8 x 4 block a thread");
    const int cq = threadIdx.x % (NC / 4), kb = threadIdx.x / (NC / 4);
    float4 rv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      rv[e] = *reinterpret_cast<const float4*>(a.R + size_t(8 * kb + e) * D + 4 * cq);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t w[3][4];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float r = j == 0 ? rv[e].x : j == 1 ? rv[e].y : j == 2 ? rv[e].z : rv[e].w;
        const uint32_t hi = __float_as_uint(r) & 0xffff0000u;
        const float rem = r - __uint_as_float(hi);  // exact
        const uint32_t lo = __float_as_uint(rem) & 0xffff0000u;
        const uint32_t lo2 = __float_as_uint(rem - __uint_as_float(lo));  // exact, low half zero
        const uint32_t pv[3] = {hi >> 16, lo >> 16, lo2 >> 16};
#pragma unroll
        for (int p = 0; p < 3; ++p) {
          if (e % 2 == 0) w[p][e / 2] = pv[p];
          else w[p][e / 2] |= pv[p] << 16;
        }
      }
      const int col = 4 * cq + j, rho = (col % 8) * 16 + col / 8;
#pragma unroll
      for (int p = 0; p < 3; ++p)
        *reinterpret_cast<uint4*>(&Rb[p * PART + rho * CS + 8 * kb]) =
            uint4{w[p][0], w[p][1], w[p][2], w[p][3]};
    }
  } else {
    // R[:, c0 : c0 + NC] into LDS, k-quarter q from q * QS (row k = q KQ +
    // kk at q * QS + kk * NC); every load of a thread is issued before its
    // stores.
    constexpr int kRIters = D * NC / 4 / kRT;
    static_assert(kRIters * kRT * 4 == D * NC, "R tiles the workgroup");
    float4 rv[kRIters];
#pragma unroll
    for (int j = 0; j < kRIters; ++j) {
      const int i = threadIdx.x + j * kRT, k = i / (NC / 4), col4 = i % (NC / 4);
      rv[j] = *reinterpret_cast<const float4*>(a.R + size_t(k) * D + c0 + 4 * col4);
    }
#pragma unroll
    for (int j = 0; j < kRIters; ++j) {
      const int i = threadIdx.x + j * kRT, k = i / (NC / 4), col4 = i % (NC / 4);
      *reinterpret_cast<float4*>(&Rl[(k / KQ) * QS + (k % KQ) * NC + 4 * col4]) = rv[j];
    }
  }
  __syncthreads();

  const int bits = a.rot.bits;
  const int lpg = a.gs / 8;                  // lanes a group
  const int groups_row = D / a.gs;
  const int words_row = D * bits / 32, words_half = NC * bits / 32;
  // 4 and 8 bits: a lane's 8 codes are whole words of the row (word c, or
  // words 2c and 2c + 1); other widths cut words from the lanes' chunks.
  const bool whole = bits == 4 || bits == 8;
  uint64_t* ch = chunks + wave * (4 * (NC / 8));
  const float* rb = Rl + q * QS + 8 * c;  // f32 path

  for (; t < a.tiles; t += stride) {
    const int64_t row0 = int64_t(t) * kTileRows;
    uint4 cur[KQ / 8];
#pragma unroll
    for (int i = 0; i < KQ / 8; ++i) cur[i] = xa[i];
    if (t + stride < a.tiles) load_x(t + stride);  // the next tile's rows, during this one

    floatx4 acc[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) acc[n] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (S::kSplit) {
#pragma unroll
      for (int ks = 0; ks < D / 32; ++ks) {
        const bf8_t av = __builtin_bit_cast(bf8_t, cur[ks]);
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          const uint16_t* bp = Rb + (n * 16 + c) * CS + 32 * ks + 8 * q;
#pragma unroll
          for (int p = 0; p < 3; ++p) {
            const bf8_t bv = __builtin_bit_cast(bf8_t, *reinterpret_cast<const uint4*>(bp + p * PART));
            acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv, acc[n], 0, 0, 0);
          }
        }
      }
    } else
#pragma unroll
    for (int kk = 0; kk < KQ; ++kk) {
      const uint4 w4 = cur[kk / 8];
      const uint32_t w = (kk % 8) / 2 == 0 ? w4.x : (kk % 8) / 2 == 1 ? w4.y
                       : (kk % 8) / 2 == 2 ? w4.z : w4.w;
      const float av = __uint_as_float((kk & 1) ? (w & 0xffff0000u) : (w << 16));
      const float4 b0 = *reinterpret_cast<const float4*>(rb + kk * NC);
      const float4 b1 = *reinterpret_cast<const float4*>(rb + kk * NC + 4);
      acc[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b0.x, acc[0], 0, 0, 0);
      acc[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b0.y, acc[1], 0, 0, 0);
      acc[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b0.z, acc[2], 0, 0, 0);
      acc[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b0.w, acc[3], 0, 0, 0);
      acc[4] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b1.x, acc[4], 0, 0, 0);
      acc[5] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b1.y, acc[5], 0, 0, 0);
      acc[6] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b1.z, acc[6], 0, 0, 0);
      acc[7] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b1.w, acc[7], 0, 0, 0);
    }

    // Rows 4 q + i, columns c0 + 8 c .. + 7, rounded to bf16 as
    // rotate_last_axis's cast does; the quantizer works on those values.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v[8];
      uint32_t pk[4];
#pragma unroll
      for (int n = 0; n < 8; n += 2) {
        // v_cvt_pk_bf16_f32: round to nearest even (finite products).
        const f2_t f = {acc[n][i], acc[n + 1][i]};
        pk[n / 2] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf2_t));
        v[n] = __uint_as_float(pk[n / 2] << 16);
        v[n + 1] = __uint_as_float(pk[n / 2] & 0xffff0000u);
      }
      const int64_t row = row0 + 4 * q + i;
      const bool live = row < a.rows;
      const int64_t dst = dst_row(live ? row : a.rows - 1, a.s, a.dst_cap, a.dst_start);
      if (a.rotated && live)
        *reinterpret_cast<uint4*>(a.rotated + row * D + c0 + 8 * c) =
            uint4{pk[0], pk[1], pk[2], pk[3]};
      float sc, bi;
      uint64_t chk[1];
      aq::quantize_elems<8, true>(v, lpg, bits, sc, bi, chk);
      if (live && c % lpg == 0) {
        const int gi = (c0 + 8 * c) / a.gs;
        a.rot.scales[dst * groups_row + gi] = f32_to_bf16(sc);
        a.rot.biases[dst * groups_row + gi] = f32_to_bf16(bi);
      }
      uint32_t* out = a.rot.packed + dst * words_row + half * words_half;
      if (whole) {
        if (live) {
          if (bits == 4) out[c] = uint32_t(chk[0]);
          else *reinterpret_cast<uint2*>(out + 2 * c) = uint2{uint32_t(chk[0]), uint32_t(chk[0] >> 32)};
        }
        continue;
      }
      // Rows 4 q' + i of the tile (q' = 0..3) exchange their chunks.
      ch[q * (NC / 8) + c] = chk[0];
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
      for (int w = lane; w < 4 * words_half; w += kWave) {
        const int rq = w / words_half, wi = w - rq * words_half;
        const int64_t r2 = row0 + 4 * rq + i;
        if (r2 < a.rows) {
          const int64_t d2 = dst_row(r2, a.s, a.dst_cap, a.dst_start);
          a.rot.packed[d2 * words_row + half * words_half + wi] =
              aq::packed_word(ch + rq * (NC / 8), wi, bits);
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();  // the chunks are reused by the next row
    }
  }
}

// Workgroups [0, rot_blocks) rotate and quantize tiles of a.rot; then every
// workgroup quantizes row blocks of a.plain (if any), grid-stride.
template <int D>
__global__ __launch_bounds__(kRT) void affine_quantize_rot_kernel(const RArgs a) {
  using S = RShape<D>;
  __shared__ __attribute__((aligned(16))) unsigned char lds_r[S::kLdsBytes];
  __shared__ uint64_t chunks[S::kChunks];
  static_assert(kRW * kWave * QShape<D, kRW>::kUnits <= S::kChunks, "plain path chunks fit");
  static_assert(kRW * 4 * (S::kNC / 8) <= S::kChunks, "rotate path chunks fit");
  if (int(blockIdx.x) < a.rot_blocks) rotate_quantize_tiles<D>(a, lds_r, chunks);
  if (a.plain_blocks > 0) {
    __syncthreads();  // every wavefront is done with its rotate-phase chunks
    for (int blk = blockIdx.x; blk < a.plain_blocks; blk += gridDim.x)
      quantize_rows_block<D, kRW>(a.plain, blk, a.rows, a.s, a.dst_cap, a.dst_start, a.gs,
                                  chunks);
  }
}

// mlx::dequantize (bf16(fma(scale, code, bias)), one rounding), one value a thread: the
// path for an output that is not 16-byte aligned.
__global__ void affine_dequantize_kernel(const uint32_t* __restrict__ packed,
                                         const uint16_t* __restrict__ scales,
                                         const uint16_t* __restrict__ biases, int64_t rows,
                                         int dim, int gs, int bits, uint16_t* __restrict__ out) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= rows * dim) return;
  const int64_t r = i / dim;
  const int e = int(i % dim);
  const uint32_t* pw = packed + r * (dim * bits / 32);
  const int bit = e * bits;
  uint64_t w = pw[bit / 32];
  if ((bit % 32) + bits > 32) w |= uint64_t(pw[bit / 32 + 1]) << 32;
  const uint32_t code = uint32_t(w >> (bit % 32)) & ((1u << bits) - 1);
  const int groups = dim / gs;
  const float sc = bf16_to_f32(scales[r * groups + e / gs]);
  const float bi = bf16_to_f32(biases[r * groups + e / gs]);
  out[i] = f32_to_bf16(fmaf(sc, float(code), bi));
}

// The same values eight at a time: a thread takes 8 consecutive values of a
// row (one 16-byte store; `out` 16-byte aligned), dim / 8 threads a row
// (lg8 = log2(dim / 8), lg_gs = log2(gs)). The 8 codes start on a byte
// (8 * bits bits from bit 8 c8 * bits) and end within the 64 bits from the
// word holding their first bit at every width: two loads, the second only
// when they run into the next word.
__global__ __launch_bounds__(256) void affine_dequantize8_kernel(
    const uint32_t* __restrict__ packed, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, int64_t n8, int lg8, int lg_gs, int bits,
    uint16_t* __restrict__ out) {
  const int64_t j = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (j >= n8) return;
  const int64_t r = j >> lg8;
  const int c8 = int(j & ((int64_t(1) << lg8) - 1)), e0 = 8 * c8;
  const int dim = 8 << lg8;
  const uint32_t* pw = packed + r * (dim * bits / 32);
  const int64_t gi = r * (dim >> lg_gs) + (e0 >> lg_gs);
  const float sc = bf16_to_f32(scales[gi]);
  const float bi = bf16_to_f32(biases[gi]);
  const int bit0 = e0 * bits, sh = bit0 % 32;
  uint64_t win = pw[bit0 / 32];
  if (sh + 8 * bits > 32) win |= uint64_t(pw[bit0 / 32 + 1]) << 32;
  win >>= sh;
  uint32_t o[4];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t code = uint32_t(win >> (e * bits)) & ((1u << bits) - 1);
    const uint32_t v = f32_to_bf16(fmaf(sc, float(code), bi));
    if (e % 2 == 0)
      o[e / 2] = v;
    else
      o[e / 2] |= v << 16;
  }
  *reinterpret_cast<uint4*>(out + j * 8) = uint4{o[0], o[1], o[2], o[3]};
}

bool valid_bits(int bits) {
  return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
}

int32_t check_affine_shape(int32_t dim, int32_t gs, int32_t bits) {
  if (!valid_bits(bits)) return fail(TQKV_EUNSUPPORTED, "affine bits=%d not in {2,3,4,5,6,8}", bits);
  if (!(gs == 32 || gs == 64 || gs == 128))
    return fail(TQKV_EUNSUPPORTED, "group_size=%d not in {32,64,128}", gs);
  if (!(dim == 32 || dim == 64 || dim == 128 || dim == 256 || dim == 512 || dim == 1024))
    return fail(TQKV_EUNSUPPORTED, "dim=%d not in {32,...,1024}", dim);
  if (dim % gs != 0 || (dim * bits) % 32 != 0)
    return fail(TQKV_EINVAL_SHAPE, "dim=%d, group_size=%d, bits=%d do not tile", dim, gs, bits);
  return TQKV_OK;
}

// Launches the quantize kernel over one or two tensors of the same shape.
int32_t launch_quantize(const QArgs& a0, int dim, tqkv_stream stream) {
  QArgs a = a0;
  int rows_per_block = 0;
  switch (dim) {
    case 32: rows_per_block = QShape<32>::kRows; break;
    case 64: rows_per_block = QShape<64>::kRows; break;
    case 128: rows_per_block = QShape<128>::kRows; break;
    case 256: rows_per_block = QShape<256>::kRows; break;
    case 512: rows_per_block = QShape<512>::kRows; break;
    case 1024: rows_per_block = QShape<1024>::kRows; break;
    default: return fail(TQKV_EUNSUPPORTED, "dim=%d", dim);
  }
  const int n_t = a.t[1].x ? 2 : 1;
  if (a.rows > 0x7fffffffLL)
    return fail(TQKV_EINVAL_SHAPE, "%lld rows exceed one launch", (long long)a.rows);
  const int64_t bpt = (a.rows + rows_per_block - 1) / rows_per_block;
  a.blocks_per_tensor = int(bpt);
  a.n_blocks = int(bpt * n_t);
  // Enough workgroups to fill the chip several times over; larger inputs
  // loop (grid stride).
  const int grid = a.n_blocks < 8192 ? a.n_blocks : 8192;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  switch (dim) {
    case 32: hipLaunchKernelGGL(affine_quantize_kernel<32>, dim3(grid), dim3(kQThreads), 0, st, a); break;
    case 64: hipLaunchKernelGGL(affine_quantize_kernel<64>, dim3(grid), dim3(kQThreads), 0, st, a); break;
    case 128: hipLaunchKernelGGL(affine_quantize_kernel<128>, dim3(grid), dim3(kQThreads), 0, st, a); break;
    case 256: hipLaunchKernelGGL(affine_quantize_kernel<256>, dim3(grid), dim3(kQThreads), 0, st, a); break;
    case 512: hipLaunchKernelGGL(affine_quantize_kernel<512>, dim3(grid), dim3(kQThreads), 0, st, a); break;
    default: hipLaunchKernelGGL(affine_quantize_kernel<1024>, dim3(grid), dim3(kQThreads), 0, st, a); break;
  }
  TQKV_LAUNCHED();
  return ok();
}

// Launches the rotate-and-quantize kernel over a.rot (and a.plain, if set).
int32_t launch_rotated(RArgs a, int dim, tqkv_stream stream) {
  if (a.rows > 0x7fffffffLL)
    return fail(TQKV_EINVAL_SHAPE, "%lld rows exceed one launch", (long long)a.rows);
  const int halves = dim / 128;
  const int64_t tiles = (a.rows + kTileRows - 1) / kTileRows;
  a.tiles = int(tiles);
  // Workgroups that fit the chip at once (one a CU: R's LDS); each rotate
  // workgroup holds its R columns in LDS, so it takes several tiles a
  // wavefront rather than being relaunched; the plain rows follow on every
  // workgroup.
  const int slots = 256;
  const int64_t want = (tiles + kRW - 1) / kRW;
  a.groups = int(want < slots / halves ? want : slots / halves);
  a.rot_blocks = a.groups * halves;
  const int rows_per_plain = dim == 128 ? QShape<128, kRW>::kRows : QShape<256, kRW>::kRows;
  a.plain_blocks = a.plain.x ? int((a.rows + rows_per_plain - 1) / rows_per_plain) : 0;
  const int plain_grid = a.plain_blocks < slots ? a.plain_blocks : slots;
  const int grid = a.rot_blocks > plain_grid ? a.rot_blocks : plain_grid;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (dim == 128)
    hipLaunchKernelGGL(affine_quantize_rot_kernel<128>, dim3(grid), dim3(kRT), 0, st, a);
  else
    hipLaunchKernelGGL(affine_quantize_rot_kernel<256>, dim3(grid), dim3(kRT), 0, st, a);
  TQKV_LAUNCHED();
  return ok();
}

int32_t check_rotated(const void* x, const float* rotation, int32_t dim, int32_t gs) {
  if (!(dim == 128 || dim == 256))
    return fail(TQKV_EUNSUPPORTED,
                "rotate-and-quantize dim=%d not in {128, 256} (use tqkv_rotate_bf16, then "
                "tqkv_affine_quantize)", dim);
  if (gs > 128) return fail(TQKV_EUNSUPPORTED, "group_size=%d above 128", gs);
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(rotation)) % 16 != 0)
    return fail(TQKV_EINVAL_ARG, "x and rotation must be 16-byte aligned");
  return TQKV_OK;
}

int32_t check_rows(int64_t n_slabs, int64_t s, int64_t dst_cap, int64_t dst_start) {
  if (n_slabs < 0 || s < 0 || dst_start < 0 || dst_start + s > dst_cap)
    return fail(TQKV_EINVAL_SHAPE, "rows [%lld, %lld) do not fit a buffer of %lld",
                (long long)dst_start, (long long)(dst_start + s), (long long)dst_cap);
  return TQKV_OK;
}

}  // namespace
}  // namespace tqkv

using namespace tqkv;

extern "C" int32_t tqkv_affine_quantize(const uint16_t* x, int64_t n_slabs, int64_t s,
                                        int32_t dim, int32_t group_size, int32_t bits,
                                        uint32_t* packed, uint16_t* scales, uint16_t* biases,
                                        int64_t dst_cap, int64_t dst_start,
                                        tqkv_stream stream) {
  if (int32_t rc = check_affine_shape(dim, group_size, bits)) return rc;
  if (int32_t rc = check_rows(n_slabs, s, dst_cap, dst_start)) return rc;
  if (n_slabs == 0 || s == 0) return ok();
  if (!x || !packed || !scales || !biases) return fail(TQKV_EINVAL_ARG, "null pointer");
  QArgs a{};
  a.t[0] = QTensor{x, packed, scales, biases, bits};
  a.s = s;
  a.rows = n_slabs * s;
  a.dst_cap = dst_cap;
  a.dst_start = dst_start;
  a.gs = group_size;
  return launch_quantize(a, dim, stream);
}

extern "C" int32_t tqkv_affine_quantize_kv(const uint16_t* k, const uint16_t* v, int64_t n_slabs,
                                           int64_t s, int32_t dim, int32_t group_size,
                                           int32_t bits_k, int32_t bits_v, uint32_t* k_packed,
                                           uint16_t* k_scales, uint16_t* k_biases,
                                           uint32_t* v_packed, uint16_t* v_scales,
                                           uint16_t* v_biases, int64_t dst_cap,
                                           int64_t dst_start, tqkv_stream stream) {
  if (int32_t rc = check_affine_shape(dim, group_size, bits_k)) return rc;
  if (int32_t rc = check_affine_shape(dim, group_size, bits_v)) return rc;
  if (int32_t rc = check_rows(n_slabs, s, dst_cap, dst_start)) return rc;
  if (n_slabs == 0 || s == 0) return ok();
  if (!k || !v || !k_packed || !k_scales || !k_biases || !v_packed || !v_scales || !v_biases)
    return fail(TQKV_EINVAL_ARG, "null pointer");
  QArgs a{};
  a.t[0] = QTensor{k, k_packed, k_scales, k_biases, bits_k};
  a.t[1] = QTensor{v, v_packed, v_scales, v_biases, bits_v};
  a.s = s;
  a.rows = n_slabs * s;
  a.dst_cap = dst_cap;
  a.dst_start = dst_start;
  a.gs = group_size;
  return launch_quantize(a, dim, stream);
}

extern "C" int32_t tqkv_affine_quantize_rotated(const uint16_t* x, int64_t n_slabs, int64_t s,
                                                int32_t dim, int32_t group_size, int32_t bits,
                                                const float* rotation, uint32_t* packed,
                                                uint16_t* scales, uint16_t* biases,
                                                int64_t dst_cap, int64_t dst_start,
                                                uint16_t* rotated, tqkv_stream stream) {
  if (int32_t rc = check_affine_shape(dim, group_size, bits)) return rc;
  if (int32_t rc = check_rows(n_slabs, s, dst_cap, dst_start)) return rc;
  if (n_slabs == 0 || s == 0) return ok();
  if (!x || !rotation || !packed || !scales || !biases) return fail(TQKV_EINVAL_ARG, "null pointer");
  if (int32_t rc = check_rotated(x, rotation, dim, group_size)) return rc;
  if (rotated && reinterpret_cast<uintptr_t>(rotated) % 16 != 0)
    return fail(TQKV_EINVAL_ARG, "rotated must be 16-byte aligned");
  RArgs a{};
  a.rot = QTensor{x, packed, scales, biases, bits};
  a.R = rotation;
  a.rotated = rotated;
  a.s = s;
  a.rows = n_slabs * s;
  a.dst_cap = dst_cap;
  a.dst_start = dst_start;
  a.gs = group_size;
  return launch_rotated(a, dim, stream);
}

extern "C" int32_t tqkv_affine_quantize_kv_rotated(
    const uint16_t* k, const uint16_t* v, int64_t n_slabs, int64_t s, int32_t dim,
    int32_t group_size, int32_t bits_k, int32_t bits_v, const float* rotation,
    uint32_t* k_packed, uint16_t* k_scales, uint16_t* k_biases, uint32_t* v_packed,
    uint16_t* v_scales, uint16_t* v_biases, int64_t dst_cap, int64_t dst_start,
    tqkv_stream stream) {
  if (int32_t rc = check_affine_shape(dim, group_size, bits_k)) return rc;
  if (int32_t rc = check_affine_shape(dim, group_size, bits_v)) return rc;
  if (int32_t rc = check_rows(n_slabs, s, dst_cap, dst_start)) return rc;
  if (n_slabs == 0 || s == 0) return ok();
  if (!k || !v || !rotation || !k_packed || !k_scales || !k_biases || !v_packed || !v_scales ||
      !v_biases)
    return fail(TQKV_EINVAL_ARG, "null pointer");
  if (int32_t rc = check_rotated(k, rotation, dim, group_size)) return rc;
  if (reinterpret_cast<uintptr_t>(v) % 16 != 0)
    return fail(TQKV_EINVAL_ARG, "v must be 16-byte aligned");
  RArgs a{};
  a.rot = QTensor{k, k_packed, k_scales, k_biases, bits_k};
  a.plain = QTensor{v, v_packed, v_scales, v_biases, bits_v};
  a.R = rotation;
  a.s = s;
  a.rows = n_slabs * s;
  a.dst_cap = dst_cap;
  a.dst_start = dst_start;
  a.gs = group_size;
  return launch_rotated(a, dim, stream);
}

extern "C" int32_t tqkv_affine_dequantize(const uint32_t* packed, const uint16_t* scales,
                                          const uint16_t* biases, int64_t rows, int32_t dim,
                                          int32_t group_size, int32_t bits, uint16_t* out,
                                          tqkv_stream stream) {
  if (int32_t rc = check_affine_shape(dim, group_size, bits)) return rc;
  if (rows < 0) return fail(TQKV_EINVAL_SHAPE, "rows=%lld", (long long)rows);
  if (rows == 0) return ok();
  if (!packed || !scales || !biases || !out) return fail(TQKV_EINVAL_ARG, "null pointer");
  const int64_t n = rows * dim;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffffLL) return fail(TQKV_EINVAL_SHAPE, "too many rows");
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (reinterpret_cast<uintptr_t>(out) % 16 == 0) {
    // dim and group_size are powers of two (check_affine_shape).
    const int lg8 = __builtin_ctz(unsigned(dim / 8)), lg_gs = __builtin_ctz(unsigned(group_size));
    const int64_t n8 = n / 8;
    hipLaunchKernelGGL(affine_dequantize8_kernel, dim3(unsigned((n8 + 255) / 256)), dim3(256), 0,
                       st, packed, scales, biases, n8, lg8, lg_gs, bits, out);
  } else {
    hipLaunchKernelGGL(affine_dequantize_kernel, dim3(unsigned(blocks)), dim3(256), 0, st,
                       packed, scales, biases, rows, dim, group_size, bits, out);
  }
  TQKV_LAUNCHED();
  return ok();
}
