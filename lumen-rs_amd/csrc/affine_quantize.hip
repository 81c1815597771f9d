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

template <int D>
struct QShape {
  static constexpr int kEpl = 16;                 // elements a lane
  static constexpr int kLpr = D / kEpl;           // lanes a row
  static constexpr int kRpw = kWave / kLpr;       // rows a wavefront
  static constexpr int kRows = kQWaves * kRpw;    // rows a block
  static constexpr int kUnits = kEpl / 8;         // 8-code chunks a lane
};

template <int D>
__global__ __launch_bounds__(kQThreads) void affine_quantize_kernel(const QArgs a) {
  using S = QShape<D>;
  constexpr int EPL = S::kEpl, LPR = S::kLpr;
  __shared__ uint64_t chunks[kQWaves][kWave * S::kUnits];
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  const int lir = lane % LPR;                // lane in its row
  const int rw = lane / LPR;                 // row in the wavefront
  uint64_t* ch = chunks[wave] + rw * (D / 8);

  for (int blk = blockIdx.x; blk < a.n_blocks; blk += gridDim.x) {
    const int ti = blk / a.blocks_per_tensor;  // uniform: K then V
    const QTensor& t = a.t[ti];
    const int64_t r = int64_t(blk % a.blocks_per_tensor) * S::kRows + wave * S::kRpw + rw;
    const bool live = r < a.rows;
    const int64_t rr = live ? r : a.rows - 1;  // dead rows recompute the last one
    // 32-bit division: the host keeps rows (and so s) below 2^31.
    const uint32_t slab = uint32_t(rr) / uint32_t(a.s), j = uint32_t(rr) - slab * uint32_t(a.s);
    const int64_t dst = int64_t(slab) * a.dst_cap + a.dst_start + j;

    float v[EPL];
    aq::load_lane(t.x + rr * D + lir * EPL, v);
    const int bits = t.bits;
    const aq::LaneCodes qc = aq::quantize_lane(v, a.gs, bits);
    const int lpg = a.gs / EPL;  // lanes a group: a power of two, <= LPR
    const int groups = D / a.gs;
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
}

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
  const float prod = bf16_to_f32(f32_to_bf16(sc * float(code)));
  out[i] = f32_to_bf16(prod + bi);
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
  hipLaunchKernelGGL(affine_dequantize_kernel, dim3(unsigned(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), packed, scales, biases, rows, dim,
                     group_size, bits, out);
  TQKV_LAUNCHED();
  return ok();
}
