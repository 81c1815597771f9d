// CPU oracle for the compressed KV-cache path. TEST INFRASTRUCTURE ONLY.
//
// A restatement of the reference's algorithms in plain C++ (g++, built with
// -ffp-contract=off -fno-fast-math so every f32/f64 operation rounds the way
// the reference's Rust does). Only tests/, __graft_entry__.smoke() and the
// cpu_baseline leg of bench.py may load it, and only as the checker. The
// product library (lumen-rs_amd/) never links, loads or calls it.
//
// Each function cites the reference file:line it restates. Where a value is
// fixed by something other than the restatement itself (a golden digest, a
// known-answer test, a closed form), the test that pins it is named in the
// function's comment; functions with no such pin say "parity unpinned".
#pragma once
#include <cstdint>
#include <cstddef>
#include <string>
#include <vector>

namespace oracle {

// ---------------------------------------------------------------- numerics
// bf16 <-> f32, round to nearest even, NaN to the canonical quiet NaN.
// Restates offload/lowbit.rs:210-218 (MLX's float_to_bfloat_bits adds the
// NaN check; inputs never carry NaN).
uint16_t f32_to_bf16(float x);
float bf16_to_f32(uint16_t b);

// SplitMix64 (native_cache/golden_tests.rs:26-35).
struct SplitMix64 {
  uint64_t s;
  explicit SplitMix64(uint64_t seed) : s(seed) {}
  uint64_t next();
};

// FNV-1a over shapes, dtypes and element bits (golden_tests.rs:70-155).
struct Digest {
  uint64_t h = 0xcbf29ce484222325ull;
  void bytes(const void* p, size_t n);
  void num(uint64_t n);
};

// ---------------------------------------------------------------- arrays
// A cache buffer as MLX holds it: shape [1, H, S, last], one dtype.
enum class DType : int { U8 = 1, U32 = 2, F32 = 3, BF16 = 4 };
size_t dtype_size(DType t);

struct Arr {
  DType dt = DType::F32;
  int h = 0, s = 0, last = 0;  // shape [1, h, s, last]
  std::vector<uint8_t> data;    // row-major bytes
  Arr() = default;
  Arr(DType d, int h_, int s_, int l_) : dt(d), h(h_), s(s_), last(l_),
      data(size_t(h_) * s_ * l_ * dtype_size(d), 0) {}
  size_t row_bytes() const { return size_t(last) * dtype_size(dt); }
  uint8_t* row(int hh, int ss) { return data.data() + (size_t(hh) * s + ss) * row_bytes(); }
  const uint8_t* row(int hh, int ss) const { return data.data() + (size_t(hh) * s + ss) * row_bytes(); }
};

// Axis-2 (token axis) slices and concatenation; zeros of a shape.
Arr zeros(DType d, int h, int s, int last);
Arr slice2(const Arr& a, int start, int end);
Arr concat2(const std::vector<const Arr*>& parts);
void slice_update2(Arr& buf, int start, const Arr& src);
void digest_array(Digest& d, const Arr& a);

// ---------------------------------------------------------------- codec
// lumen-core/src/lloyd_max.rs:74-122 (compute), :132-144 (quantize),
// :165-187 (mse). Pinned by Max (1960) N(0,1) tables and the reference's own
// thresholds (lloyd_max.rs:216-322).
struct Codebook {
  uint32_t bits = 0;
  std::vector<double> boundaries;  // n_levels + 1, first -inf, last +inf
  std::vector<double> centroids;   // n_levels
  int n_levels() const { return 1 << bits; }
  uint8_t quantize(double x) const;
  double mse() const;
};
bool codebook_compute(uint32_t bits, size_t n_iter, Codebook* out);

// Seeded Haar rotation by modified Gram-Schmidt plus Mezzadri's sign fix
// (rotation.rs:35-89). The algorithm is the reference's; the N(0,1) stream is
// this build's own (SplitMix64 + Box-Muller), because the reference's rand
// 0.10 ChaCha12 stream is not available here: R values are parity unpinned
// and enter every bit-exact check as an input.
std::vector<float> rotation_random(int dim, uint64_t seed);
// y = R x, sequential f32 sum per row (rotation.rs:91-99).
void rotation_apply(const float* R, int dim, const float* x, float* y);
// x = R^T y, accumulated row by row (rotation.rs:102-113).
void rotation_apply_inverse(const float* R, int dim, const float* y, float* x);

// bitpack.rs:11-52: LSB-first, 64/bits codes per u64 word.
size_t packed_words(size_t n, uint32_t bits);
std::vector<uint64_t> pack_codes(const uint8_t* codes, size_t n, uint32_t bits);
std::vector<uint8_t> unpack_codes(const uint64_t* packed, size_t n, uint32_t bits);

// qjl.rs:40-127. Phi entries N(0,1)/sqrt(m) from this build's own stream
// (values parity unpinned, an input like R).
std::vector<float> qjl_random(int dim, int m, uint64_t seed);
size_t qjl_packed_len(size_t m);
std::vector<uint64_t> qjl_project_and_pack(const float* phi, int m, int dim, const float* r);
std::vector<float> qjl_project_query(const float* phi, int m, int dim, const float* q);
float qjl_correction_from_projection(const float* pq, int m, const uint64_t* packed, float rnorm);

// compressor.rs:61-107 and config.rs:32-57.
struct Compressed {
  std::vector<uint64_t> stage1;
  std::vector<uint64_t> stage2;
  float residual_norm = 0.f;
  float scale = 0.f;
};
struct Compressor {
  int dim = 0, m = 0;
  uint32_t bits = 0;
  std::vector<float> R, phi;
  Codebook cb;
  Compressed compress_one(const float* x) const;
  // compressor.rs:165-184
  std::vector<float> scores_stage1(const float* q, const std::vector<Compressed>& cs) const;
  // compressor.rs:122-159
  std::vector<float> scores_two_stage(const float* q, const std::vector<Compressed>& cs) const;
  // simple.rs:40-62 + 105-118
  std::vector<float> attend_values(const float* w, const std::vector<Compressed>& cs) const;
};

// ---------------------------------------------------------------- MLX affine
// MLX affine quantization of bf16 rows of length `dim` with groups of `gs`,
// as the Metal kernel computes it (MLX v0.2x-0.3x quantized.h
// affine_quantize; the reference calls it at native_cache.rs:968-971).
// Packed codes are an LSB-first stream of u32 words (offload/lowbit.rs:220-240).
// Pinned at 4 bits / gs64 by the reference's recorded golden digests
// (golden_tests.rs:425-463); 3 and 8 bits are parity unpinned.
enum class RoundMode : int { HalfAway = 0, HalfEven = 1 };
struct AffineOpts {
  RoundMode round = RoundMode::HalfAway;
  bool wmax_starts_at_zero = true;  // the Metal kernel's w_max init (see affine.cpp)
  bool clip_low = false;            // the CPU fallback clips codes at 0
};
void affine_quantize_rows(const uint16_t* w, size_t rows, int dim, int gs, int bits,
                          uint32_t* packed, uint16_t* scales, uint16_t* biases,
                          const AffineOpts& o = AffineOpts());
// The same over f32 rows with f32 scales and biases (MLX's quantize of an
// f32 tensor; w_min starts from FLT_MAX in the Metal kernel).
void affine_quantize_rows_f32(const float* w, size_t rows, int dim, int gs, int bits,
                              uint32_t* packed, float* scales, float* biases,
                              const AffineOpts& o = AffineOpts());
// MLX dequantize to bf16: bf16(fma(scale, code, bias)), one rounding (what
// the reference's fixture records for MLX's kernel, see affine.cpp), or
// with two_roundings bf16(bf16(scale * code) + bias), the secondary reading.
void affine_dequantize_rows(const uint32_t* packed, const uint16_t* scales,
                            const uint16_t* biases, size_t rows, int dim, int gs,
                            int bits, uint16_t* out, bool two_roundings = false);
// MLX dequantize of an f32-scaled table: fmaf(scale, code, bias).
void affine_dequantize_rows_f32(const uint32_t* packed, const float* scales, const float* biases,
                                size_t rows, int dim, int gs, int bits, float* out);
uint32_t read_code(const uint32_t* words, size_t i, int bits);
// Code i of an LSB-first u32 stream (offload/lowbit.rs:220-240 write_code).
void write_code(uint32_t* words, size_t i, int bits, uint32_t code);

// ---------------------------------------------------------------- caches
// Every cache kind of native_cache.rs restated over Arr buffers, replaying the
// reference's golden plans (golden_tests.rs:157-497). prealloc mirrors
// LUMEN_NATIVE_KV_STEP_PREALLOC.
uint64_t golden_digest(const std::string& kind, const std::string& plan, bool prealloc,
                       const AffineOpts& ao = AffineOpts());

// A golden plan's inputs without the cache (see caches.cpp): events are
// ('U', rows S, byte offset of the update's arrays in data) or
// ('R', rewind target, -).
struct GoldenEvent {
  char op;
  int64_t n;
  int64_t at;
};
struct GoldenTape {
  int64_t max_size = 0, keep = 0;
  std::vector<GoldenEvent> events;
  std::vector<uint8_t> data;
};
GoldenTape golden_tape(const std::string& kind, const std::string& plan);

// ---------------------------------------------------------------- attention
// native_attention.rs:545-622: may query row i (absolute q_start+i) attend to
// key k (absolute first_held+k)?
bool mask_allowed(size_t q_abs, size_t k_abs, long window /* <0: none */);

}  // namespace oracle
