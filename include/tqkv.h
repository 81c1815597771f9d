/*
 * tqkv.h — C ABI of the MI355X-native compressed KV cache (libtqkv.so).
 *
 * The drop-in boundary for lumen-rs's compressed-KV path. Every entry point is
 * plain C: pointers, sizes and an explicit HIP stream, no C++ or torch types,
 * no exceptions across the boundary, an int32 status on return. Each
 * declaration names the reference interface it replaces (paths relative to
 * the lumen-rs tree).
 *
 * Conventions
 *   - Device pointers are caller-owned unless stated otherwise; host pointers
 *     are marked "host".
 *   - bf16 values travel as uint16_t bit patterns.
 *   - Cache tensors use the reference's layout [B, H_kv, cap, .] (token axis
 *     third, native_cache.rs:370-371): row (b, h, t) of a buffer with token
 *     capacity `cap` sits at ((b * H_kv + h) * cap + t) * row_elems.
 *   - Affine-quantized rows are MLX's triple: packed codes as an LSB-first
 *     stream of u32 words (D * bits / 32 per row), then bf16 scales and bf16
 *     biases (D / group_size per row each) (offload/lowbit.rs:220-240).
 *   - Stream arguments are hipStream_t; NULL means the default stream. Calls
 *     are asynchronous on that stream unless stated otherwise.
 *   - TQKV_EUNSUPPORTED is distinct from argument errors: it is the "layout
 *     unsupported, fall back" answer the reference's callers act on
 *     (gemma4_moe.rs:2357-2372).
 *   - One cache object per thread at a time; the library is reentrant across
 *     objects.
 */
#ifndef TQKV_H
#define TQKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* tqkv_stream;

#define TQKV_OK 0
#define TQKV_EINVAL_SHAPE 1  /* a shape, dimension or size is invalid */
#define TQKV_EINVAL_TARGET 2 /* a truncation target or position is out of range */
#define TQKV_EUNSUPPORTED 3  /* valid request this build does not implement */
#define TQKV_EDEVICE 4       /* a HIP runtime call failed */
#define TQKV_ENOMEM 5        /* a device or host allocation failed */
#define TQKV_EINVAL_ARG 6    /* a null pointer or an out-of-range scalar */

/* Name of a status code. */
const char* tqkv_status_string(int32_t status);
/* Detail of the last failing call on this thread ("" if none). */
const char* tqkv_last_error(void);
/* ABI version, major * 10000 + minor * 100 + patch. */
int32_t tqkv_version(void);

/* ======================================================================
 * Stateless kernels
 * ====================================================================== */

/*
 * Quantize-on-append, affine format: mlx::quantize(x, group_size, bits) as the
 * reference's caches call it (native_cache.rs:968-971, 1445-1448), bit-exact
 * with MLX's Metal kernel: per group, min/max, scale snapped so zero is a
 * level, round half away from zero, bf16 scale and bias.
 *
 * x: bf16 [n_slabs, s, dim]. Row j of slab i is written to row
 * (i * dst_cap + dst_start + j) of packed [., dim*bits/32] u32,
 * scales [., dim/group_size] bf16 and biases [., dim/group_size] bf16, so the
 * kernel writes straight into a cache buffer [B, H_kv, dst_cap, .] with
 * n_slabs = B * H_kv. bits in {2, 3, 4, 5, 6, 8}; group_size in {32, 64, 128}
 * dividing dim; dim <= 1024 and dim * bits % 32 == 0.
 */
int32_t tqkv_affine_quantize(const uint16_t* x, int64_t n_slabs, int64_t s, int32_t dim,
                             int32_t group_size, int32_t bits, uint32_t* packed,
                             uint16_t* scales, uint16_t* biases, int64_t dst_cap,
                             int64_t dst_start, tqkv_stream stream);

/*
 * mlx::dequantize(packed, scales, biases, group_size, bits) to bf16, as the
 * reference's prefill fallback uses it (gemma4_moe.rs:2394-2399):
 * out = bf16(bf16(scale * code) + bias). rows = number of [dim] rows.
 */
int32_t tqkv_affine_dequantize(const uint32_t* packed, const uint16_t* scales,
                               const uint16_t* biases, int64_t rows, int32_t dim,
                               int32_t group_size, int32_t bits, uint16_t* out,
                               tqkv_stream stream);

/*
 * One contiguous run of affine-quantized K/V rows for the decode kernel: the
 * fetched view of a cache (native_cache.rs:953, 1418) or a shared prefix
 * (native_cache.rs:2044-2051). Tokens [0, n) of each (b, kv head) slab are
 * attended; slabs are `cap` rows apart. shared = 1 means one batch-1 buffer
 * serves every batch row (the single-copy shared prefix).
 */
typedef struct tqkv_affine_seg {
  const uint32_t* k_packed;
  const uint16_t* k_scales;
  const uint16_t* k_biases;
  const uint32_t* v_packed;
  const uint16_t* v_scales;
  const uint16_t* v_biases;
  int64_t cap;
  int64_t n;
  int32_t shared;
  int32_t reserved;
} tqkv_affine_seg;

/*
 * Fused decode attention over affine-packed K/V: softmax(scale * q.K^T) . V
 * for one query position per head, dequantizing in registers, one read of the
 * packed cache. Replaces quantized_sdpa_decode (native_quant_attention.rs:
 * 237-338) and, for the layouts that kernel rejects (D=128 at 4 bits, any
 * 3-bit cache, K and V at different widths), its three-op fallback
 * quantized_kv_attention (native_attention.rs:396-453). With two segments it
 * is also sdpa_split over a shared prefix and a suffix (native_attention.rs:
 * 174-208): the keys of both segments enter one softmax.
 *
 * q: bf16 [B, H, 1, D]; out: bf16 [B, H, 1, D]. Query head h reads KV head
 * h / (H / H_kv). bits_k, bits_v in {3, 4, 8}; group_size in {32, 64, 128};
 * D in {64, 128, 256, 512}; H / H_kv in {1, 2, 3, 4, 6, 8} (at most 4 when
 * either width is 3 bits). n_segs in {1, 2}.
 * workspace: device scratch of tqkv_decode_workspace_size() bytes for the
 * split partials, or NULL to use a buffer the library keeps per device (grown
 * on demand); calls that share a workspace must not overlap in time. One
 * kernel launch when B * H_kv fills the GPU, else a split launch plus a merge.
 * Returns TQKV_EUNSUPPORTED for a layout outside these sets.
 */
int32_t tqkv_decode_attend_affine(const uint16_t* q, int32_t B, int32_t H, int32_t H_kv,
                                  int32_t D, int32_t group_size, int32_t bits_k,
                                  int32_t bits_v, float scale, const tqkv_affine_seg* segs,
                                  int32_t n_segs, uint16_t* out, void* workspace,
                                  size_t workspace_bytes, tqkv_stream stream);

/*
 * Which decode kernel tqkv_decode_attend_affine runs for a layout: "mfma"
 * (scores on the matrix cores; group_size 64, D in {64, 128, 256},
 * H / H_kv in {1, 2, 4, 8} with H / H_kv * D / 64 <= 16), "dot2" (every other
 * supported layout, or any layout when the environment variable
 * TQKV_DECODE_KERNEL=dot2 is set), or "" (unsupported). No counterpart in the
 * reference; for tests and benchmarks.
 */
const char* tqkv_decode_kernel_name(int32_t H, int32_t H_kv, int32_t D, int32_t group_size,
                                    int32_t bits_k, int32_t bits_v);

/* Bytes of workspace tqkv_decode_attend_affine needs for this shape. */
size_t tqkv_decode_workspace_size(int32_t B, int32_t H, int32_t H_kv, int32_t D,
                                  int64_t total_tokens);

/* ======================================================================
 * Benchmark utilities (no counterpart in the reference)
 * ====================================================================== */

/*
 * Fill out (bf16 [rows, dim]) with seeded N(0,1) values, a seeded fraction
 * `outlier_frac` of the channels multiplied by `outlier_mult`: the synthetic
 * K/V BASELINE-style workloads describe, generated on the device so a
 * multi-gigabyte cache needs no host copy. Deterministic for a given seed.
 */
int32_t tqkv_synth_bf16(uint16_t* out, int64_t rows, int32_t dim, uint64_t seed,
                        float outlier_frac, float outlier_mult, tqkv_stream stream);

/*
 * The reference's memory-bandwidth probe (bandwidth.rs:73-100) for this GPU:
 * *out = sum of the `bytes / 4` floats at `data` (16-byte aligned), reading
 * each byte once. scratch: device floats, at least 4096 of them. Two launches
 * per call; time a call to get the read bandwidth a streaming kernel can
 * reach, the practical ceiling beside the data-sheet peak.
 */
int32_t tqkv_read_probe(const float* data, size_t bytes, float* scratch, size_t scratch_bytes,
                        float* out, tqkv_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* TQKV_H */
