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
#define TQKV_ECORRUPT 7      /* a snapshot's bytes fail a format check (kv_disk's Err) */

/* Name of a status code. */
const char* tqkv_status_string(int32_t status);
/* Detail of the last failing call on this thread ("" if none). */
const char* tqkv_last_error(void);
/* ABI version, major * 10000 + minor * 100 + patch: tqkv_version() returns
 * the TQKV_ABI_VERSION this header declares. 0.2.0 added tqkv_cache_config's
 * encode and reserved fields (its size went from 64 to 72 bytes). */
#define TQKV_ABI_VERSION 200
int32_t tqkv_version(void);
/* Frees the scratch the library keeps per device for calls given no
 * workspace (no counterpart in the reference). The scratch grows by at
 * least doubling and keeps outgrown buffers until this call (so a growing
 * call never waits for queued work); this waits for every device that holds
 * scratch to finish its work, then frees it all. The next call that needs
 * scratch allocates again. */
int32_t tqkv_scratch_release(void);
/* Bytes of that scratch the library holds now, over every device (current
 * buffers and outgrown ones not yet released). Host bookkeeping only. */
size_t tqkv_scratch_bytes(void);

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
 * Both quantize calls of one cache append (K with bits_k, V with bits_v;
 * native_cache.rs:968-971 and 1445-1448 quantize keys, then values) in one
 * launch, each bit-exact with tqkv_affine_quantize on the same arguments.
 * K and V share n_slabs, s, dim, group_size, dst_cap and dst_start.
 */
int32_t tqkv_affine_quantize_kv(const uint16_t* k, const uint16_t* v, int64_t n_slabs, int64_t s,
                                int32_t dim, int32_t group_size, int32_t bits_k, int32_t bits_v,
                                uint32_t* k_packed, uint16_t* k_scales, uint16_t* k_biases,
                                uint32_t* v_packed, uint16_t* v_scales, uint16_t* v_biases,
                                int64_t dst_cap, int64_t dst_start, tqkv_stream stream);

/*
 * The affine + rotation cache mode (gemma4_moe.rs:4154-4173): k_to_cache =
 * rotate_last_axis(k, R) (turboquant.rs:258-267: bf16(f32(x) @ R)), then the
 * cache's mlx::quantize, in one pass with no rotated copy in HBM. The product
 * runs on the matrix cores in f32 (MLX's summation order is its own; each
 * rotated element is within an f32 sum's error bound plus half a bf16 step
 * of the exact product), the quantize is tqkv_affine_quantize's bit for bit
 * on the rotated bf16 rows.
 * rotation: device f32 [dim, dim] row-major (y = x R). dim in {128, 256}
 * (TQKV_EUNSUPPORTED otherwise: use tqkv_rotate_bf16, then
 * tqkv_affine_quantize), group_size <= 128; x and rotation 16-byte aligned.
 * `rotated` (optional, NULL for none): bf16 [n_slabs * s, dim] receives the
 * rotated rows. Device.
 */
int32_t tqkv_affine_quantize_rotated(const uint16_t* x, int64_t n_slabs, int64_t s, int32_t dim,
                                     int32_t group_size, int32_t bits, const float* rotation,
                                     uint32_t* packed, uint16_t* scales, uint16_t* biases,
                                     int64_t dst_cap, int64_t dst_start, uint16_t* rotated,
                                     tqkv_stream stream);
/*
 * A cache append of that mode in one launch: K rotated by R and quantized
 * (as tqkv_affine_quantize_rotated), V quantized as it is (the reference does
 * not rotate V). Arguments as tqkv_affine_quantize_kv plus `rotation`.
 */
int32_t tqkv_affine_quantize_kv_rotated(const uint16_t* k, const uint16_t* v, int64_t n_slabs,
                                        int64_t s, int32_t dim, int32_t group_size,
                                        int32_t bits_k, int32_t bits_v, const float* rotation,
                                        uint32_t* k_packed, uint16_t* k_scales,
                                        uint16_t* k_biases, uint32_t* v_packed,
                                        uint16_t* v_scales, uint16_t* v_biases, int64_t dst_cap,
                                        int64_t dst_start, tqkv_stream stream);

/*
 * mlx::dequantize(packed, scales, biases, group_size, bits) to bf16, as the
 * reference's prefill fallback uses it (gemma4_moe.rs:2394-2399):
 * out = bf16(fma(scale, code, bias)), one rounding of the f32 multiply-add
 * (MLX's dequantize as the reference's qwen4exp_tiny fixture records it,
 * reference/mtp_outputs.safetensors mtp_embedded). rows = number of [dim]
 * rows.
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
 * h / (H / H_kv). (bits_k, bits_v): 3, 4 or 8 bits each in any pair, or 2,
 * 5 or 6 bits for both; group_size in {32, 64, 128}; D in {64, 128, 256,
 * 512}; H / H_kv from 1 to 32 (the reference's limit): groups of 1, 2, 3, 4,
 * 6 or 8 heads in one launch (6 or 8 heads of a 2/3/5/6-bit cache as two
 * launches of half the heads), any other group as launches of its largest
 * such divisor, each launch reading the keys once (16 heads: two of 8).
 * n_segs in {1, 2}.
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
 * tqkv_decode_attend_affine without any allocation: no counterpart in the
 * reference. For callers that cannot call hipMalloc (code under HIP graph
 * capture, tight serving loops, harnesses that forbid it). Same arguments
 * and results (bit-identical: the same kernels and split plan) as
 * tqkv_decode_attend_affine without a workspace: the split partials live in
 * a static device array of TQKV_NOALLOC_SCRATCH_BYTES that every device
 * running the library holds until the process ends. The first call on a
 * device looks up that device's copy (make it outside any graph capture);
 * later calls allocate nothing. A call needing more partial bytes than the
 * array holds returns TQKV_EINVAL_SHAPE. All calls on one device share the
 * array: calls that overlap in time on one device race.
 */
#define TQKV_NOALLOC_SCRATCH_BYTES 33554432 /* 32 MiB */
int32_t tqkv_decode_attend_affine_noalloc(const uint16_t* q, int32_t B, int32_t H,
                                          int32_t H_kv, int32_t D, int32_t group_size,
                                          int32_t bits_k, int32_t bits_v, float scale,
                                          const tqkv_affine_seg* segs, int32_t n_segs,
                                          uint16_t* out, tqkv_stream stream);

/*
 * A decode step's append and attention in one kernel: the reference's
 * update_and_fetch of one token followed by quantized_decode_attention over
 * the fetched view (gemma4_moe.rs:4081, 4125). Same result as
 * tqkv_affine_quantize_kv(k, v, B * H_kv slabs, s = 1, ..., dst_cap,
 * dst_row) and then tqkv_decode_attend_affine over `segs` plus the new row:
 * the new K and V rows (bf16 [B, H_kv, 1, D], 16-byte aligned) are quantized
 * bit-exactly as that call would, written at row dst_row of every slab of
 * the destination buffers ([B, H_kv, dst_cap, .]), and enter the softmax as
 * one more key. `segs` must not hold that row (they may hold no rows at all).
 * Layouts of the MFMA decode kernel only (group_size 64, D in {64, 128, 256},
 * tqkv_decode_kernel_name() == "mfma"); TQKV_EUNSUPPORTED otherwise, and the
 * caller appends and attends in two calls.
 */
int32_t tqkv_decode_attend_affine_append(
    const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t D, int32_t group_size,
    int32_t bits_k, int32_t bits_v, float scale, const tqkv_affine_seg* segs, int32_t n_segs,
    const uint16_t* k, const uint16_t* v, uint32_t* k_packed, uint16_t* k_scales,
    uint16_t* k_biases, uint32_t* v_packed, uint16_t* v_scales, uint16_t* v_biases,
    int64_t dst_cap, int64_t dst_row, uint16_t* out, void* workspace, size_t workspace_bytes,
    tqkv_stream stream);

/*
 * Page-sparse decode over an affine cache, after sdpa_page_sparse
 * (native_attention.rs:210-329) and PageDigest (native_cache.rs:352-445).
 * Pages are 64 rows; a cache segment's buffers are [B, H_kv, cap, .].
 *
 * tqkv_page_digest_affine: key_min / key_max [n_slabs, max_pages, dim] bf16
 * get, for pages [page_from, page_to) of every slab, the elementwise min and
 * max over the page's 64 mlx::dequantize'd keys (bf16(fma(scale, code,
 * bias))). Digesting only the newly filled pages keeps the digest current, as
 * page_digest does.
 */
int32_t tqkv_page_digest_affine(const uint32_t* k_packed, const uint16_t* k_scales,
                                const uint16_t* k_biases, int64_t n_slabs, int64_t cap,
                                int32_t dim, int32_t group_size, int32_t bits, int64_t page_from,
                                int64_t page_to, uint16_t* key_min, uint16_t* key_max,
                                int64_t max_pages, tqkv_stream stream);

/* sparse_keep_pages (native_attention.rs:325-329): max(pages / 8, 64). */
int64_t tqkv_sparse_keep_pages(int64_t pages);

/*
 * The page choice of sdpa_page_sparse (native_attention.rs:240-271): per
 * (batch row, KV head), bound(p) = max over the query group of
 * sum_d max(q_d * key_max[p][d], q_d * key_min[p][d]) (f32); page 0 and the
 * last 4 of `pages` digested pages are always taken; the `keep` largest
 * bounds win, ties to the lower page. chosen: int32 [B, H_kv, keep] in
 * ascending page order. pages <= 4096, keep <= pages, D in {64, 128, 256,
 * 512}.
 */
int32_t tqkv_page_select(const uint16_t* q, int32_t B, int32_t H, int32_t H_kv, int32_t D,
                         const uint16_t* key_min, const uint16_t* key_max, int64_t max_pages,
                         int64_t pages, int32_t keep, int32_t* chosen, void* workspace,
                         size_t workspace_bytes, tqkv_stream stream);
/* Workspace of tqkv_page_select: the f32 bounds [B, H_kv, pages]. */
size_t tqkv_page_select_workspace_size(int32_t B, int32_t H_kv, int64_t pages);

/*
 * Decode attention over the chosen pages of one (unshared) segment plus its
 * undigested tail, rows [pages * 64, seg->n) (the attention of
 * sdpa_page_sparse, native_attention.rs:272-291): one softmax over both, as
 * tqkv_decode_attend_affine would give over those keys. Matrix-core layouts
 * only (tqkv_decode_kernel_name "mfma"); TQKV_EUNSUPPORTED otherwise.
 */
int32_t tqkv_decode_attend_affine_pages(const uint16_t* q, int32_t B, int32_t H, int32_t H_kv,
                                        int32_t D, int32_t group_size, int32_t bits_k,
                                        int32_t bits_v, float scale, const tqkv_affine_seg* seg,
                                        const int32_t* chosen, int32_t keep, int64_t pages,
                                        uint16_t* out, void* workspace, size_t workspace_bytes,
                                        tqkv_stream stream);

/*
 * sdpa_page_sparse whole: with pages <= keep, dense tqkv_decode_attend_affine
 * over the segment; otherwise tqkv_page_select into chosen_out (or the
 * workspace when chosen_out is NULL), then tqkv_decode_attend_affine_pages.
 * workspace: tqkv_sparse_workspace_size() bytes (required).
 */
int32_t tqkv_decode_attend_affine_sparse(const uint16_t* q, int32_t B, int32_t H, int32_t H_kv,
                                         int32_t D, int32_t group_size, int32_t bits_k,
                                         int32_t bits_v, float scale, const tqkv_affine_seg* seg,
                                         const uint16_t* key_min, const uint16_t* key_max,
                                         int64_t max_pages, int64_t pages, int32_t keep,
                                         uint16_t* out, int32_t* chosen_out, void* workspace,
                                         size_t workspace_bytes, tqkv_stream stream);
size_t tqkv_sparse_workspace_size(int32_t B, int32_t H, int32_t H_kv, int32_t D,
                                  int64_t total_tokens, int32_t keep);

/*
 * Which decode kernel tqkv_decode_attend_affine runs for a layout: "mfma"
 * (scores on the matrix cores; group_size 32, 64 or 128, D in {64, 128, 256},
 * heads a launch in {1, 2, 4, 8} with heads * D / group_size <= 16), "tiles"
 * (head dim 512: the prefill tile kernel with f16 operands, a sequence's
 * heads as one block's rows), "dot2" (every other
 * supported layout, or any layout when the environment variable
 * TQKV_DECODE_KERNEL=dot2 is set), or "" (unsupported). No counterpart in the
 * reference; for tests and benchmarks.
 */
const char* tqkv_decode_kernel_name(int32_t H, int32_t H_kv, int32_t D, int32_t group_size,
                                    int32_t bits_k, int32_t bits_v);
/* The same for a context whose longest segment holds max_rows rows: the
 * MFMA kernel addresses a (batch row, KV head)'s rows through 32-bit byte
 * offsets, so from max_rows * D >= 2^31 on the dot2 kernel serves the
 * layout (and a fused append, which needs the MFMA kernel, runs as two
 * calls). Host arithmetic only. */
const char* tqkv_decode_kernel_for_rows(int32_t H, int32_t H_kv, int32_t D, int32_t group_size,
                                        int32_t bits_k, int32_t bits_v, int64_t max_rows);

/*
 * Fused decode attention over a codebook cache (the GPU TurboQuant caches'
 * attention, turboquant.rs:763-923, for one query position): keys and
 * values stored rotated (y = R x) as u8 codes + f32 sigma [B, H_kv, cap, .];
 * the query is rotated, attention runs over centroid[c] * sigma in the
 * rotated basis, and the output returns through R^T. rotation f32 [D, D],
 * centroids f32 [2^bits] (device). D in {64, 128, 256, 512}; H / H_kv in
 * {1, 2, 4, 8, 16}. v_codes 4-byte aligned at D >= 256, 2-byte at D = 128
 * (TQKV_EINVAL_ARG otherwise). workspace:
 * tqkv_decode_codebook_workspace_size() bytes, or NULL for the library's
 * per-device buffer.
 */
int32_t tqkv_decode_attend_codebook(const uint16_t* q, int32_t B, int32_t H, int32_t H_kv,
                                    int32_t D, float scale, const float* rotation,
                                    const float* centroids_k, int32_t bits_k,
                                    const float* centroids_v, int32_t bits_v,
                                    const uint8_t* k_codes, const float* k_sigma,
                                    const uint8_t* v_codes, const float* v_sigma, int64_t cap,
                                    int64_t n, uint16_t* out, void* workspace,
                                    size_t workspace_bytes, tqkv_stream stream);
size_t tqkv_decode_codebook_workspace_size(int32_t B, int32_t H, int32_t D, int64_t total_tokens);
/*
 * The same attention over a codebook cache with QJL residual signs: each
 * key's score is the two-stage estimate of estimate_inner_products
 * (compressor.rs:122-159): stage 1 on the codes plus ||r|| sqrt(pi/2) /
 * sqrt(m) * sum_i sign_i (Phi q)_i (qjl.rs:76-118), the QJL stage of the
 * reference's TurboQuant attention (turboquant.rs:539-691) taken on the
 * scores instead of materializing K_eff. k_signs u32 [B, H_kv, cap,
 * ceil(m/32)], k_rnorm f32 [B, H_kv, cap], qjl f32 [m, D] (device),
 * 1 <= qjl_m <= 1024.
 */
int32_t tqkv_decode_attend_codebook_qjl(const uint16_t* q, int32_t B, int32_t H, int32_t H_kv,
                                        int32_t D, float scale, const float* rotation,
                                        const float* centroids_k, int32_t bits_k,
                                        const float* centroids_v, int32_t bits_v,
                                        const uint8_t* k_codes, const float* k_sigma,
                                        const uint32_t* k_signs, const float* k_rnorm,
                                        const float* qjl, int32_t qjl_m, const uint8_t* v_codes,
                                        const float* v_sigma, int64_t cap, int64_t n,
                                        uint16_t* out, void* workspace, size_t workspace_bytes,
                                        tqkv_stream stream);

/*
 * Prefill-chunk attention over affine-packed K/V on the matrix cores:
 * softmax(scale * Q K^T + mask) V for a chunk of L query rows per head.
 * Replaces dequantized_prefill_attention (gemma4_moe.rs:2382-2411): K and V
 * dequantize as mlx::dequantize does for bf16 (bf16(fma(scale, code,
 * bias)), one rounding), then attention runs with bf16 operands and f32 accumulation. When
 * 8 or more 256-row blocks share a KV head, the keys are dequantized once
 * into the library's per-device scratch (2 * B * H_kv * keys * D * 2 bytes,
 * at most 4 GiB; larger contexts dequantize in every block instead, in LDS)
 * and read from there; the two ways give the same bits. The mask is build_causal_mask_abs (native_attention.rs:
 * 545-622) in absolute positions: query row l sits at q_start + l and key k
 * (counted across both segments) at k_start + k; with causal != 0, key k is
 * visible iff k_abs <= q_abs and, when window > 0, q_abs < k_abs + window
 * (window < 0: no window; window == 0 is rejected). causal == 0: every key is
 * visible. That one rule covers the reference's causal SDPA,
 * lumen_sdpa_windowed and sdpa_with_mask branches. A row that sees no key
 * returns zeros.
 *
 * q: bf16 [B, H, L, D]; out: bf16 [B, H, L, D]; segs as for
 * tqkv_decode_attend_affine (1 or 2: a shared prefix, then a suffix).
 * D in {64, 128, 256, 512}; bits_k, bits_v in {2, 3, 4, 5, 6, 8}; group_size in
 * {32, 64, 128}. Uses the library's scratch for the dequantize-once rows:
 * calls that use it (this one, and decodes given a null workspace) must not
 * overlap in time on one device; tqkv_prefill_attend_affine_ws takes a
 * workspace instead.
 */
int32_t tqkv_prefill_attend_affine(const uint16_t* q, int32_t B, int32_t H, int32_t H_kv,
                                   int32_t L, int32_t D, int32_t group_size, int32_t bits_k,
                                   int32_t bits_v, float scale, const tqkv_affine_seg* segs,
                                   int32_t n_segs, int64_t q_start, int64_t k_start,
                                   int32_t causal, int64_t window, uint16_t* out,
                                   tqkv_stream stream);
/* tqkv_prefill_attend_affine with the caller's workspace (no counterpart in
 * the reference, whose prefill dequantizes into a fresh MLX array): the
 * dequantize-once rows go into `workspace` when it holds
 * tqkv_prefill_workspace_size(B, H_kv, D, keys of both segments) bytes;
 * with less (or NULL) every block dequantizes its own tiles in LDS. Either
 * way the same bits, no library allocation, and calls with different
 * workspaces may run concurrently. */
int32_t tqkv_prefill_attend_affine_ws(const uint16_t* q, int32_t B, int32_t H, int32_t H_kv,
                                      int32_t L, int32_t D, int32_t group_size, int32_t bits_k,
                                      int32_t bits_v, float scale, const tqkv_affine_seg* segs,
                                      int32_t n_segs, int64_t q_start, int64_t k_start,
                                      int32_t causal, int64_t window, uint16_t* out,
                                      void* workspace, size_t workspace_bytes,
                                      tqkv_stream stream);
/* Bytes of the prefill's dequantize-once rows: 2 * B * H_kv * rows * D * 2,
 * rows = keys, rounded up to a multiple of 64 at D = 128 (V is held there as
 * 64-key tiles). */
size_t tqkv_prefill_workspace_size(int32_t B, int32_t H_kv, int32_t D, int64_t total_keys);

/* Bytes of workspace tqkv_decode_attend_affine needs for this shape. */
size_t tqkv_decode_workspace_size(int32_t B, int32_t H, int32_t H_kv, int32_t D,
                                  int64_t total_tokens);

/* ======================================================================
 * The cache object: growing, rotating and shared-prefix KV caches
 * ====================================================================== */

/*
 * Device-resident KV cache with the reference's update/fetch/truncate
 * semantics, bit for bit (the recorded digests of native_cache/
 * golden_tests.rs:413-497 replay through it). Kinds and their slots (the
 * parallel buffers an update extends together, each [B, H_kv, cap, row]):
 *   TQKV_CACHE_BF16      keys bf16 [k_dim], values bf16 [v_dim]
 *                        (NativeKvCache :369-812, NativeRotatingKvCache
 *                        :1145-1280)
 *   TQKV_CACHE_AFFINE    MLX triples: k packed, k scales, k biases, v packed,
 *                        v scales, v biases (NativeKvCacheQuantized
 *                        :835-1126, NativeRotatingKvCacheQuantized :1297-1467)
 *   TQKV_CACHE_CODEBOOK  k codes u8 [k_dim], k sigma f32, [k QJL signs u32
 *                        [qjl_words], k residual norm f32,] v codes u8
 *                        [v_dim], v sigma f32 (NativeRotatingKvCacheTurboQuant
 *                        :1517-1856; rotating only)
 * max_size > 0 makes the cache a rotating window of max_size tokens whose
 * first `keep` are never evicted; max_size == 0 grows in 256-token steps.
 * prealloc mirrors LUMEN_NATIVE_KV_STEP_PREALLOC (native_cache.rs:39-59):
 * 1 = step-256 in-place growth and in-place ring writes for one-token
 * updates, 0 = the legacy concatenating path.
 */
#define TQKV_CACHE_BF16 0
#define TQKV_CACHE_AFFINE 1
#define TQKV_CACHE_CODEBOOK 2

typedef struct tqkv_cache tqkv_cache;

typedef struct tqkv_cache_config {
  int32_t kind;
  int32_t batch;
  int32_t kv_heads;
  int32_t k_dim;
  int32_t v_dim;
  int32_t group_size; /* affine */
  int32_t bits_k;     /* affine */
  int32_t bits_v;     /* affine */
  int32_t qjl_words;  /* codebook: u32 sign words per key row, 0 = no QJL */
  int32_t prealloc;
  int64_t max_size;
  int64_t keep;
  uint64_t seed;      /* codebook: rotation seed (QJL at seed + 1); the reference uses 42 */
  int32_t encode;     /* codebook: 0 = compress_one (tqkv_tq_encode: codes of R x), 1 = the
                         reference GPU cache's chain (tqkv_tq_encode_gpu_path mode 1 on keys
                         and values: codes of x R; QJL signs of the rotated residual) */
  int32_t reserved;
} tqkv_cache_config;

/*
 * A view of a cache's slots: rows [0, n) of every (batch row, KV head) slab,
 * slabs `cap` rows apart; slot[i] is the device address of row 0 of slab 0.
 * Valid until the next call that updates, truncates, splits or destroys the
 * cache.
 */
typedef struct tqkv_cache_view {
  int64_t n;
  int64_t cap;
  int32_t n_slots;
  int32_t reserved;
  void* slot[6];
  int64_t row_bytes[6];
} tqkv_cache_view;

typedef struct tqkv_cache_state {
  int64_t offset;      /* base_offset + tokens held (the reference's offset()) */
  int64_t idx;         /* ring write position (idx()) */
  int64_t cached_len;  /* buffer length in tokens (cached_len()), 0 if empty */
  int64_t base_offset; /* absolute position of the buffer's first token */
  int64_t view;        /* rows of the last fetched view */
  int32_t empty;       /* 1 before the first update (empty()) */
  int32_t n_slots;
} tqkv_cache_state;

/* Constructors NativeKvCache::new / NativeKvCacheQuantized::new /
 * NativeRotatingKvCache*::new (native_cache.rs:392, 845, 1159, 1313, 1541);
 * destroy frees the device buffers. */
int32_t tqkv_cache_create(const tqkv_cache_config* cfg, tqkv_cache** out);
int32_t tqkv_cache_destroy(tqkv_cache* cache);
/*
 * deep_clone (native_cache.rs:1575-1610; native_snapshot.rs:87-121 for the
 * fork of a prompt cache): a new cache with the source's configuration,
 * state and tables and its own copy of every buffer (stream-ordered device
 * copies), independent of the source from then on. A shared prefix the
 * source reads stays shared.
 */
int32_t tqkv_cache_clone(const tqkv_cache* src, tqkv_cache** out, tqkv_stream stream);

/*
 * update_and_fetch with the slots' new rows given as they are stored
 * (native_cache.rs:591, 953, 1235, 1418, 1756, 1804): rows[i] is a device
 * array [B, H_kv, s, row_i] for slot i. `fetched` (may be NULL) receives the
 * view the reference returns.
 */
int32_t tqkv_cache_update(tqkv_cache* cache, const void* const* rows, int64_t s,
                          tqkv_cache_view* fetched, tqkv_stream stream);

/*
 * update_and_fetch from bf16 keys and values [B, H_kv, s, dim]: stored as is
 * (bf16 kind), quantized on append straight into the cache rows (affine
 * kind, mlx::quantize as native_cache.rs:968-971, 1445-1448 call it), or
 * compressed by tqkv_tq_encode into codes + sigma (+ QJL signs and residual
 * norm for keys) (codebook kind; k_dim == v_dim in {64, 128, 256, 512}).
 */
int32_t tqkv_cache_append(tqkv_cache* cache, const uint16_t* k, const uint16_t* v, int64_t s,
                          tqkv_cache_view* fetched, tqkv_stream stream);

/*
 * truncate_to (native_cache.rs:778-811, 913-940, ring_truncate :304-335):
 * TQKV_EINVAL_TARGET where the reference returns Err (a target past the
 * tokens held; a rotating cache that has wrapped; an affine growing cache on
 * the legacy path). As in the reference, `target` counts the tokens this
 * buffer holds. Host-side bookkeeping only.
 */
int32_t tqkv_cache_truncate(tqkv_cache* cache, int64_t target);
/* clear() (native_cache.rs:739, 895, 1484): back to empty. */
int32_t tqkv_cache_clear(tqkv_cache* cache);
/* offset() / idx() / cached_len() / base_offset() / empty(). */
int32_t tqkv_cache_get_state(const tqkv_cache* cache, tqkv_cache_state* out);
/* The whole buffers (keys() / values(): n = cached_len, zero padding included). */
int32_t tqkv_cache_buffers(const tqkv_cache* cache, tqkv_cache_view* out);

/*
 * keep_suffix_from (native_cache.rs:464-494): drop the first prefix_len
 * tokens (now held once by a shared prefix cache) and record base_offset =
 * prefix_len. Growing caches only.
 */
int32_t tqkv_cache_keep_suffix_from(tqkv_cache* cache, int64_t prefix_len, tqkv_stream stream);
/*
 * Codebook kind: use the given rotation (host f32 [k_dim, k_dim] row-major,
 * the reference's TQRM matrix) and QJL matrix (host f32 [32 * qjl_words,
 * k_dim], or NULL) instead of drawing them from the seed
 * (TurboQuantCompressor::from_files, compressor.rs:35-58). Call before the
 * first append.
 */
int32_t tqkv_cache_set_tables(tqkv_cache* cache, const float* rotation, const float* qjl);

/*
 * Attach a batch-1 cache holding the shared prefix (SharedPrefixKv,
 * native_cache.rs:2044-2051); NULL detaches. Decode attention then reads the
 * prefix's first base_offset tokens once for every batch row and the cache's
 * own suffix, in one softmax (sdpa_split, native_attention.rs:174-208). The
 * prefix must outlive the attachment.
 */
int32_t tqkv_cache_attach_prefix(tqkv_cache* cache, const tqkv_cache* prefix);

/*
 * Fused decode attention over the last fetched view, plus the attached
 * prefix: tqkv_decode_attend_affine on the cache's own buffers (affine kind,
 * k_dim == v_dim), or tqkv_decode_attend_codebook (codebook kind). q: bf16
 * [B, H, 1, D]; out: bf16 [B, H, 1, D].
 */
int32_t tqkv_cache_decode_attend(const tqkv_cache* cache, const uint16_t* q, int32_t H,
                                 float scale, uint16_t* out, void* workspace,
                                 size_t workspace_bytes, tqkv_stream stream);

/*
 * One decode step: tqkv_cache_append of one token (k, v: bf16 [B, H_kv, 1,
 * dim]) then tqkv_cache_decode_attend (the reference's update_and_fetch +
 * quantized_decode_attention, gemma4_moe.rs:4081, 4125). On an affine cache
 * whose layout the MFMA decode kernel serves, the new token is quantized
 * inside the decode kernel (tqkv_decode_attend_affine_append): one launch
 * fewer, the same cache bytes. Otherwise the two calls. Growth and
 * rotation follow tqkv_cache_append exactly.
 */
int32_t tqkv_cache_append_decode(tqkv_cache* cache, const uint16_t* k, const uint16_t* v,
                                 const uint16_t* q, int32_t H, float scale, uint16_t* out,
                                 void* workspace, size_t workspace_bytes, tqkv_stream stream);

/*
 * Prefill-chunk attention over the last fetched view (plus the attached
 * prefix) for the L tokens just appended: tqkv_prefill_attend_affine with
 * queries at absolute positions [offset - L, offset) and the view's keys
 * ending at offset, causal, with the given sliding window (< 0: none). The
 * reference derives the same positions (cache_first_held_pos = kv_offset +
 * L - kv_actual, gemma4_moe.rs:2228). k_dim == v_dim. Affine caches read
 * their packed rows directly. Codebook caches follow the reference's
 * TurboQuant branch (gemma4_moe.rs:4546-4600): K and V dequantized to
 * bf16(centroid * sigma) (lloyd_max_dequantize_scaled), keys with QJL signs
 * corrected to K_eff, queries rotated by R and the output rotated back (the
 * cache holds rotated rows); this uses library scratch. bf16 caches attend
 * their rows as they are. An attached prefix is read for affine caches only.
 * q: bf16 [B, H, L, D]; out: bf16 [B, H, L, D].
 */
int32_t tqkv_cache_prefill_attend(const tqkv_cache* cache, const uint16_t* q, int32_t H,
                                  int32_t L, float scale, int64_t window, uint16_t* out,
                                  tqkv_stream stream);

/* ======================================================================
 * LKV2 snapshots (crates/lumen-mlx/src/kv_disk.rs)
 * ====================================================================== */

/* KvManifest's snapshot-level fields (kv_disk.rs:347-368). */
typedef struct tqkv_lkv_info {
  const char* model_fingerprint; /* NUL-terminated UTF-8 */
  uint64_t created_at_unix;
  uint64_t position;
  const uint32_t* prefix_tokens;
  int64_t n_prefix_tokens;
  int32_t has_last_token;
  uint32_t last_token;
  int32_t is_deep;
} tqkv_lkv_info;

/*
 * write_lkv (kv_disk.rs:371-404) of a snapshot whose layers are the given
 * caches, one LayerMeta each, laid out as the reference's snapshot code lays
 * its caches out (gemma4_moe.rs:1617-1693, turboquant_meta kv_disk.rs:
 * 2005-2025): bf16 growing = Full (the logical view [0, offset)), bf16
 * rotating = Sliding (the whole ring), affine = FullQuantized /
 * SlidingQuantized (whole (packed, scales, biases) buffers, group_size, bits
 * = the key width), codebook = FullTurboquant (max_size >= 2^31) /
 * SlidingTurboquant ([keys_codes u8, keys_sigma f32, values_codes,
 * values_sigma, keys_signs bf16 +-1 [.., m]?, keys_residual_norm f32?],
 * bits, qjl_m). Records are the rows the device holds, copied out after the
 * stream's pending work. out == NULL: only *bytes (the file size) is set;
 * else capacity must be at least that.
 */
int32_t tqkv_lkv_export(const tqkv_cache* const* layers, int32_t n_layers,
                        const tqkv_lkv_info* info, uint8_t* out, size_t capacity,
                        size_t* bytes, tqkv_stream stream);

/*
 * read_lkv's checks (kv_disk.rs:408-448) on a whole file in memory: magic,
 * version, manifest CRC and fields, every record's dtype, rank (<= 8),
 * dimensions, declared length (exactly what shape x dtype imply, and within
 * the file) and CRC, and no trailing bytes. TQKV_ECORRUPT names the first
 * fault (tqkv_last_error) where the reference returns Err; nothing is
 * allocated from an unchecked field.
 */
int32_t tqkv_lkv_check(const uint8_t* data, size_t bytes);

/* After the same checks: the manifest JSON as stored (NUL-terminated into
 * json, if given), its length, and the layer and record counts. */
int32_t tqkv_lkv_manifest(const uint8_t* data, size_t bytes, char* json, size_t capacity,
                          size_t* json_bytes, int32_t* n_layers, int32_t* n_records);

/*
 * from_disk_records / from_parts (gemma4_moe.rs:1700-1830,
 * turboquant_from_meta kv_disk.rs:2028-2061) for one layer: a new device
 * cache holding the layer's records with its offset, base_offset, idx,
 * max_size and keep. Geometry comes from the record shapes; an affine value
 * width from its packed record. A codebook layer's rotation and QJL tables
 * are drawn from `seed` (the file does not hold them; the reference uses
 * 42), or replaced with tqkv_cache_set_tables. Linear (SSM) and empty
 * layers: TQKV_EUNSUPPORTED.
 */
int32_t tqkv_lkv_import(const uint8_t* data, size_t bytes, int32_t layer, uint64_t seed,
                        tqkv_cache** out, tqkv_stream stream);

/* read_lkv then write_lkv: the same snapshot with its manifest re-serialized
 * (serde_json's compact form, fields in declaration order) and its records
 * copied. out == NULL: only *out_bytes. Host only. */
int32_t tqkv_lkv_rewrite(const uint8_t* data, size_t bytes, uint8_t* out, size_t capacity,
                         size_t* out_bytes);

/* CRC-32 (IEEE, the crc32fast crate's) of a host buffer. */
int32_t tqkv_crc32(const void* data, size_t bytes, uint32_t* out);

/* ======================================================================
 * TurboQuant codebook format
 * ====================================================================== */

/*
 * LloydMaxCodebook::compute (lumen-core/src/lloyd_max.rs:74-122): the 2^bits
 * level Lloyd-Max quantizer of N(0,1) after n_iter EM iterations, bit-
 * identical to the reference. Host memory: boundaries [2^bits + 1] (first
 * -inf, last +inf), centroids [2^bits]. Host-only (no GPU needed).
 */
int32_t tqkv_lloyd_max(uint32_t bits, size_t n_iter, double* boundaries, double* centroids);
/*
 * RotationMatrix::random (rotation.rs:35-89): a Haar orthogonal [dim, dim]
 * f32 matrix, row-major, by modified Gram-Schmidt with Mezzadri's sign fix,
 * from this library's seeded N(0,1) stream (SplitMix64 + Box-Muller; the
 * reference's rand/ChaCha12 stream is not reproduced: pass the reference's R
 * where its exact values matter). Host-only.
 */
int32_t tqkv_rotation_matrix(int32_t dim, uint64_t seed, float* out);
/* QJLProjector::new (qjl.rs:40-55): [m, dim] entries N(0,1)/sqrt(m), same
 * stream. Host-only. */
int32_t tqkv_qjl_matrix(int32_t dim, int32_t m, uint64_t seed, float* out);

/*
 * TurboQuantCompressor::compress (compressor.rs:61-116) on the device,
 * bit-exact given the same R, codebook and Phi: y = R x (sequential f32),
 * sigma = sqrt(sum y^2 / dim), codes = codebook level of y * (1/sigma)
 * (f64 decisions; all zero when sigma < 1e-10), and with qjl_m > 0 the
 * residual against R^T(centroid * sigma), its norm and the QJL sign bits
 * (bit r of a vector = (Phi_r . residual >= 0), LSB-first in u32 words).
 * x: [n_slabs, s, dim] f32 (x_is_bf16 = 0) or bf16; row j of slab i writes
 * row (i * dst_cap + dst_start + j) of codes u8 [., dim], sigma f32 [.],
 * signs u32 [., ceil(qjl_m / 32)], rnorm f32 [.] (device). rotation f32
 * [dim, dim] row-major, boundaries f64 [2^bits + 1], centroids_f32 [2^bits]
 * (the f64 centroids rounded), qjl f32 [qjl_m, dim] (device).
 * dim in {64, 128, 256, 512}.
 */
int32_t tqkv_tq_encode(const void* x, int32_t x_is_bf16, int64_t n_slabs, int64_t s,
                       int32_t dim, const float* rotation, const double* boundaries,
                       const float* centroids_f32, int32_t bits, const float* qjl, int32_t qjl_m,
                       uint8_t* codes, float* sigma, uint32_t* signs, float* rnorm,
                       int64_t dst_cap, int64_t dst_start, tqkv_stream stream);
/* rq = R q (RotationMatrix::apply, rotation.rs:91-99), f32 [dim], device. */
/*
 * The reference GPU cache's TurboQuant encode (the codes its TurboQuant
 * caches hold, turboquant.rs:398-423, 708-745; called at gemma4_moe.rs:
 * 4396-4430): y = x (mode 0, lloyd_max_quantize_stage1{,_fused}), y =
 * bf16(x M) (mode 1, rotate_last_axis then the encode: the reference's
 * default for K and V), or y = x M in f32 (mode 2,
 * rotate_and_lloyd_max_quantize_stage1_fused), M = rotation (transpose = 0)
 * or its transpose; sigma = sqrt(sum y^2 / dim) (f32), codes = the number
 * of boundaries_inner (f32 [2^bits - 1], lloyd_max_boundaries_inner,
 * ascending) at or below bf16(y / sigma) (IEEE divide). compress_one's
 * codes (tqkv_tq_encode) differ from these by the bf16 rounding of y /
 * sigma, the f32 boundaries and the rotation convention (R x there, x R
 * here). x: bf16 [n_slabs, s, dim]; row j of slab i writes row (i * dst_cap
 * + dst_start + j) of codes u8 [., dim] and sigma f32 [.]. dim in {64, 128,
 * 256, 512}. Device.
 */
int32_t tqkv_tq_encode_gpu_path(const uint16_t* x, int64_t n_slabs, int64_t s, int32_t dim,
                                const float* rotation, int32_t mode, int32_t transpose,
                                const float* boundaries_inner, int32_t bits, uint8_t* codes,
                                float* sigma, int64_t dst_cap, int64_t dst_start,
                                tqkv_stream stream);
int32_t tqkv_tq_rotate_query(const float* rotation, const float* q, int32_t dim, float* rq,
                             tqkv_stream stream);
/* estimate_inner_products_stage1 (compressor.rs:165-184) for n stored keys:
 * scores[t] = (sum_i rq_i * centroid[c_ti]) * sigma_t, bit-exact. Device. */
int32_t tqkv_tq_scores(const float* rq, const uint8_t* codes, const float* sigma,
                       const float* centroids_f32, int32_t dim, int64_t n, float* scores,
                       tqkv_stream stream);
/* QJLProjector::project_query (qjl.rs:76-84): pq[row] = Phi[row] . q, f32
 * [m], bit-exact (sums folded from -0.0 in index order). Device. */
int32_t tqkv_qjl_project_query(const float* qjl, int32_t m, int32_t dim, const float* q,
                               float* pq, tqkv_stream stream);
/* estimate_inner_products (compressor.rs:122-159): stage 1 as tqkv_tq_scores
 * plus estimate_correction_from_projection (qjl.rs:86-118) of each key's
 * residual signs (u32 words [n, ceil(m/32)], bit i of a key = sign of row
 * i) and norm, bit-exact. Device. */
int32_t tqkv_tq_scores_two_stage(const float* rq, const float* pq, const uint8_t* codes,
                                 const float* sigma, const float* centroids_f32,
                                 const uint32_t* signs, const float* rnorm, int32_t dim,
                                 int32_t m, int64_t n, float* scores, tqkv_stream stream);
/* qjl_encode_stage2_packed (turboquant.rs:592-622): residual = K_rot - K_dq
 * (bf16 in, f32), r_norm = sqrt(sum r^2), sign bit i = (Phi[i] . r >= 0),
 * packed LSB-first into u32 [rows, ceil(m/32)]. Sums run in index order
 * from +0.0. Device. */
int32_t tqkv_qjl_encode_stage2(const uint16_t* k_rot, const uint16_t* k_dq, const float* qjl,
                               int64_t rows, int32_t dim, int32_t m, uint32_t* signs,
                               float* rnorm, tqkv_stream stream);
/* qjl_apply_correction_packed (turboquant.rs:624-691): K_eff = bf16(K_dq +
 * bf16((sum_i sign_i Phi[i][d]) * (r_norm * sqrt(pi/2) / sqrt(m)))), bf16
 * [rows, dim]. Device. */
int32_t tqkv_qjl_apply_correction(const uint16_t* k_dq, const uint32_t* signs,
                                  const float* rnorm, const float* qjl, int64_t rows, int32_t dim,
                                  int32_t m, uint16_t* k_eff, tqkv_stream stream);
/* lloyd_max_dequantize_scaled (turboquant.rs:428-439): out = bf16(centroids[c]
 * * sigma) for codes u8 [rows, dim] and sigma f32 [rows] (the TurboQuant
 * cache's codes and scales), centroids f32 [2^bits]. codes and out 16-byte
 * aligned; dim a multiple of 8. Device. */
int32_t tqkv_codebook_dequantize(const uint8_t* codes, const float* sigma,
                                 const float* centroids, int32_t bits, int64_t rows, int32_t dim,
                                 uint16_t* out, tqkv_stream stream);
/* SimpleCache::attend_values (simple.rs:40-62, 105-118): out = sum_t w_t *
 * R^T(centroid[c_t] * sigma_t), tokens with |w_t| < 1e-10 skipped, in the
 * reference's accumulation order. Device. */
int32_t tqkv_tq_values(const float* rotation, const uint8_t* codes, const float* sigma,
                       const float* centroids_f32, const float* weights, int32_t dim, int64_t n,
                       float* out, tqkv_stream stream);
/* bitpack::packed_words (bitpack.rs:9-14): u64 words a vector of `dim`
 * codes at `bits` (1..8) takes, 64 / bits codes a word; -1 for bits or dim
 * out of range. Host only. */
int64_t tqkv_packed_words(int32_t dim, int32_t bits);
/* bitpack::pack_codes (bitpack.rs:17-33) over n vectors: codes u8 [n, dim]
 * -> words u64 [n, tqkv_packed_words(dim, bits)], code j of a vector at
 * bits (j % (64 / bits)) * bits of word j / (64 / bits), unused high bits
 * zero. Device. */
int32_t tqkv_pack_codes(const uint8_t* codes, int64_t n, int32_t dim, int32_t bits,
                        uint64_t* words, tqkv_stream stream);
/* bitpack::unpack_codes (bitpack.rs:36-49), the inverse over n vectors.
 * Device. */
int32_t tqkv_unpack_codes(const uint64_t* words, int64_t n, int32_t dim, int32_t bits,
                          uint8_t* codes, tqkv_stream stream);
/* tqkv_tq_scores over codes in the packed layout, as
 * estimate_inner_products_stage1 reads CompressedVector::stage1_packed
 * (compressor.rs:165-184, simple.rs:50-56). Bit-identical to
 * tqkv_tq_scores on the unpacked codes. Device. */
int32_t tqkv_tq_scores_packed(const float* rq, const uint64_t* words, const float* sigma,
                              const float* centroids_f32, int32_t bits, int32_t dim, int64_t n,
                              float* scores, tqkv_stream stream);
/* tqkv_tq_values over codes in the packed layout (simple.rs:40-62).
 * Bit-identical to tqkv_tq_values on the unpacked codes. Device. */
int32_t tqkv_tq_values_packed(const float* rotation, const uint64_t* words, const float* sigma,
                              const float* centroids_f32, const float* weights, int32_t bits,
                              int32_t dim, int64_t n, float* out, tqkv_stream stream);
/* rotate_last_axis (turboquant.rs:258-267): y = x R (transpose = 0) or
 * y = x R^T (transpose = 1), bf16 rows [rows, dim] in and out, f32
 * accumulation. The affine+rotation cache mode (gemma4_moe.rs:4154-4173)
 * rotates keys and queries with it. Device. */
int32_t tqkv_rotate_bf16(const uint16_t* x, int64_t rows, int32_t dim, const float* rotation,
                         int32_t transpose, uint16_t* y, tqkv_stream stream);

/* ======================================================================
 * turboquant_cache::KVCache (traits.rs:9-36) as SimpleCache implements it
 * ====================================================================== */

/* TurboQuantConfig (lumen-core/src/config.rs:5-28); lloyd_max_iter 0 = 1000. */
typedef struct tqkv_tq_config {
  int32_t head_dim;
  int32_t bits;
  int32_t qjl_m;
  int32_t lloyd_max_iter;
  uint64_t seed;
} tqkv_tq_config;

typedef struct tqkv_kvcache tqkv_kvcache;

/*
 * SimpleCache::new(Arc<TurboQuantCompressor>, n_layers, n_kv_heads,
 * head_dim) (simple.rs:23-37) with TurboQuantCompressor::new(config)
 * (compressor.rs:20-32), or ::from_files (:35-58) when `rotation` (host
 * [head_dim, head_dim] row-major) and `qjl` (host [qjl_m, head_dim]) are
 * given; NULL draws them from the seed (R at seed, Phi at seed + 1).
 * head_dim in {64, 128, 256, 512}. Compressed vectors live on the device,
 * their codes packed as CompressedVector::stage1_packed packs them
 * (tqkv_pack_codes), with scale, QJL sign words and residual norm.
 */
int32_t tqkv_kvcache_create(const tqkv_tq_config* cfg, const float* rotation, const float* qjl,
                            int32_t n_layers, int32_t n_kv_heads, tqkv_kvcache** out);
int32_t tqkv_kvcache_destroy(tqkv_kvcache* cache);
/* KVCache::store: keys and values host f32 [n_tokens, head_dim], both
 * compressed (two-stage) and appended. Synchronous. Out-of-range layer or
 * head (a panic in the reference) is TQKV_EINVAL_ARG. */
int32_t tqkv_kvcache_store(tqkv_kvcache* cache, int32_t layer, int32_t head, const float* keys,
                           const float* values, int64_t n_tokens);
/* KVCache::attend_keys: stage-1 scores (host f32 [seq_len]) for a host f32
 * query [head_dim], bit-exact with the reference. */
int32_t tqkv_kvcache_attend_keys(tqkv_kvcache* cache, int32_t layer, int32_t head,
                                 const float* query, float* scores);
/* KVCache::attend_values: host weights [seq_len] -> host out [head_dim],
 * bit-exact with the reference. */
int32_t tqkv_kvcache_attend_values(tqkv_kvcache* cache, int32_t layer, int32_t head,
                                   const float* weights, float* out);
/* KVCache::seq_len (-1 for an out-of-range layer or head). */
int64_t tqkv_kvcache_seq_len(const tqkv_kvcache* cache, int32_t layer, int32_t head);
/* KVCache::clear. */
int32_t tqkv_kvcache_clear(tqkv_kvcache* cache);
/* KVCache::truncate: keep the first n_keep tokens of every head of a layer
 * (no-op where fewer are held). */
int32_t tqkv_kvcache_truncate(tqkv_kvcache* cache, int32_t layer, int64_t n_keep);
/* SimpleCache::memory_bytes (simple.rs:65-80): the sum of
 * CompressedVector::size_bytes (config.rs:50-55) over the stored vectors,
 * the reference's own accounting (its dim and bits fields and u64 sign
 * words included). tqkv_kvcache_device_bytes reports what the device
 * holds. */
int64_t tqkv_kvcache_memory_bytes(const tqkv_kvcache* cache);
/* Device bytes of the cache (no counterpart in the reference): *held = the
 * stored vectors' packed codes, scales, and with QJL their u32 sign words
 * and residual norms; *reserved = all device memory the cache owns (array
 * capacity, the R / Phi / codebook tables and its staging buffer). Either
 * pointer may be NULL. */
int32_t tqkv_kvcache_device_bytes(const tqkv_kvcache* cache, int64_t* held, int64_t* reserved);
/* The stored CompressedVector fields of vectors [first, first + n) of a
 * (layer, head) (which_values = 0 keys, 1 values), to host: codes u8 [n,
 * head_dim], scale [n], QJL sign words u32 [n, ceil(qjl_m / 32)] and
 * residual norms [n] (any pointer may be NULL). */
int32_t tqkv_kvcache_read(tqkv_kvcache* cache, int32_t layer, int32_t head,
                          int32_t which_values, int64_t first, int64_t n, uint8_t* codes,
                          float* scale, uint32_t* signs, float* residual_norm);

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

/*
 * An empty kernel of `workgroups` x 256 work-items: timed back to back, the
 * floor a launch costs on this GPU, which latency-bound steps (a decode of
 * a short context, one per layer) are measured beside.
 */
int32_t tqkv_empty_launch(int32_t workgroups, tqkv_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* TQKV_H */
