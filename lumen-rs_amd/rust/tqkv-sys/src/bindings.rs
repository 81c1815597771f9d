// Generated from include/tqkv.h by gen_bindings.py; do not edit.
#![allow(non_camel_case_types, non_snake_case, dead_code)]

use core::ffi::{c_char, c_void};

/// hipStream_t: the HIP stream work is queued on (null: the default stream).
pub type tqkv_stream = *mut c_void;

pub const TQKV_OK: i32 = 0;
pub const TQKV_EINVAL_SHAPE: i32 = 1;
pub const TQKV_EINVAL_TARGET: i32 = 2;
pub const TQKV_EUNSUPPORTED: i32 = 3;
pub const TQKV_EDEVICE: i32 = 4;
pub const TQKV_ENOMEM: i32 = 5;
pub const TQKV_EINVAL_ARG: i32 = 6;
pub const TQKV_ECORRUPT: i32 = 7;
pub const TQKV_ABI_VERSION: i32 = 200;
pub const TQKV_NOALLOC_SCRATCH_BYTES: i32 = 33554432;
pub const TQKV_CACHE_BF16: i32 = 0;
pub const TQKV_CACHE_AFFINE: i32 = 1;
pub const TQKV_CACHE_CODEBOOK: i32 = 2;

#[repr(C)]
pub struct tqkv_cache {
    _private: [u8; 0],
}

#[repr(C)]
pub struct tqkv_kvcache {
    _private: [u8; 0],
}

#[repr(C)]
#[derive(Debug, Copy, Clone)]
pub struct tqkv_affine_seg {
    pub k_packed: *const u32,
    pub k_scales: *const u16,
    pub k_biases: *const u16,
    pub v_packed: *const u32,
    pub v_scales: *const u16,
    pub v_biases: *const u16,
    pub cap: i64,
    pub n: i64,
    pub shared: i32,
    pub reserved: i32,
}

#[repr(C)]
#[derive(Debug, Copy, Clone)]
pub struct tqkv_cache_config {
    pub kind: i32,
    pub batch: i32,
    pub kv_heads: i32,
    pub k_dim: i32,
    pub v_dim: i32,
    pub group_size: i32,
    pub bits_k: i32,
    pub bits_v: i32,
    pub qjl_words: i32,
    pub prealloc: i32,
    pub max_size: i64,
    pub keep: i64,
    pub seed: u64,
    pub encode: i32,
    pub reserved: i32,
}

#[repr(C)]
#[derive(Debug, Copy, Clone)]
pub struct tqkv_cache_view {
    pub n: i64,
    pub cap: i64,
    pub n_slots: i32,
    pub reserved: i32,
    pub slot: [*mut c_void; 6],
    pub row_bytes: [i64; 6],
}

#[repr(C)]
#[derive(Debug, Copy, Clone)]
pub struct tqkv_cache_state {
    pub offset: i64,
    pub idx: i64,
    pub cached_len: i64,
    pub base_offset: i64,
    pub view: i64,
    pub empty: i32,
    pub n_slots: i32,
}

#[repr(C)]
#[derive(Debug, Copy, Clone)]
pub struct tqkv_lkv_info {
    pub model_fingerprint: *const c_char,
    pub created_at_unix: u64,
    pub position: u64,
    pub prefix_tokens: *const u32,
    pub n_prefix_tokens: i64,
    pub has_last_token: i32,
    pub last_token: u32,
    pub is_deep: i32,
}

#[repr(C)]
#[derive(Debug, Copy, Clone)]
pub struct tqkv_tq_config {
    pub head_dim: i32,
    pub bits: i32,
    pub qjl_m: i32,
    pub lloyd_max_iter: i32,
    pub seed: u64,
}

extern "C" {
    pub fn tqkv_status_string(status: i32) -> *const c_char;
    pub fn tqkv_last_error() -> *const c_char;
    pub fn tqkv_version() -> i32;
    pub fn tqkv_scratch_release() -> i32;
    pub fn tqkv_scratch_bytes() -> usize;
    pub fn tqkv_affine_quantize(x: *const u16, n_slabs: i64, s: i64, dim: i32, group_size: i32, bits: i32, packed: *mut u32, scales: *mut u16, biases: *mut u16, dst_cap: i64, dst_start: i64, stream: tqkv_stream) -> i32;
    pub fn tqkv_affine_quantize_kv(k: *const u16, v: *const u16, n_slabs: i64, s: i64, dim: i32, group_size: i32, bits_k: i32, bits_v: i32, k_packed: *mut u32, k_scales: *mut u16, k_biases: *mut u16, v_packed: *mut u32, v_scales: *mut u16, v_biases: *mut u16, dst_cap: i64, dst_start: i64, stream: tqkv_stream) -> i32;
    pub fn tqkv_affine_quantize_rotated(x: *const u16, n_slabs: i64, s: i64, dim: i32, group_size: i32, bits: i32, rotation: *const f32, packed: *mut u32, scales: *mut u16, biases: *mut u16, dst_cap: i64, dst_start: i64, rotated: *mut u16, stream: tqkv_stream) -> i32;
    pub fn tqkv_affine_quantize_kv_rotated(k: *const u16, v: *const u16, n_slabs: i64, s: i64, dim: i32, group_size: i32, bits_k: i32, bits_v: i32, rotation: *const f32, k_packed: *mut u32, k_scales: *mut u16, k_biases: *mut u16, v_packed: *mut u32, v_scales: *mut u16, v_biases: *mut u16, dst_cap: i64, dst_start: i64, stream: tqkv_stream) -> i32;
    pub fn tqkv_affine_dequantize(packed: *const u32, scales: *const u16, biases: *const u16, rows: i64, dim: i32, group_size: i32, bits: i32, out: *mut u16, stream: tqkv_stream) -> i32;
    pub fn tqkv_decode_attend_affine(q: *const u16, B: i32, H: i32, H_kv: i32, D: i32, group_size: i32, bits_k: i32, bits_v: i32, scale: f32, segs: *const tqkv_affine_seg, n_segs: i32, out: *mut u16, workspace: *mut c_void, workspace_bytes: usize, stream: tqkv_stream) -> i32;
    pub fn tqkv_decode_attend_affine_noalloc(q: *const u16, B: i32, H: i32, H_kv: i32, D: i32, group_size: i32, bits_k: i32, bits_v: i32, scale: f32, segs: *const tqkv_affine_seg, n_segs: i32, out: *mut u16, stream: tqkv_stream) -> i32;
    pub fn tqkv_decode_attend_affine_append(q: *const u16, B: i32, H: i32, H_kv: i32, D: i32, group_size: i32, bits_k: i32, bits_v: i32, scale: f32, segs: *const tqkv_affine_seg, n_segs: i32, k: *const u16, v: *const u16, k_packed: *mut u32, k_scales: *mut u16, k_biases: *mut u16, v_packed: *mut u32, v_scales: *mut u16, v_biases: *mut u16, dst_cap: i64, dst_row: i64, out: *mut u16, workspace: *mut c_void, workspace_bytes: usize, stream: tqkv_stream) -> i32;
    pub fn tqkv_page_digest_affine(k_packed: *const u32, k_scales: *const u16, k_biases: *const u16, n_slabs: i64, cap: i64, dim: i32, group_size: i32, bits: i32, page_from: i64, page_to: i64, key_min: *mut u16, key_max: *mut u16, max_pages: i64, stream: tqkv_stream) -> i32;
    pub fn tqkv_sparse_keep_pages(pages: i64) -> i64;
    pub fn tqkv_page_select(q: *const u16, B: i32, H: i32, H_kv: i32, D: i32, key_min: *const u16, key_max: *const u16, max_pages: i64, pages: i64, keep: i32, chosen: *mut i32, workspace: *mut c_void, workspace_bytes: usize, stream: tqkv_stream) -> i32;
    pub fn tqkv_page_select_workspace_size(B: i32, H_kv: i32, pages: i64) -> usize;
    pub fn tqkv_decode_attend_affine_pages(q: *const u16, B: i32, H: i32, H_kv: i32, D: i32, group_size: i32, bits_k: i32, bits_v: i32, scale: f32, seg: *const tqkv_affine_seg, chosen: *const i32, keep: i32, pages: i64, out: *mut u16, workspace: *mut c_void, workspace_bytes: usize, stream: tqkv_stream) -> i32;
    pub fn tqkv_decode_attend_affine_sparse(q: *const u16, B: i32, H: i32, H_kv: i32, D: i32, group_size: i32, bits_k: i32, bits_v: i32, scale: f32, seg: *const tqkv_affine_seg, key_min: *const u16, key_max: *const u16, max_pages: i64, pages: i64, keep: i32, out: *mut u16, chosen_out: *mut i32, workspace: *mut c_void, workspace_bytes: usize, stream: tqkv_stream) -> i32;
    pub fn tqkv_sparse_workspace_size(B: i32, H: i32, H_kv: i32, D: i32, total_tokens: i64, keep: i32) -> usize;
    pub fn tqkv_decode_kernel_name(H: i32, H_kv: i32, D: i32, group_size: i32, bits_k: i32, bits_v: i32) -> *const c_char;
    pub fn tqkv_decode_kernel_for_rows(H: i32, H_kv: i32, D: i32, group_size: i32, bits_k: i32, bits_v: i32, max_rows: i64) -> *const c_char;
    pub fn tqkv_decode_attend_codebook(q: *const u16, B: i32, H: i32, H_kv: i32, D: i32, scale: f32, rotation: *const f32, centroids_k: *const f32, bits_k: i32, centroids_v: *const f32, bits_v: i32, k_codes: *const u8, k_sigma: *const f32, v_codes: *const u8, v_sigma: *const f32, cap: i64, n: i64, out: *mut u16, workspace: *mut c_void, workspace_bytes: usize, stream: tqkv_stream) -> i32;
    pub fn tqkv_decode_codebook_workspace_size(B: i32, H: i32, D: i32, total_tokens: i64) -> usize;
    pub fn tqkv_decode_attend_codebook_qjl(q: *const u16, B: i32, H: i32, H_kv: i32, D: i32, scale: f32, rotation: *const f32, centroids_k: *const f32, bits_k: i32, centroids_v: *const f32, bits_v: i32, k_codes: *const u8, k_sigma: *const f32, k_signs: *const u32, k_rnorm: *const f32, qjl: *const f32, qjl_m: i32, v_codes: *const u8, v_sigma: *const f32, cap: i64, n: i64, out: *mut u16, workspace: *mut c_void, workspace_bytes: usize, stream: tqkv_stream) -> i32;
    pub fn tqkv_prefill_attend_affine(q: *const u16, B: i32, H: i32, H_kv: i32, L: i32, D: i32, group_size: i32, bits_k: i32, bits_v: i32, scale: f32, segs: *const tqkv_affine_seg, n_segs: i32, q_start: i64, k_start: i64, causal: i32, window: i64, out: *mut u16, stream: tqkv_stream) -> i32;
    pub fn tqkv_prefill_attend_affine_ws(q: *const u16, B: i32, H: i32, H_kv: i32, L: i32, D: i32, group_size: i32, bits_k: i32, bits_v: i32, scale: f32, segs: *const tqkv_affine_seg, n_segs: i32, q_start: i64, k_start: i64, causal: i32, window: i64, out: *mut u16, workspace: *mut c_void, workspace_bytes: usize, stream: tqkv_stream) -> i32;
    pub fn tqkv_prefill_workspace_size(B: i32, H_kv: i32, D: i32, total_keys: i64) -> usize;
    pub fn tqkv_decode_workspace_size(B: i32, H: i32, H_kv: i32, D: i32, total_tokens: i64) -> usize;
    pub fn tqkv_cache_create(cfg: *const tqkv_cache_config, out: *mut *mut tqkv_cache) -> i32;
    pub fn tqkv_cache_destroy(cache: *mut tqkv_cache) -> i32;
    pub fn tqkv_cache_clone(src: *const tqkv_cache, out: *mut *mut tqkv_cache, stream: tqkv_stream) -> i32;
    pub fn tqkv_cache_update(cache: *mut tqkv_cache, rows: *const *const c_void, s: i64, fetched: *mut tqkv_cache_view, stream: tqkv_stream) -> i32;
    pub fn tqkv_cache_append(cache: *mut tqkv_cache, k: *const u16, v: *const u16, s: i64, fetched: *mut tqkv_cache_view, stream: tqkv_stream) -> i32;
    pub fn tqkv_cache_truncate(cache: *mut tqkv_cache, target: i64) -> i32;
    pub fn tqkv_cache_clear(cache: *mut tqkv_cache) -> i32;
    pub fn tqkv_cache_get_state(cache: *const tqkv_cache, out: *mut tqkv_cache_state) -> i32;
    pub fn tqkv_cache_buffers(cache: *const tqkv_cache, out: *mut tqkv_cache_view) -> i32;
    pub fn tqkv_cache_keep_suffix_from(cache: *mut tqkv_cache, prefix_len: i64, stream: tqkv_stream) -> i32;
    pub fn tqkv_cache_set_tables(cache: *mut tqkv_cache, rotation: *const f32, qjl: *const f32) -> i32;
    pub fn tqkv_cache_attach_prefix(cache: *mut tqkv_cache, prefix: *const tqkv_cache) -> i32;
    pub fn tqkv_cache_decode_attend(cache: *const tqkv_cache, q: *const u16, H: i32, scale: f32, out: *mut u16, workspace: *mut c_void, workspace_bytes: usize, stream: tqkv_stream) -> i32;
    pub fn tqkv_cache_append_decode(cache: *mut tqkv_cache, k: *const u16, v: *const u16, q: *const u16, H: i32, scale: f32, out: *mut u16, workspace: *mut c_void, workspace_bytes: usize, stream: tqkv_stream) -> i32;
    pub fn tqkv_cache_prefill_attend(cache: *const tqkv_cache, q: *const u16, H: i32, L: i32, scale: f32, window: i64, out: *mut u16, stream: tqkv_stream) -> i32;
    pub fn tqkv_lkv_export(layers: *const *const tqkv_cache, n_layers: i32, info: *const tqkv_lkv_info, out: *mut u8, capacity: usize, bytes: *mut usize, stream: tqkv_stream) -> i32;
    pub fn tqkv_lkv_check(data: *const u8, bytes: usize) -> i32;
    pub fn tqkv_lkv_manifest(data: *const u8, bytes: usize, json: *mut c_char, capacity: usize, json_bytes: *mut usize, n_layers: *mut i32, n_records: *mut i32) -> i32;
    pub fn tqkv_lkv_import(data: *const u8, bytes: usize, layer: i32, seed: u64, out: *mut *mut tqkv_cache, stream: tqkv_stream) -> i32;
    pub fn tqkv_lkv_rewrite(data: *const u8, bytes: usize, out: *mut u8, capacity: usize, out_bytes: *mut usize) -> i32;
    pub fn tqkv_crc32(data: *const c_void, bytes: usize, out: *mut u32) -> i32;
    pub fn tqkv_lloyd_max(bits: u32, n_iter: usize, boundaries: *mut f64, centroids: *mut f64) -> i32;
    pub fn tqkv_rotation_matrix(dim: i32, seed: u64, out: *mut f32) -> i32;
    pub fn tqkv_qjl_matrix(dim: i32, m: i32, seed: u64, out: *mut f32) -> i32;
    pub fn tqkv_tq_encode(x: *const c_void, x_is_bf16: i32, n_slabs: i64, s: i64, dim: i32, rotation: *const f32, boundaries: *const f64, centroids_f32: *const f32, bits: i32, qjl: *const f32, qjl_m: i32, codes: *mut u8, sigma: *mut f32, signs: *mut u32, rnorm: *mut f32, dst_cap: i64, dst_start: i64, stream: tqkv_stream) -> i32;
    pub fn tqkv_tq_encode_gpu_path(x: *const u16, n_slabs: i64, s: i64, dim: i32, rotation: *const f32, mode: i32, transpose: i32, boundaries_inner: *const f32, bits: i32, codes: *mut u8, sigma: *mut f32, dst_cap: i64, dst_start: i64, stream: tqkv_stream) -> i32;
    pub fn tqkv_tq_rotate_query(rotation: *const f32, q: *const f32, dim: i32, rq: *mut f32, stream: tqkv_stream) -> i32;
    pub fn tqkv_tq_scores(rq: *const f32, codes: *const u8, sigma: *const f32, centroids_f32: *const f32, dim: i32, n: i64, scores: *mut f32, stream: tqkv_stream) -> i32;
    pub fn tqkv_qjl_project_query(qjl: *const f32, m: i32, dim: i32, q: *const f32, pq: *mut f32, stream: tqkv_stream) -> i32;
    pub fn tqkv_tq_scores_two_stage(rq: *const f32, pq: *const f32, codes: *const u8, sigma: *const f32, centroids_f32: *const f32, signs: *const u32, rnorm: *const f32, dim: i32, m: i32, n: i64, scores: *mut f32, stream: tqkv_stream) -> i32;
    pub fn tqkv_qjl_encode_stage2(k_rot: *const u16, k_dq: *const u16, qjl: *const f32, rows: i64, dim: i32, m: i32, signs: *mut u32, rnorm: *mut f32, stream: tqkv_stream) -> i32;
    pub fn tqkv_qjl_apply_correction(k_dq: *const u16, signs: *const u32, rnorm: *const f32, qjl: *const f32, rows: i64, dim: i32, m: i32, k_eff: *mut u16, stream: tqkv_stream) -> i32;
    pub fn tqkv_codebook_dequantize(codes: *const u8, sigma: *const f32, centroids: *const f32, bits: i32, rows: i64, dim: i32, out: *mut u16, stream: tqkv_stream) -> i32;
    pub fn tqkv_tq_values(rotation: *const f32, codes: *const u8, sigma: *const f32, centroids_f32: *const f32, weights: *const f32, dim: i32, n: i64, out: *mut f32, stream: tqkv_stream) -> i32;
    pub fn tqkv_packed_words(dim: i32, bits: i32) -> i64;
    pub fn tqkv_pack_codes(codes: *const u8, n: i64, dim: i32, bits: i32, words: *mut u64, stream: tqkv_stream) -> i32;
    pub fn tqkv_unpack_codes(words: *const u64, n: i64, dim: i32, bits: i32, codes: *mut u8, stream: tqkv_stream) -> i32;
    pub fn tqkv_tq_scores_packed(rq: *const f32, words: *const u64, sigma: *const f32, centroids_f32: *const f32, bits: i32, dim: i32, n: i64, scores: *mut f32, stream: tqkv_stream) -> i32;
    pub fn tqkv_tq_values_packed(rotation: *const f32, words: *const u64, sigma: *const f32, centroids_f32: *const f32, weights: *const f32, bits: i32, dim: i32, n: i64, out: *mut f32, stream: tqkv_stream) -> i32;
    pub fn tqkv_rotate_bf16(x: *const u16, rows: i64, dim: i32, rotation: *const f32, transpose: i32, y: *mut u16, stream: tqkv_stream) -> i32;
    pub fn tqkv_kvcache_create(cfg: *const tqkv_tq_config, rotation: *const f32, qjl: *const f32, n_layers: i32, n_kv_heads: i32, out: *mut *mut tqkv_kvcache) -> i32;
    pub fn tqkv_kvcache_destroy(cache: *mut tqkv_kvcache) -> i32;
    pub fn tqkv_kvcache_store(cache: *mut tqkv_kvcache, layer: i32, head: i32, keys: *const f32, values: *const f32, n_tokens: i64) -> i32;
    pub fn tqkv_kvcache_attend_keys(cache: *mut tqkv_kvcache, layer: i32, head: i32, query: *const f32, scores: *mut f32) -> i32;
    pub fn tqkv_kvcache_attend_values(cache: *mut tqkv_kvcache, layer: i32, head: i32, weights: *const f32, out: *mut f32) -> i32;
    pub fn tqkv_kvcache_seq_len(cache: *const tqkv_kvcache, layer: i32, head: i32) -> i64;
    pub fn tqkv_kvcache_clear(cache: *mut tqkv_kvcache) -> i32;
    pub fn tqkv_kvcache_truncate(cache: *mut tqkv_kvcache, layer: i32, n_keep: i64) -> i32;
    pub fn tqkv_kvcache_memory_bytes(cache: *const tqkv_kvcache) -> i64;
    pub fn tqkv_kvcache_device_bytes(cache: *const tqkv_kvcache, held: *mut i64, reserved: *mut i64) -> i32;
    pub fn tqkv_kvcache_read(cache: *mut tqkv_kvcache, layer: i32, head: i32, which_values: i32, first: i64, n: i64, codes: *mut u8, scale: *mut f32, signs: *mut u32, residual_norm: *mut f32) -> i32;
    pub fn tqkv_synth_bf16(out: *mut u16, rows: i64, dim: i32, seed: u64, outlier_frac: f32, outlier_mult: f32, stream: tqkv_stream) -> i32;
    pub fn tqkv_read_probe(data: *const f32, bytes: usize, scratch: *mut f32, scratch_bytes: usize, out: *mut f32, stream: tqkv_stream) -> i32;
    pub fn tqkv_empty_launch(workgroups: i32, stream: tqkv_stream) -> i32;
}
