"""ctypes bindings to the CPU oracle (oracle/liboracle.so), the checker every
parity test compares against. Test infrastructure: nothing in the product
imports this module."""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "oracle", "liboracle.so")

_lib = None

P = ctypes.c_void_p
SZ = ctypes.c_size_t
I = ctypes.c_int
U32 = ctypes.c_uint32
U64 = ctypes.c_uint64
F = ctypes.c_float
L = ctypes.c_long


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
        _lib = ctypes.CDLL(LIB_PATH)
        sigs = {
            "oracle_golden_digest": (U64, [ctypes.c_char_p, ctypes.c_char_p, I, I, I, I]),
            "oracle_f32_to_bf16": (None, [P, SZ, P]),
            "oracle_codebook": (I, [U32, SZ, P, P, P]),
            "oracle_codebook_quantize": (I, [U32, P, SZ, P]),
            "oracle_rotation_random": (None, [I, U64, P]),
            "oracle_rotation_apply": (None, [P, I, P, P]),
            "oracle_rotation_apply_inverse": (None, [P, I, P, P]),
            "oracle_qjl_random": (None, [I, I, U64, P]),
            "oracle_packed_words": (SZ, [SZ, U32]),
            "oracle_pack_codes": (None, [P, SZ, U32, P]),
            "oracle_unpack_codes": (None, [P, SZ, U32, P]),
            "oracle_qjl_packed_len": (SZ, [SZ]),
            "oracle_qjl_project_and_pack": (None, [P, I, I, P, P]),
            "oracle_qjl_estimate": (F, [P, I, I, P, P, F]),
            "oracle_compressor_new": (P, [I, U32, I, P, P]),
            "oracle_compressor_free": (None, [P]),
            "oracle_compress": (None, [P, P, SZ, P, P, P, P]),
            "oracle_scores": (None, [P, P, SZ, P, P, P, P, I, P]),
            "oracle_attend_values": (None, [P, P, SZ, P, P, P, P, P]),
            "oracle_affine_quantize": (None, [P, SZ, I, I, I, P, P, P, I, I, I]),
            "oracle_affine_dequantize": (None, [P, P, P, SZ, I, I, I, P]),
            "oracle_affine_dequantize_two_roundings": (None, [P, P, P, SZ, I, I, I, P]),
            "oracle_affine_quantize_f32": (None, [P, SZ, I, I, I, P, P, P, I, I, I]),
            "oracle_affine_dequantize_f32": (None, [P, P, P, SZ, I, I, I, P]),
            "oracle_write_code": (None, [P, SZ, I, U32]),
            "oracle_read_code": (U32, [P, SZ, I]),
            "oracle_mask_allowed": (I, [SZ, SZ, L]),
            "oracle_attend_bf16": (None, [P, P, P, I, I, I, I, SZ, I, F, I, SZ, SZ, L, P, P, P]),
            "oracle_attend_affine": (None, [P, P, P, P, P, P, P, I, I, I, I, SZ, I, I, I, I, F, I,
                                            SZ, SZ, L, P, P, P, I]),
            "oracle_tq_encode_gpu_path": (None, [P, SZ, I, P, I, I, P, I, P, P]),
            "oracle_attend_affine_f32": (None, [P, P, P, P, P, P, P, I, I, I, I, SZ, SZ, I, I,
                                                I, I, F, I, SZ, SZ, L, I, I, P]),
            "oracle_attend_codebook": (None, [P, P, P, P, P, P, P, I, I, I, I, SZ, I, F, I, SZ,
                                              SZ, L, P, P, P]),
            "oracle_golden_tape": (ctypes.c_int64, [ctypes.c_char_p, ctypes.c_char_p, P,
                                                    ctypes.c_int64, P, ctypes.c_int64, P, P, P]),
            "oracle_page_digest_affine": (None, [P, P, P, SZ, SZ, I, I, I, SZ, SZ, P, P]),
            "oracle_page_bounds": (None, [P, P, P, I, I, I, I, SZ, SZ, P]),
            "oracle_sparse_keep_pages": (SZ, [SZ]),
            "oracle_select_pages": (None, [P, SZ, SZ, SZ, P]),
            "oracle_qjl_encode_stage2": (None, [P, P, P, SZ, I, I, P, P]),
            "oracle_qjl_apply_correction": (None, [P, P, P, P, SZ, I, I, P]),
            "oracle_attend_codebook_qjl": (None, [P, P, P, P, P, P, P, P, P, P, P, I, I, I, SZ,
                                                  I, I, F, P]),
            "oracle_fnv_num": (U64, [U64, U64]),
            "oracle_fnv_array": (U64, [U64, I, I, I, I, P]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


# ------------------------------------------------------------------ helpers
def bf16_from_f32(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16(ptr(x), x.size, ptr(out))
    return out


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def golden_digest(kind, plan, prealloc, round_mode=0, wmax0=1, clip_low=0):
    return lib().oracle_golden_digest(kind.encode(), plan.encode(), int(prealloc), round_mode,
                                      wmax0, clip_low)


FNV_OFFSET = 0xCBF29CE484222325


def golden_tape(kind, plan):
    """A golden plan's inputs: ([(op, n, at)], data bytes, max_size, keep);
    op 'U' = update of n rows with arrays at data[at:], 'R' = rewind to n."""
    ev = np.zeros(3 * 8192, np.int64)
    data = np.zeros(1 << 24, np.uint8)
    dl, mx, kp = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    n = lib().oracle_golden_tape(kind.encode(), plan.encode(), ptr(ev), 8192, ptr(data),
                                 data.size, ctypes.byref(dl), ctypes.byref(mx), ctypes.byref(kp))
    assert n >= 0
    events = [(chr(ev[3 * i]), int(ev[3 * i + 1]), int(ev[3 * i + 2])) for i in range(n)]
    return events, data[:dl.value].copy(), mx.value, kp.value


def fnv_num(h, n):
    return lib().oracle_fnv_num(h, n)


def fnv_array(h, dtype_code, arr):
    """arr: [1 or h, s, last] numpy array; dtype_code 1 u8, 2 u32, 3 f32, 4 bf16."""
    a = np.ascontiguousarray(arr)
    hh, s, last = a.shape[-3], a.shape[-2], a.shape[-1]
    return lib().oracle_fnv_array(h, dtype_code, hh, s, last, ptr(a))


def pack_codes(codes, bits):
    """bitpack::pack_codes (bitpack.rs:17-33): u8 codes -> u64 words."""
    c = np.ascontiguousarray(codes, np.uint8)
    out = np.zeros(lib().oracle_packed_words(c.size, bits), np.uint64)
    lib().oracle_pack_codes(ptr(c), c.size, bits, ptr(out))
    return out


def unpack_codes(packed, n, bits):
    """bitpack::unpack_codes (bitpack.rs:35-52): u64 words -> n u8 codes."""
    p = np.ascontiguousarray(packed, np.uint64)
    out = np.zeros(n, np.uint8)
    lib().oracle_unpack_codes(ptr(p), n, bits, ptr(out))
    return out


def codebook(bits, n_iter=1000):
    n = 1 << bits
    b = np.empty(n + 1, np.float64)
    c = np.empty(n, np.float64)
    mse = ctypes.c_double()
    rc = lib().oracle_codebook(bits, n_iter, ptr(b), ptr(c), ctypes.byref(mse))
    assert rc == 0
    return b, c, mse.value


def rotation(dim, seed):
    r = np.empty((dim, dim), np.float32)
    lib().oracle_rotation_random(dim, seed, ptr(r))
    return r


def qjl_matrix(dim, m, seed):
    p = np.empty((m, dim), np.float32)
    lib().oracle_qjl_random(dim, m, seed, ptr(p))
    return p


def affine_quantize(w_bf16, gs, bits, round_mode=0, wmax0=1, clip_low=0):
    w = np.ascontiguousarray(w_bf16, dtype=np.uint16)
    d = w.shape[-1]
    rows = w.size // d
    packed = np.zeros(w.shape[:-1] + (d * bits // 32,), np.uint32)
    scales = np.zeros(w.shape[:-1] + (d // gs,), np.uint16)
    biases = np.zeros_like(scales)
    lib().oracle_affine_quantize(ptr(w), rows, d, gs, bits, ptr(packed), ptr(scales),
                                 ptr(biases), round_mode, wmax0, clip_low)
    return packed, scales, biases


def affine_dequantize(packed, scales, biases, gs, bits, two_roundings=False):
    """mlx::dequantize to bf16: bf16(fma(scale, code, bias)), one rounding
    (what the reference's qwen4exp_tiny fixture records for MLX), or with
    two_roundings=True bf16(bf16(scale * code) + bias), the secondary
    reading."""
    d = packed.shape[-1] * 32 // bits
    rows = packed.size // packed.shape[-1]
    out = np.empty(packed.shape[:-1] + (d,), np.uint16)
    fn = lib().oracle_affine_dequantize_two_roundings if two_roundings \
        else lib().oracle_affine_dequantize
    fn(ptr(np.ascontiguousarray(packed)), ptr(np.ascontiguousarray(scales)),
       ptr(np.ascontiguousarray(biases)), rows, d, gs, bits, ptr(out))
    return out


def affine_quantize_f32(w, gs, bits, round_mode=0, wmax0=1, clip_low=0):
    """MLX's quantize of f32 rows: (packed u32, scales f32, biases f32)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    d = w.shape[-1]
    rows = w.size // d
    packed = np.zeros(w.shape[:-1] + (d * bits // 32,), np.uint32)
    scales = np.zeros(w.shape[:-1] + (d // gs,), np.float32)
    biases = np.zeros_like(scales)
    lib().oracle_affine_quantize_f32(ptr(w), rows, d, gs, bits, ptr(packed), ptr(scales),
                                     ptr(biases), round_mode, wmax0, clip_low)
    return packed, scales, biases


def affine_dequantize_f32(packed, scales, biases, gs, bits):
    """MLX's dequantize of an f32-scaled table: fmaf(scale, code, bias)."""
    d = packed.shape[-1] * 32 // bits
    rows = packed.size // packed.shape[-1]
    out = np.empty(packed.shape[:-1] + (d,), np.float32)
    lib().oracle_affine_dequantize_f32(ptr(np.ascontiguousarray(packed, np.uint32)),
                                       ptr(np.ascontiguousarray(scales, np.float32)),
                                       ptr(np.ascontiguousarray(biases, np.float32)), rows, d,
                                       gs, bits, ptr(out))
    return out


def write_code(words, i, bits, code):
    """offload/lowbit.rs write_code into a u32 array, in place."""
    assert words.dtype == np.uint32 and words.flags.c_contiguous
    lib().oracle_write_code(ptr(words), i, bits, code)


def read_code(words, i, bits):
    return int(lib().oracle_read_code(ptr(np.ascontiguousarray(words, np.uint32)), i, bits))


class Compressor:
    """TurboQuantCompressor over given R and Phi."""

    def __init__(self, dim, bits, m, R, phi):
        self.dim, self.bits, self.m = dim, bits, m
        self.R = np.ascontiguousarray(R, np.float32)
        self.phi = np.ascontiguousarray(phi, np.float32)
        self.h = lib().oracle_compressor_new(dim, bits, m, ptr(self.R), ptr(self.phi))
        assert self.h
        self.w1 = lib().oracle_packed_words(dim, bits)
        self.w2 = lib().oracle_qjl_packed_len(m)

    def __del__(self):
        if getattr(self, "h", None):
            lib().oracle_compressor_free(self.h)

    def compress(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, self.dim)
        n = x.shape[0]
        s1 = np.zeros((n, self.w1), np.uint64)
        s2 = np.zeros((n, self.w2), np.uint64)
        rn = np.zeros(n, np.float32)
        sc = np.zeros(n, np.float32)
        lib().oracle_compress(self.h, ptr(x), n, ptr(s1), ptr(s2), ptr(rn), ptr(sc))
        return s1, s2, rn, sc

    def scores(self, q, comp, two_stage=False):
        s1, s2, rn, sc = comp
        q = np.ascontiguousarray(q, np.float32)
        out = np.empty(s1.shape[0], np.float32)
        lib().oracle_scores(self.h, ptr(q), s1.shape[0], ptr(s1), ptr(s2), ptr(rn), ptr(sc),
                            int(two_stage), ptr(out))
        return out

    def attend_values(self, w, comp):
        s1, s2, rn, sc = comp
        w = np.ascontiguousarray(w, np.float32)
        out = np.empty(self.dim, np.float32)
        lib().oracle_attend_values(self.h, ptr(w), s1.shape[0], ptr(s1), ptr(s2), ptr(rn),
                                   ptr(sc), ptr(out))
        return out


def attend_bf16(q, K, V, scale, causal=False, q_start=0, first_held=0, window=-1):
    """q [B,H,L,D] bf16 bits; K,V [B,Hkv,N,D] bf16 bits."""
    B, H, Lq, D = q.shape
    Hkv, N = K.shape[1], K.shape[2]
    of = np.empty((B, H, Lq, D), np.float32)
    ob = np.empty((B, H, Lq, D), np.uint16)
    lse = np.empty((B, H, Lq), np.float32)
    lib().oracle_attend_bf16(ptr(np.ascontiguousarray(q)), ptr(np.ascontiguousarray(K)),
                             ptr(np.ascontiguousarray(V)), B, H, Hkv, Lq, N, D, scale,
                             int(causal), q_start, first_held, window, ptr(of), ptr(ob), ptr(lse))
    return of, ob, lse


def attend_affine(q, kt, vt, gs, bits_k, bits_v, scale, causal=False, q_start=0, first_held=0,
                  window=-1, dequant="f32"):
    """dequant="f32": exact scale * code + bias (the reference's decode paths);
    "bf16": mlx::dequantize to bf16 first (its prefill path), one rounding of
    the fused multiply-add; "bf16_2r": the same read as two bf16 roundings
    (the secondary reading)."""
    B, H, Lq, D = q.shape
    Hkv, N = kt[0].shape[1], kt[0].shape[2]
    of = np.empty((B, H, Lq, D), np.float32)
    ob = np.empty((B, H, Lq, D), np.uint16)
    lse = np.empty((B, H, Lq), np.float32)
    c = [np.ascontiguousarray(a) for a in (*kt, *vt)]
    lib().oracle_attend_affine(ptr(np.ascontiguousarray(q)), *[ptr(a) for a in c], B, H, Hkv, Lq,
                               N, D, gs, bits_k, bits_v, scale, int(causal), q_start, first_held,
                               window, ptr(of), ptr(ob), ptr(lse),
                               {"bf16": 0, "f32": 1, "bf16_2r": 2}[dequant])
    return of, ob, lse


def attend_affine_f32(q, kt, vt, n, gs, bits_k, bits_v, scale, threads=1, causal=False,
                      q_start=0, first_held=0, window=-1, dequant="f32"):
    """The CPU baseline (f32 dequantize-then-attend, bf16 out) over rows
    [0, n) of [B, H_kv, cap, .] triples; dequant "f32" (exact, the decode
    paths) or "bf16" (mlx::dequantize, the prefill path)."""
    B, H, Lq, D = q.shape
    Hkv, cap = kt[0].shape[1], kt[0].shape[2]
    out = np.empty((B, H, Lq, D), np.uint16)
    c = [np.ascontiguousarray(a) for a in (*kt, *vt)]
    lib().oracle_attend_affine_f32(ptr(np.ascontiguousarray(q)), *[ptr(a) for a in c], B, H, Hkv,
                                   Lq, cap, n, D, gs, bits_k, bits_v, scale, int(causal), q_start,
                                   first_held, window, int(dequant == "bf16"), threads, ptr(out))
    return out


# ------------------------------------------------------------- page-sparse
PAGE = 64


def page_digest_affine(kt, gs, bits, pages, max_pages=None):
    """kt: (packed, scales, biases) [B, H_kv, cap, .]; key_min / key_max
    bf16 [B, H_kv, max_pages, D] over pages [0, pages) (the rest zero)."""
    kw, ks, kb = (np.ascontiguousarray(a) for a in kt)
    B, Hkv, cap = kw.shape[:3]
    D = kw.shape[3] * 32 // bits
    mp = pages if max_pages is None else max_pages
    kmin = np.zeros((B, Hkv, mp, D), np.uint16)
    kmax = np.zeros((B, Hkv, mp, D), np.uint16)
    lib().oracle_page_digest_affine(ptr(kw), ptr(ks), ptr(kb), B * Hkv, cap, D, gs, bits, pages,
                                    mp, ptr(kmin), ptr(kmax))
    return kmin, kmax


def page_bounds(q, kmin, kmax, pages):
    """f64 [B, H_kv, pages] page bounds (unpinned)."""
    B, H, _, D = q.shape
    Hkv, mp = kmin.shape[1], kmin.shape[2]
    out = np.empty((B, Hkv, pages), np.float64)
    lib().oracle_page_bounds(ptr(np.ascontiguousarray(q)), ptr(np.ascontiguousarray(kmin)),
                             ptr(np.ascontiguousarray(kmax)), B, H, Hkv, D, pages, mp, ptr(out))
    return out


def sparse_keep_pages(pages):
    return int(lib().oracle_sparse_keep_pages(pages))


def select_pages(bounds, keep):
    B, Hkv, pages = bounds.shape
    out = np.empty((B, Hkv, keep), np.int32)
    lib().oracle_select_pages(ptr(np.ascontiguousarray(bounds)), B * Hkv, pages, keep, ptr(out))
    return out


def gather_pages(t, chosen, n):
    """Rows of the chosen pages of each (batch row, KV head), then the tail
    [pages * 64, n) (pages = the digested count): one array per input array."""
    B, Hkv, keep = chosen.shape
    out = []
    for a in t:
        rows = []
        for b in range(B):
            per = []
            for h in range(Hkv):
                idx = (chosen[b, h][:, None] * PAGE + np.arange(PAGE)[None, :]).reshape(-1)
                per.append(a[b, h, idx])
            rows.append(per)
        out.append(np.array(rows))
    return out


def attend_affine_pages(q, kt, vt, chosen, pages, n, gs, bits_k, bits_v, scale):
    """sdpa_page_sparse's attention over the chosen pages plus the tail
    [pages * 64, n), with the exact dequantization of the decode paths."""
    kg, vg = gather_pages(kt, chosen, n), gather_pages(vt, chosen, n)
    tail = lambda a: a[:, :, pages * PAGE:n]
    kc = tuple(np.concatenate([g, tail(a)], axis=2) for g, a in zip(kg, kt))
    vc = tuple(np.concatenate([g, tail(a)], axis=2) for g, a in zip(vg, vt))
    return attend_affine(q, kc, vc, gs, bits_k, bits_v, scale)


# ------------------------------------------------------- QJL (GPU path)
def tq_encode_gpu_path(x_bf16, inner, R=None, mode=0, transpose=False):
    """The GPU TurboQuant encode restated: (codes u8 [rows, D], sigma f32)."""
    x = np.ascontiguousarray(x_bf16, np.uint16)
    D = x.shape[-1]
    rows = x.size // D
    codes = np.zeros((rows, D), np.uint8)
    sigma = np.zeros(rows, np.float32)
    Rm = np.ascontiguousarray(R if R is not None else np.zeros((1,)), np.float32)
    inner = np.ascontiguousarray(inner, np.float32)
    lib().oracle_tq_encode_gpu_path(ptr(x), rows, D, ptr(Rm), mode, int(transpose), ptr(inner),
                                    inner.size, ptr(codes), ptr(sigma))
    return codes, sigma


def boundaries_inner(bits):
    """lloyd_max_boundaries_inner (turboquant.rs:310-331): the f64 inner
    boundaries of the codebook as f32."""
    b = codebook(bits)[0]
    return np.asarray(b[1:-1], np.float64).astype(np.float32)

def qjl_encode_stage2(k_rot, k_dq, phi, m):
    """turboquant.rs:592-622 restated: (signs u32 [rows, ceil(m/32)], r_norm)."""
    k_rot = np.ascontiguousarray(k_rot, np.uint16)
    D = k_rot.shape[-1]
    rows = k_rot.size // D
    signs = np.zeros((rows, (m + 31) // 32), np.uint32)
    rn = np.zeros(rows, np.float32)
    lib().oracle_qjl_encode_stage2(ptr(k_rot), ptr(np.ascontiguousarray(k_dq, np.uint16)),
                                   ptr(np.ascontiguousarray(phi, np.float32)), rows, D, m,
                                   ptr(signs), ptr(rn))
    return signs, rn


def qjl_apply_correction(k_dq, signs, rnorm, phi, m):
    """turboquant.rs:624-691 restated: K_eff bf16."""
    k_dq = np.ascontiguousarray(k_dq, np.uint16)
    D = k_dq.shape[-1]
    rows = k_dq.size // D
    out = np.zeros_like(k_dq)
    lib().oracle_qjl_apply_correction(ptr(k_dq), ptr(np.ascontiguousarray(signs, np.uint32)),
                                      ptr(np.ascontiguousarray(rnorm, np.float32)),
                                      ptr(np.ascontiguousarray(phi, np.float32)), rows, D, m,
                                      ptr(out))
    return out


def attend_codebook_qjl(q, kc, ks, ksg, krn, vc, vs, cent_k, cent_v, R, phi, m, scale):
    """Codebook attention with the two-stage (QJL-corrected) scores; f32
    [B, H, D] in the original basis."""
    B, H, _, D = q.shape
    Hkv, N = kc.shape[1], kc.shape[2]
    out = np.zeros((B, H, D), np.float32)
    c = lambda a, t: np.ascontiguousarray(a, t)
    lib().oracle_attend_codebook_qjl(ptr(c(q, np.uint16)), ptr(c(kc, np.uint8)), ptr(c(ks, np.float32)),
                                     ptr(c(ksg, np.uint32)), ptr(c(krn, np.float32)),
                                     ptr(c(vc, np.uint8)), ptr(c(vs, np.float32)),
                                     ptr(c(cent_k, np.float32)), ptr(c(cent_v, np.float32)),
                                     ptr(c(R, np.float32)), ptr(c(phi, np.float32)), B, H, Hkv, N,
                                     D, m, scale, ptr(out))
    return out
