"""ctypes binding to libtqkv.so (the C ABI in include/tqkv.h) plus a minimal
HIP runtime helper for device buffers, streams and events.

Device memory comes from the same HIP runtime libtqkv.so links
(/opt/rocm/lib/libamdhip64.so), so no second runtime (such as the one bundled
with PyTorch wheels) is loaded into the process. The library fails loudly when
it is not built: there is no CPU fallback.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtqkv.so")
HIP_PATH = "/opt/rocm/lib/libamdhip64.so"

P = ctypes.c_void_p
SZ = ctypes.c_size_t
I32 = ctypes.c_int32
I64 = ctypes.c_int64
F32 = ctypes.c_float

OK = 0
EINVAL_SHAPE = 1
EINVAL_TARGET = 2
EUNSUPPORTED = 3
EDEVICE = 4
ENOMEM = 5
EINVAL_ARG = 6
ECORRUPT = 7


class TqkvError(RuntimeError):
    def __init__(self, status, detail):
        super().__init__(f"{status_name(status)}: {detail}")
        self.status = status


class AffineSeg(ctypes.Structure):
    _fields_ = [("k_packed", P), ("k_scales", P), ("k_biases", P),
                ("v_packed", P), ("v_scales", P), ("v_biases", P),
                ("cap", I64), ("n", I64), ("shared", I32), ("reserved", I32)]


class LkvInfo(ctypes.Structure):
    _fields_ = [("model_fingerprint", ctypes.c_char_p), ("created_at_unix", ctypes.c_uint64),
                ("position", ctypes.c_uint64), ("prefix_tokens", P), ("n_prefix_tokens", I64),
                ("has_last_token", I32), ("last_token", ctypes.c_uint32), ("is_deep", I32)]


class CacheConfig(ctypes.Structure):
    _fields_ = [("kind", I32), ("batch", I32), ("kv_heads", I32), ("k_dim", I32),
                ("v_dim", I32), ("group_size", I32), ("bits_k", I32), ("bits_v", I32),
                ("qjl_words", I32), ("prealloc", I32), ("max_size", I64), ("keep", I64),
                ("seed", ctypes.c_uint64), ("encode", I32), ("reserved", I32)]


class CacheView(ctypes.Structure):
    _fields_ = [("n", I64), ("cap", I64), ("n_slots", I32), ("reserved", I32),
                ("slot", P * 6), ("row_bytes", I64 * 6)]


class CacheState(ctypes.Structure):
    _fields_ = [("offset", I64), ("idx", I64), ("cached_len", I64), ("base_offset", I64),
                ("view", I64), ("empty", I32), ("n_slots", I32)]


CACHE_BF16, CACHE_AFFINE, CACHE_CODEBOOK = 0, 1, 2


class TqConfig(ctypes.Structure):
    _fields_ = [("head_dim", I32), ("bits", I32), ("qjl_m", I32), ("lloyd_max_iter", I32),
                ("seed", ctypes.c_uint64)]

_lib = None
_hip = None

_SIGS = {
    "tqkv_status_string": (ctypes.c_char_p, [I32]),
    "tqkv_last_error": (ctypes.c_char_p, []),
    "tqkv_version": (I32, []),
    "tqkv_affine_quantize": (I32, [P, I64, I64, I32, I32, I32, P, P, P, I64, I64, P]),
    "tqkv_affine_quantize_kv": (I32, [P, P, I64, I64, I32, I32, I32, I32, P, P, P, P, P, P, I64,
                                      I64, P]),
    "tqkv_affine_quantize_rotated": (I32, [P, I64, I64, I32, I32, I32, P, P, P, P, I64, I64, P,
                                           P]),
    "tqkv_affine_quantize_kv_rotated": (I32, [P, P, I64, I64, I32, I32, I32, I32, P, P, P, P, P,
                                              P, P, I64, I64, P]),
    "tqkv_affine_dequantize": (I32, [P, P, P, I64, I32, I32, I32, P, P]),
    "tqkv_prefill_attend_affine_ws": (I32, [P, I32, I32, I32, I32, I32, I32, I32, I32, F32, P, I32,
                                            I64, I64, I32, I64, P, P, SZ, P]),
    "tqkv_prefill_workspace_size": (SZ, [I32, I32, I32, I64]),
    "tqkv_scratch_release": (I32, []),
    "tqkv_scratch_bytes": (SZ, []),
    "tqkv_empty_launch": (I32, [I32, P]),
    "tqkv_decode_attend_affine": (I32, [P, I32, I32, I32, I32, I32, I32, I32, F32,
                                        ctypes.POINTER(AffineSeg), I32, P, P, SZ, P]),
    "tqkv_decode_attend_affine_noalloc": (I32, [P, I32, I32, I32, I32, I32, I32, I32, F32,
                                                ctypes.POINTER(AffineSeg), I32, P, P]),
    "tqkv_decode_attend_affine_append": (I32, [P, I32, I32, I32, I32, I32, I32, I32, F32,
                                               ctypes.POINTER(AffineSeg), I32, P, P, P, P, P,
                                               P, P, P, I64, I64, P, P, SZ, P]),
    "tqkv_prefill_attend_affine": (I32, [P, I32, I32, I32, I32, I32, I32, I32, I32, F32,
                                         ctypes.POINTER(AffineSeg), I32, I64, I64, I32, I64, P,
                                         P]),
    "tqkv_decode_workspace_size": (SZ, [I32, I32, I32, I32, I64]),
    "tqkv_decode_kernel_name": (ctypes.c_char_p, [I32, I32, I32, I32, I32, I32]),
    "tqkv_decode_kernel_for_rows": (ctypes.c_char_p, [I32, I32, I32, I32, I32, I32, I64]),
    "tqkv_page_digest_affine": (I32, [P, P, P, I64, I64, I32, I32, I32, I64, I64, P, P, I64, P]),
    "tqkv_sparse_keep_pages": (I64, [I64]),
    "tqkv_page_select": (I32, [P, I32, I32, I32, I32, P, P, I64, I64, I32, P, P, SZ, P]),
    "tqkv_page_select_workspace_size": (SZ, [I32, I32, I64]),
    "tqkv_decode_attend_affine_pages": (I32, [P, I32, I32, I32, I32, I32, I32, I32, F32, P, P,
                                              I32, I64, P, P, SZ, P]),
    "tqkv_decode_attend_affine_sparse": (I32, [P, I32, I32, I32, I32, I32, I32, I32, F32, P, P,
                                               P, I64, I64, I32, P, P, P, SZ, P]),
    "tqkv_sparse_workspace_size": (SZ, [I32, I32, I32, I32, I64, I32]),
    "tqkv_synth_bf16": (I32, [P, I64, I32, ctypes.c_uint64, F32, F32, P]),
    "tqkv_lloyd_max": (I32, [ctypes.c_uint32, SZ, P, P]),
    "tqkv_rotation_matrix": (I32, [I32, ctypes.c_uint64, P]),
    "tqkv_qjl_matrix": (I32, [I32, I32, ctypes.c_uint64, P]),
    "tqkv_tq_encode": (I32, [P, I32, I64, I64, I32, P, P, P, I32, P, I32, P, P, P, P, I64, I64,
                             P]),
    "tqkv_tq_rotate_query": (I32, [P, P, I32, P, P]),
    "tqkv_tq_encode_gpu_path": (I32, [P, I64, I64, I32, P, I32, I32, P, I32, P, P, I64, I64, P]),
    "tqkv_tq_scores": (I32, [P, P, P, P, I32, I64, P, P]),
    "tqkv_qjl_project_query": (I32, [P, I32, I32, P, P, P]),
    "tqkv_tq_scores_two_stage": (I32, [P, P, P, P, P, P, P, I32, I32, I64, P, P]),
    "tqkv_qjl_encode_stage2": (I32, [P, P, P, I64, I32, I32, P, P, P]),
    "tqkv_qjl_apply_correction": (I32, [P, P, P, P, I64, I32, I32, P, P]),
    "tqkv_decode_attend_codebook": (I32, [P, I32, I32, I32, I32, F32, P, P, I32, P, I32, P, P,
                                          P, P, I64, I64, P, P, SZ, P]),
    "tqkv_decode_codebook_workspace_size": (SZ, [I32, I32, I32, I64]),
    "tqkv_decode_attend_codebook_qjl": (I32, [P, I32, I32, I32, I32, F32, P, P, I32, P, I32, P, P,
                                              P, P, P, I32, P, P, I64, I64, P, P, SZ, P]),
    "tqkv_tq_values": (I32, [P, P, P, P, P, I32, I64, P, P]),
    "tqkv_packed_words": (I64, [I32, I32]),
    "tqkv_pack_codes": (I32, [P, I64, I32, I32, P, P]),
    "tqkv_unpack_codes": (I32, [P, I64, I32, I32, P, P]),
    "tqkv_tq_scores_packed": (I32, [P, P, P, P, I32, I32, I64, P, P]),
    "tqkv_tq_values_packed": (I32, [P, P, P, P, P, I32, I32, I64, P, P]),
    "tqkv_codebook_dequantize": (I32, [P, P, P, I32, I64, I32, P, P]),
    "tqkv_rotate_bf16": (I32, [P, I64, I32, P, I32, P, P]),
    "tqkv_kvcache_create": (I32, [ctypes.POINTER(TqConfig), P, P, I32, I32, ctypes.POINTER(P)]),
    "tqkv_kvcache_destroy": (I32, [P]),
    "tqkv_kvcache_store": (I32, [P, I32, I32, P, P, I64]),
    "tqkv_kvcache_attend_keys": (I32, [P, I32, I32, P, P]),
    "tqkv_kvcache_attend_values": (I32, [P, I32, I32, P, P]),
    "tqkv_kvcache_seq_len": (I64, [P, I32, I32]),
    "tqkv_kvcache_clear": (I32, [P]),
    "tqkv_kvcache_truncate": (I32, [P, I32, I64]),
    "tqkv_kvcache_memory_bytes": (I64, [P]),
    "tqkv_kvcache_device_bytes": (I32, [P, ctypes.POINTER(I64), ctypes.POINTER(I64)]),
    "tqkv_kvcache_read": (I32, [P, I32, I32, I32, I64, I64, P, P, P, P]),
    "tqkv_cache_create": (I32, [ctypes.POINTER(CacheConfig), ctypes.POINTER(P)]),
    "tqkv_cache_destroy": (I32, [P]),
    "tqkv_cache_clone": (I32, [P, ctypes.POINTER(P), P]),
    "tqkv_cache_update": (I32, [P, ctypes.POINTER(P), I64, ctypes.POINTER(CacheView), P]),
    "tqkv_cache_append": (I32, [P, P, P, I64, ctypes.POINTER(CacheView), P]),
    "tqkv_cache_truncate": (I32, [P, I64]),
    "tqkv_cache_clear": (I32, [P]),
    "tqkv_cache_get_state": (I32, [P, ctypes.POINTER(CacheState)]),
    "tqkv_cache_buffers": (I32, [P, ctypes.POINTER(CacheView)]),
    "tqkv_cache_keep_suffix_from": (I32, [P, I64, P]),
    "tqkv_cache_attach_prefix": (I32, [P, P]),
    "tqkv_cache_set_tables": (I32, [P, P, P]),
    "tqkv_cache_decode_attend": (I32, [P, P, I32, F32, P, P, SZ, P]),
    "tqkv_cache_append_decode": (I32, [P, P, P, P, I32, F32, P, P, SZ, P]),
    "tqkv_cache_prefill_attend": (I32, [P, P, I32, I32, F32, I64, P, P]),
    "tqkv_read_probe": (I32, [P, SZ, P, SZ, P, P]),
    "tqkv_lkv_export": (I32, [P, I32, ctypes.POINTER(LkvInfo), P, SZ, ctypes.POINTER(SZ), P]),
    "tqkv_lkv_check": (I32, [P, SZ]),
    "tqkv_lkv_manifest": (I32, [P, SZ, P, SZ, ctypes.POINTER(SZ), ctypes.POINTER(I32),
                                ctypes.POINTER(I32)]),
    "tqkv_lkv_import": (I32, [P, SZ, I32, ctypes.c_uint64, ctypes.POINTER(P), P]),
    "tqkv_crc32": (I32, [P, SZ, ctypes.POINTER(ctypes.c_uint32)]),
    "tqkv_lkv_rewrite": (I32, [P, SZ, P, SZ, ctypes.POINTER(SZ)]),
}


def lib():
    """Load libtqkv.so; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `make -C lumen-rs_amd` "
                               "or __graft_entry__.build()")
        hip()  # the runtime first, from /opt/rocm
        _lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(_lib, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
    return _lib


def exported_symbols():
    """Names libtqkv.so exports (dlsym succeeds), for the ABI check."""
    out = []
    for name in _SIGS:
        try:
            getattr(lib(), name)
            out.append(name)
        except AttributeError:
            pass
    return out


def status_name(status):
    return lib().tqkv_status_string(status).decode()


def check(status):
    if status != OK:
        raise TqkvError(status, lib().tqkv_last_error().decode())
    return status


# ---------------------------------------------------------------- HIP runtime
class Hip:
    """The few HIP runtime calls the tests and the bench need."""

    H2D, D2H, D2D = 1, 2, 3

    def __init__(self):
        self.h = ctypes.CDLL(HIP_PATH, mode=ctypes.RTLD_GLOBAL)
        sig = {
            "hipMalloc": [ctypes.POINTER(P), SZ],
            "hipFree": [P],
            "hipMemcpy": [P, P, SZ, I32],
            "hipMemcpyAsync": [P, P, SZ, I32, P],
            "hipMemsetAsync": [P, I32, SZ, P],
            "hipDeviceSynchronize": [],
            "hipStreamCreate": [ctypes.POINTER(P)],
            "hipStreamDestroy": [P],
            "hipStreamSynchronize": [P],
            "hipEventCreate": [ctypes.POINTER(P)],
            "hipEventDestroy": [P],
            "hipEventRecord": [P, P],
            "hipEventSynchronize": [P],
            "hipEventElapsedTime": [ctypes.POINTER(F32), P, P],
            "hipGetDeviceCount": [ctypes.POINTER(I32)],
            "hipGetErrorString": [I32],
            "hipSetDevice": [I32],
        }
        for name, args in sig.items():
            fn = getattr(self.h, name)
            fn.argtypes = args
            fn.restype = ctypes.c_char_p if name == "hipGetErrorString" else I32

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {self.h.hipGetErrorString(rc).decode()}")

    def device_count(self):
        n = I32(0)
        rc = self.h.hipGetDeviceCount(ctypes.byref(n))
        return n.value if rc == 0 else 0

    def malloc(self, nbytes):
        p = P()
        self._ok(self.h.hipMalloc(ctypes.byref(p), max(int(nbytes), 1)), "hipMalloc")
        return p.value

    def free(self, p):
        if p:
            self._ok(self.h.hipFree(p), "hipFree")

    def sync(self):
        self._ok(self.h.hipDeviceSynchronize(), "hipDeviceSynchronize")

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.malloc(arr.nbytes)
        self._ok(self.h.hipMemcpy(p, arr.ctypes.data, arr.nbytes, self.H2D), "hipMemcpy H2D")
        return p

    def copy_in(self, dst, arr):
        arr = np.ascontiguousarray(arr)
        self._ok(self.h.hipMemcpy(dst, arr.ctypes.data, arr.nbytes, self.H2D), "hipMemcpy H2D")

    def download(self, p, shape, dtype):
        out = np.empty(shape, dtype)
        self._ok(self.h.hipMemcpy(out.ctypes.data, p, out.nbytes, self.D2H), "hipMemcpy D2H")
        return out

    def stream(self):
        s = P()
        self._ok(self.h.hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        return s.value

    def event(self):
        e = P()
        self._ok(self.h.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e.value

    def record(self, ev, stream=None):
        self._ok(self.h.hipEventRecord(ev, stream), "hipEventRecord")

    def elapsed_ms(self, a, b):
        self._ok(self.h.hipEventSynchronize(b), "hipEventSynchronize")
        ms = F32(0)
        self._ok(self.h.hipEventElapsedTime(ctypes.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value


def hip():
    global _hip
    if _hip is None:
        _hip = Hip()
    return _hip


class DeviceArray:
    """A device buffer with a numpy shape and dtype; freed on delete."""

    def __init__(self, shape, dtype, data=None):
        self.shape = tuple(shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = hip().malloc(self.nbytes)
        if data is not None:
            data = np.ascontiguousarray(data, dtype=self.dtype)
            assert data.shape == self.shape, (data.shape, self.shape)
            hip().copy_in(self.ptr, data)

    @classmethod
    def of(cls, arr):
        arr = np.ascontiguousarray(arr)
        return cls(arr.shape, arr.dtype, arr)

    def numpy(self):
        return hip().download(self.ptr, self.shape, self.dtype)

    def __del__(self):
        try:
            if self.ptr and _hip is not None:
                _hip.free(self.ptr)
        except Exception:
            pass
        self.ptr = None


# ---------------------------------------------------------------- wrappers
def affine_quantize(x, n_slabs, s, dim, gs, bits, packed, scales, biases, dst_cap=None,
                    dst_start=0, stream=None):
    """x, packed, scales, biases: device pointers."""
    check(lib().tqkv_affine_quantize(x, n_slabs, s, dim, gs, bits, packed, scales, biases,
                                     s if dst_cap is None else dst_cap, dst_start, stream))


def affine_quantize_kv(k, v, n_slabs, s, dim, gs, bits_k, bits_v, kt, vt, dst_cap=None,
                       dst_start=0, stream=None):
    """K and V in one launch; kt, vt: (packed, scales, biases) device
    pointers of each."""
    check(lib().tqkv_affine_quantize_kv(k, v, n_slabs, s, dim, gs, bits_k, bits_v, *kt, *vt,
                                        s if dst_cap is None else dst_cap, dst_start, stream))


def affine_quantize_rotated(x, n_slabs, s, dim, gs, bits, R, packed, scales, biases,
                            dst_cap=None, dst_start=0, rotated=None, stream=None):
    """bf16(x R) quantized in one pass; `rotated` (optional) receives the
    rotated bf16 rows. Device pointers."""
    check(lib().tqkv_affine_quantize_rotated(x, n_slabs, s, dim, gs, bits, R, packed, scales,
                                             biases, s if dst_cap is None else dst_cap,
                                             dst_start, rotated, stream))


def affine_quantize_kv_rotated(k, v, n_slabs, s, dim, gs, bits_k, bits_v, R, kt, vt,
                               dst_cap=None, dst_start=0, stream=None):
    """K rotated by R and quantized, V quantized as it is, in one launch."""
    check(lib().tqkv_affine_quantize_kv_rotated(k, v, n_slabs, s, dim, gs, bits_k, bits_v, R,
                                                *kt, *vt, s if dst_cap is None else dst_cap,
                                                dst_start, stream))


def affine_dequantize(packed, scales, biases, rows, dim, gs, bits, out, stream=None):
    check(lib().tqkv_affine_dequantize(packed, scales, biases, rows, dim, gs, bits, out, stream))


def affine_seg(k_triple, v_triple, cap, n, shared=False):
    """k_triple / v_triple: (packed, scales, biases) device pointers."""
    return AffineSeg(k_triple[0], k_triple[1], k_triple[2], v_triple[0], v_triple[1],
                     v_triple[2], cap, n, int(shared), 0)


def decode_attend_affine(q, B, H, H_kv, D, gs, bits_k, bits_v, scale, segs, out,
                         workspace=None, workspace_bytes=0, stream=None):
    arr = (AffineSeg * len(segs))(*segs)
    check(lib().tqkv_decode_attend_affine(q, B, H, H_kv, D, gs, bits_k, bits_v, scale, arr,
                                          len(segs), out, workspace, workspace_bytes, stream))


def decode_attend_affine_noalloc(q, B, H, H_kv, D, gs, bits_k, bits_v, scale, segs, out,
                                 stream=None):
    """tqkv_decode_attend_affine with its split partials in the library's
    static device scratch (no allocation)."""
    arr = (AffineSeg * len(segs))(*segs)
    check(lib().tqkv_decode_attend_affine_noalloc(q, B, H, H_kv, D, gs, bits_k, bits_v, scale,
                                                  arr, len(segs), out, stream))


def decode_attend_affine_append(q, B, H, H_kv, D, gs, bits_k, bits_v, scale, segs, k, v, dst,
                                dst_cap, dst_row, out, workspace=None, workspace_bytes=0,
                                stream=None):
    """Quantize the new rows k, v into dst (six device pointers: K packed,
    scales, biases, V packed, scales, biases) at row dst_row of every slab
    and attend over segs plus that row, in one kernel."""
    arr = (AffineSeg * max(len(segs), 1))(*segs)
    check(lib().tqkv_decode_attend_affine_append(q, B, H, H_kv, D, gs, bits_k, bits_v, scale,
                                                 arr, len(segs), k, v, *dst, dst_cap, dst_row,
                                                 out, workspace, workspace_bytes, stream))


def prefill_attend_affine(q, B, H, H_kv, L, D, gs, bits_k, bits_v, scale, segs, out,
                          q_start=0, k_start=0, causal=True, window=-1, stream=None):
    """Chunk attention: query row l at q_start + l, key k at k_start + k."""
    arr = (AffineSeg * len(segs))(*segs)
    check(lib().tqkv_prefill_attend_affine(q, B, H, H_kv, L, D, gs, bits_k, bits_v, scale, arr,
                                           len(segs), q_start, k_start, int(causal), window, out,
                                           stream))


def prefill_attend_affine_ws(q, B, H, H_kv, L, D, gs, bits_k, bits_v, scale, segs, out,
                             workspace, workspace_bytes, q_start=0, k_start=0, causal=True,
                             window=-1, stream=None):
    """prefill_attend_affine with a caller workspace (None: dequantize in
    every block)."""
    arr = (AffineSeg * len(segs))(*segs)
    check(lib().tqkv_prefill_attend_affine_ws(q, B, H, H_kv, L, D, gs, bits_k, bits_v, scale, arr,
                                              len(segs), q_start, k_start, int(causal), window,
                                              out, workspace, workspace_bytes, stream))


def prefill_workspace_size(B, H_kv, D, total_keys):
    return lib().tqkv_prefill_workspace_size(B, H_kv, D, total_keys)


def scratch_release():
    check(lib().tqkv_scratch_release())


def scratch_bytes():
    """Bytes of per-device scratch the library holds (tqkv_scratch_bytes)."""
    return int(lib().tqkv_scratch_bytes())


def empty_launch(workgroups=256, stream=None):
    check(lib().tqkv_empty_launch(workgroups, stream))


def decode_kernel_name(H, H_kv, D, gs, bits_k, bits_v):
    """"mfma", "dot2" or "" (unsupported) for a decode layout."""
    return lib().tqkv_decode_kernel_name(H, H_kv, D, gs, bits_k, bits_v).decode()


def decode_kernel_for_rows(H, H_kv, D, gs, bits_k, bits_v, max_rows):
    """The decode kernel for a context whose longest segment holds max_rows."""
    return lib().tqkv_decode_kernel_for_rows(H, H_kv, D, gs, bits_k, bits_v, max_rows).decode()


def page_digest_affine(kt, n_slabs, cap, dim, gs, bits, page_from, page_to, key_min, key_max,
                       max_pages, stream=None):
    """kt: (packed, scales, biases) device pointers of a K buffer."""
    check(lib().tqkv_page_digest_affine(*kt, n_slabs, cap, dim, gs, bits, page_from, page_to,
                                        key_min, key_max, max_pages, stream))


def sparse_keep_pages(pages):
    return lib().tqkv_sparse_keep_pages(pages)


def page_select(q, B, H, H_kv, D, key_min, key_max, max_pages, pages, keep, chosen, workspace,
                workspace_bytes, stream=None):
    check(lib().tqkv_page_select(q, B, H, H_kv, D, key_min, key_max, max_pages, pages, keep,
                                 chosen, workspace, workspace_bytes, stream))


def page_select_workspace_size(B, H_kv, pages):
    return lib().tqkv_page_select_workspace_size(B, H_kv, pages)


def decode_attend_affine_pages(q, B, H, H_kv, D, gs, bits_k, bits_v, scale, seg, chosen, keep,
                               pages, out, workspace=None, workspace_bytes=0, stream=None):
    check(lib().tqkv_decode_attend_affine_pages(q, B, H, H_kv, D, gs, bits_k, bits_v, scale,
                                                ctypes.byref(seg), chosen, keep, pages, out,
                                                workspace, workspace_bytes, stream))


def decode_attend_affine_sparse(q, B, H, H_kv, D, gs, bits_k, bits_v, scale, seg, key_min,
                                key_max, max_pages, pages, keep, out, workspace, workspace_bytes,
                                chosen_out=None, stream=None):
    check(lib().tqkv_decode_attend_affine_sparse(q, B, H, H_kv, D, gs, bits_k, bits_v, scale,
                                                 ctypes.byref(seg), key_min, key_max, max_pages,
                                                 pages, keep, out, chosen_out, workspace,
                                                 workspace_bytes, stream))


def sparse_workspace_size(B, H, H_kv, D, total, keep):
    return lib().tqkv_sparse_workspace_size(B, H, H_kv, D, total, keep)


def tq_rotate_query(rotation, q, dim, rq, stream=None):
    check(lib().tqkv_tq_rotate_query(rotation, q, dim, rq, stream))


def qjl_project_query(qjl, m, dim, q, pq, stream=None):
    check(lib().tqkv_qjl_project_query(qjl, m, dim, q, pq, stream))


def tq_scores_two_stage(rq, pq, codes, sigma, centroids, signs, rnorm, dim, m, n, scores,
                        stream=None):
    check(lib().tqkv_tq_scores_two_stage(rq, pq, codes, sigma, centroids, signs, rnorm, dim, m,
                                         n, scores, stream))


def qjl_encode_stage2(k_rot, k_dq, qjl, rows, dim, m, signs, rnorm, stream=None):
    check(lib().tqkv_qjl_encode_stage2(k_rot, k_dq, qjl, rows, dim, m, signs, rnorm, stream))


def qjl_apply_correction(k_dq, signs, rnorm, qjl, rows, dim, m, k_eff, stream=None):
    check(lib().tqkv_qjl_apply_correction(k_dq, signs, rnorm, qjl, rows, dim, m, k_eff, stream))


def decode_workspace_size(B, H, H_kv, D, total):
    return lib().tqkv_decode_workspace_size(B, H, H_kv, D, total)


def synth_bf16(out, rows, dim, seed, outlier_frac=0.0, outlier_mult=1.0, stream=None):
    check(lib().tqkv_synth_bf16(out, rows, dim, seed, outlier_frac, outlier_mult, stream))


def read_probe(data, nbytes, scratch, scratch_bytes, out, stream=None):
    check(lib().tqkv_read_probe(data, nbytes, scratch, scratch_bytes, out, stream))


def measure_read_bandwidth(stream=None, nbytes=1 << 30, warmup=3, passes=15):
    """bandwidth.rs:73-100 on this GPU: median and best GB/s of summing a
    1 GiB random float array (3 warm-up passes, 15 timed, HIP events)."""
    h = hip()
    buf = DeviceArray((nbytes // 2,), np.uint16)
    synth_bf16(buf.ptr, nbytes // 2 // 256, 256, 12345, 0.0, 1.0, stream)
    scratch = DeviceArray((4096,), np.float32)
    out = DeviceArray((1,), np.float32)
    a, b = h.event(), h.event()
    rates = []
    for i in range(warmup + passes):
        h.record(a, stream)
        read_probe(buf.ptr, nbytes, scratch.ptr, 4096 * 4, out.ptr, stream)
        h.record(b, stream)
        ms = h.elapsed_ms(a, b)
        if i >= warmup:
            rates.append(nbytes / (ms * 1e-3) / 1e9)
    rates.sort()
    mid = len(rates) // 2
    median = rates[mid] if len(rates) % 2 else 0.5 * (rates[mid - 1] + rates[mid])
    return {"median_gbps": round(median, 1), "best_gbps": round(rates[-1], 1),
            "bytes": nbytes, "passes": passes}


# ---------------------------------------------------------------- the cache object
class Cache:
    """The device KV cache (tqkv_cache_*): growing, rotating or shared-prefix,
    bf16 / affine / codebook slots."""

    def __init__(self, kind, batch, kv_heads, k_dim, v_dim, group_size=64, bits_k=4, bits_v=4,
                 qjl_words=0, prealloc=True, max_size=0, keep=0, seed=42, encode=0):
        self.cfg = CacheConfig(kind, batch, kv_heads, k_dim, v_dim, group_size, bits_k, bits_v,
                               qjl_words, int(prealloc), max_size, keep, seed, encode, 0)
        h = P()
        check(lib().tqkv_cache_create(ctypes.byref(self.cfg), ctypes.byref(h)))
        self.h = h.value

    @classmethod
    def adopt(cls, handle):
        """Wrap a cache made by the library (tqkv_lkv_import)."""
        c = cls.__new__(cls)
        c.cfg = None
        c.h = handle
        return c

    def clone(self, stream=None):
        """An independent deep copy (tqkv_cache_clone)."""
        h = P()
        check(lib().tqkv_cache_clone(self.h, ctypes.byref(h), stream))
        c = Cache.adopt(h.value)
        c.cfg = self.cfg
        return c

    def close(self):
        if self.h:
            lib().tqkv_cache_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def update(self, rows, s, stream=None):
        """rows: device pointers, one per slot ([B, H_kv, s, row])."""
        arr = (P * len(rows))(*rows)
        v = CacheView()
        check(lib().tqkv_cache_update(self.h, arr, s, ctypes.byref(v), stream))
        return v

    def append(self, k, v, s, stream=None):
        view = CacheView()
        check(lib().tqkv_cache_append(self.h, k, v, s, ctypes.byref(view), stream))
        return view

    def truncate(self, target):
        """True if accepted, False where the reference returns Err."""
        rc = lib().tqkv_cache_truncate(self.h, target)
        if rc == EINVAL_TARGET:
            return False
        check(rc)
        return True

    def clear(self):
        check(lib().tqkv_cache_clear(self.h))

    def state(self):
        st = CacheState()
        check(lib().tqkv_cache_get_state(self.h, ctypes.byref(st)))
        return st

    def buffers(self):
        v = CacheView()
        check(lib().tqkv_cache_buffers(self.h, ctypes.byref(v)))
        return v

    def keep_suffix_from(self, prefix_len, stream=None):
        check(lib().tqkv_cache_keep_suffix_from(self.h, prefix_len, stream))

    def set_tables(self, rotation, qjl=None):
        self._tables = (np.ascontiguousarray(rotation, np.float32),
                        None if qjl is None else np.ascontiguousarray(qjl, np.float32))
        r, q = self._tables
        check(lib().tqkv_cache_set_tables(self.h, r.ctypes.data_as(P),
                                          None if q is None else q.ctypes.data_as(P)))

    def attach_prefix(self, prefix):
        check(lib().tqkv_cache_attach_prefix(self.h, prefix.h if prefix is not None else None))

    def decode_attend(self, q, H, scale, out, workspace=None, workspace_bytes=0, stream=None):
        check(lib().tqkv_cache_decode_attend(self.h, q, H, scale, out, workspace,
                                             workspace_bytes, stream))

    def append_decode(self, k, v, q, H, scale, out, workspace=None, workspace_bytes=0,
                      stream=None):
        """One decode step: append one token, attend over the new view."""
        check(lib().tqkv_cache_append_decode(self.h, k, v, q, H, scale, out, workspace,
                                             workspace_bytes, stream))

    def prefill_attend(self, q, H, L, scale, out, window=-1, stream=None):
        check(lib().tqkv_cache_prefill_attend(self.h, q, H, L, scale, window, out, stream))


def view_slot(view, i, n_slabs, dtype, last):
    """Download rows [0, view.n) of slot i of a view as [n_slabs, n, last]."""
    dtype = np.dtype(dtype)
    if view.n == 0:
        return np.zeros((n_slabs, 0, last), dtype)
    full = hip().download(view.slot[i], (n_slabs, view.cap, last), dtype)
    return np.ascontiguousarray(full[:, :view.n])


# ---------------------------------------------------------------- TurboQuant codebook
def _np_ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def lloyd_max(bits, n_iter=1000):
    """Host-only: (boundaries f64 [2^bits + 1], centroids f64 [2^bits])."""
    n = 1 << bits
    b = np.empty(n + 1, np.float64)
    c = np.empty(n, np.float64)
    check(lib().tqkv_lloyd_max(bits, n_iter, _np_ptr(b), _np_ptr(c)))
    return b, c


def rotation_matrix(dim, seed):
    out = np.empty((dim, dim), np.float32)
    check(lib().tqkv_rotation_matrix(dim, seed, _np_ptr(out)))
    return out


def qjl_matrix(dim, m, seed):
    out = np.empty((m, dim), np.float32)
    check(lib().tqkv_qjl_matrix(dim, m, seed, _np_ptr(out)))
    return out


def tq_encode(x, x_is_bf16, n_slabs, s, dim, R, bnd, cent, bits, phi, m, codes, sigma, signs,
              rnorm, dst_cap=None, dst_start=0, stream=None):
    """All pointers device."""
    check(lib().tqkv_tq_encode(x, int(x_is_bf16), n_slabs, s, dim, R, bnd, cent, bits, phi, m,
                               codes, sigma, signs, rnorm, s if dst_cap is None else dst_cap,
                               dst_start, stream))


def decode_attend_codebook(q, B, H, H_kv, D, scale, rotation, cent_k, bits_k, cent_v, bits_v,
                           k_codes, k_sigma, v_codes, v_sigma, cap, n, out, workspace=None,
                           workspace_bytes=0, stream=None):
    """Fused decode attention over a codebook cache; device pointers."""
    check(lib().tqkv_decode_attend_codebook(q, B, H, H_kv, D, scale, rotation, cent_k, bits_k,
                                            cent_v, bits_v, k_codes, k_sigma, v_codes, v_sigma,
                                            cap, n, out, workspace, workspace_bytes, stream))


def decode_codebook_workspace_size(B, H, D, total_tokens):
    return int(lib().tqkv_decode_codebook_workspace_size(B, H, D, total_tokens))


def codebook_dequantize(codes, sigma, centroids, bits, rows, dim, out, stream=None):
    """bf16(centroids[c] * sigma) of codebook rows; device pointers."""
    check(lib().tqkv_codebook_dequantize(codes, sigma, centroids, bits, rows, dim, out, stream))


def tq_encode_gpu_path(x, n_slabs, s, dim, R, mode, transpose, inner, bits, codes, sigma,
                       dst_cap=None, dst_start=0, stream=None):
    """The reference GPU cache's TurboQuant encode; device pointers."""
    check(lib().tqkv_tq_encode_gpu_path(x, n_slabs, s, dim, R, mode, int(transpose), inner, bits,
                                        codes, sigma, s if dst_cap is None else dst_cap, dst_start,
                                        stream))


def rotate_bf16(x, rows, dim, R, transpose, y, stream=None):
    check(lib().tqkv_rotate_bf16(x, rows, dim, R, int(transpose), y, stream))


def packed_words(dim, bits):
    """u64 words one vector of `dim` codes at `bits` packs into (-1 if out
    of range)."""
    return lib().tqkv_packed_words(dim, bits)


def pack_codes(codes, n, dim, bits, words, stream=None):
    """u8 codes [n, dim] -> u64 words in the stage1_packed layout; device."""
    check(lib().tqkv_pack_codes(codes, n, dim, bits, words, stream))


def unpack_codes(words, n, dim, bits, codes, stream=None):
    check(lib().tqkv_unpack_codes(words, n, dim, bits, codes, stream))


def tq_scores_packed(rq, words, sigma, centroids, bits, dim, n, scores, stream=None):
    check(lib().tqkv_tq_scores_packed(rq, words, sigma, centroids, bits, dim, n, scores, stream))


def tq_values_packed(R, words, sigma, centroids, weights, bits, dim, n, out, stream=None):
    check(lib().tqkv_tq_values_packed(R, words, sigma, centroids, weights, bits, dim, n, out,
                                      stream))


class KVCache:
    """turboquant_cache::KVCache (SimpleCache semantics) on the device."""

    def __init__(self, head_dim, bits=3, qjl_m=64, seed=42, n_layers=1, n_kv_heads=1,
                 rotation=None, qjl=None, lloyd_max_iter=1000):
        self.cfg = TqConfig(head_dim, bits, qjl_m, lloyd_max_iter, seed)
        self.D = head_dim
        self.m = qjl_m
        self._r = None if rotation is None else np.ascontiguousarray(rotation, np.float32)
        self._q = None if qjl is None else np.ascontiguousarray(qjl, np.float32)
        h = P()
        check(lib().tqkv_kvcache_create(ctypes.byref(self.cfg),
                                        None if self._r is None else _np_ptr(self._r),
                                        None if self._q is None else _np_ptr(self._q),
                                        n_layers, n_kv_heads, ctypes.byref(h)))
        self.h = h.value

    def close(self):
        if self.h:
            lib().tqkv_kvcache_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def store(self, layer, head, keys, values):
        k = np.ascontiguousarray(keys, np.float32).reshape(-1, self.D)
        v = np.ascontiguousarray(values, np.float32).reshape(-1, self.D)
        check(lib().tqkv_kvcache_store(self.h, layer, head, _np_ptr(k), _np_ptr(v), k.shape[0]))

    def seq_len(self, layer, head):
        return lib().tqkv_kvcache_seq_len(self.h, layer, head)

    def attend_keys(self, layer, head, query):
        q = np.ascontiguousarray(query, np.float32)
        out = np.empty(self.seq_len(layer, head), np.float32)
        check(lib().tqkv_kvcache_attend_keys(self.h, layer, head, _np_ptr(q), _np_ptr(out)))
        return out

    def attend_values(self, layer, head, weights):
        w = np.ascontiguousarray(weights, np.float32)
        out = np.empty(self.D, np.float32)
        check(lib().tqkv_kvcache_attend_values(self.h, layer, head, _np_ptr(w), _np_ptr(out)))
        return out

    def clear(self):
        check(lib().tqkv_kvcache_clear(self.h))

    def truncate(self, layer, n_keep):
        check(lib().tqkv_kvcache_truncate(self.h, layer, n_keep))

    def memory_bytes(self):
        return lib().tqkv_kvcache_memory_bytes(self.h)

    def device_bytes(self):
        """(held, reserved): bytes of the stored vectors on the device, and
        all device memory the cache owns."""
        held, reserved = I64(), I64()
        check(lib().tqkv_kvcache_device_bytes(self.h, ctypes.byref(held), ctypes.byref(reserved)))
        return held.value, reserved.value

    def read(self, layer, head, values=False, first=0, n=None):
        if n is None:
            n = self.seq_len(layer, head) - first
        W = (self.m + 31) // 32
        codes = np.empty((n, self.D), np.uint8)
        scale = np.empty(n, np.float32)
        signs = np.empty((n, max(W, 1)), np.uint32)
        rn = np.empty(n, np.float32)
        check(lib().tqkv_kvcache_read(self.h, layer, head, int(values), first, n, _np_ptr(codes),
                                      _np_ptr(scale), _np_ptr(signs), _np_ptr(rn)))
        return codes, scale, signs[:, :W], rn


# ---------------------------------------------------------------- LKV2 snapshots
def _buf(data):
    data = bytes(data)
    return data, ctypes.cast(ctypes.c_char_p(data), P) if data else None


def lkv_export(caches, fingerprint="", created_at_unix=0, position=0, prefix_tokens=(),
               last_token=None, is_deep=False, stream=None):
    """An LKV2 snapshot (bytes) whose layers are the given caches."""
    toks = np.ascontiguousarray(np.asarray(prefix_tokens, np.uint32))
    info = LkvInfo(fingerprint.encode(), created_at_unix, position,
                   toks.ctypes.data if toks.size else None, toks.size,
                   int(last_token is not None), 0 if last_token is None else last_token,
                   int(is_deep))
    arr = (P * max(len(caches), 1))(*[c.h for c in caches])
    n = SZ(0)
    check(lib().tqkv_lkv_export(arr, len(caches), ctypes.byref(info), None, 0, ctypes.byref(n),
                                stream))
    out = np.empty(n.value, np.uint8)
    check(lib().tqkv_lkv_export(arr, len(caches), ctypes.byref(info), out.ctypes.data, out.size,
                                ctypes.byref(n), stream))
    return out.tobytes()


def lkv_check(data):
    """Raises TqkvError (ECORRUPT) where the reference's read_lkv errs."""
    data, p = _buf(data)
    check(lib().tqkv_lkv_check(p, len(data)))


def lkv_manifest(data):
    """(manifest JSON text, layer count, record count)."""
    data, p = _buf(data)
    n = SZ(0)
    nl, nr = I32(0), I32(0)
    check(lib().tqkv_lkv_manifest(p, len(data), None, 0, ctypes.byref(n), ctypes.byref(nl),
                                  ctypes.byref(nr)))
    buf = ctypes.create_string_buffer(n.value + 1)
    check(lib().tqkv_lkv_manifest(p, len(data), buf, n.value + 1, ctypes.byref(n),
                                  ctypes.byref(nl), ctypes.byref(nr)))
    return buf.raw[:n.value].decode(), nl.value, nr.value


def lkv_import(data, layer, seed=42, stream=None):
    """A new device cache from layer `layer` of an LKV2 snapshot."""
    data, p = _buf(data)
    h = P()
    check(lib().tqkv_lkv_import(p, len(data), layer, seed, ctypes.byref(h), stream))
    return Cache.adopt(h.value)


def lkv_rewrite(data):
    """read_lkv then write_lkv, on the host."""
    data, p = _buf(data)
    n = SZ(0)
    check(lib().tqkv_lkv_rewrite(p, len(data), None, 0, ctypes.byref(n)))
    out = ctypes.create_string_buffer(max(n.value, 1))
    check(lib().tqkv_lkv_rewrite(p, len(data), out, n.value, ctypes.byref(n)))
    return out.raw[:n.value]


def crc32(data):
    data, p = _buf(data)
    out = ctypes.c_uint32(0)
    check(lib().tqkv_crc32(p, len(data), ctypes.byref(out)))
    return out.value
