"""BASELINE configs 2, 3 and 4 at their full sizes, through the C ABI, against
the CPU oracle on sampled sequences and rows.

Contexts are generated on the device (seeded N(0,1) with 1% of channels x10,
tqkv_synth_bf16) and quantized into place by the append kernel, whose bytes
are checked against the oracle on one sampled chunk; the attention oracle then
reads the packed cache bytes downloaded from the device, so the comparison
covers the decode and prefill kernels on exactly what they read.

- Config 2 (the headline): B=32 x 32,768 tokens, 16/8 heads, D=256, 3-bit
  gs64, through tqkv_decode_attend_affine_append with the default split
  policy: 256 (batch row, KV head) units fill the chip, so each workgroup owns
  its unit's keys, quantizes the new token in the kernel and writes the
  normalized output itself (no partials: a zero-byte workspace is accepted).
  Two steps; every appended row bit-exact with the oracle's quantization,
  sequences 0 and 31 (all heads) within 2e-2 max-abs / 1e-3 mean-abs of
  dequantize-then-attend (native_quant_attention.rs:353-403 is the
  reference's own parity form for this kernel).
- Config 4: 8 sequences over one 65,536-token prefix stored once plus 4,096
  own tokens, K 8-bit / V 4-bit: one fused step, sequences 0 and 7.
- Config 3: the global layer's last 2,048-token chunk over 16,384 keys
  (rows 2,016-2,047 of batch rows 0 and 3) and a 2,048-token chunk over a
  1,024-token ring (window 1,024; first and last 32 rows).
"""
import ctypes

import numpy as np
import pytest

import oracle_lib as O
from bars import check_bf16
from inputs import kv_bf16

pytestmark = pytest.mark.gpu



@pytest.fixture(scope="module")
def T():
    import tqkv
    assert tqkv.hip().device_count() > 0, "no GPU visible"
    return tqkv


def triple(T, slabs, cap, D, gs, bits):
    return (T.DeviceArray((slabs, cap, D * bits // 32), np.uint32),
            T.DeviceArray((slabs, cap, D // gs), np.uint16),
            T.DeviceArray((slabs, cap, D // gs), np.uint16))


def fill(T, t3, slabs, N, D, gs, bits, cap, seed, check_slabs=None):
    """Rows [0, N) of every slab: device-synthesized bf16 quantized by the
    append kernel. The first chunk of `check_slabs` is checked bit-exact
    against the oracle's quantization."""
    chunk = 1024
    tmp = T.DeviceArray((slabs, chunk, D), np.uint16)
    for c0 in range(0, N, chunk):
        n = min(chunk, N - c0)
        T.synth_bf16(tmp.ptr, slabs * n, D, seed * 1000003 + c0, 0.01, 10.0)
        T.affine_quantize(tmp.ptr, slabs, n, D, gs, bits, *(a.ptr for a in t3), cap, c0)
        if c0 == 0 and check_slabs is not None:
            T.hip().sync()
            x = tmp.numpy()[:slabs * n].reshape(slabs, n, D)[check_slabs]
            want = O.affine_quantize(x, gs, bits)
            for a, w in zip(t3, want):
                got = download_slabs(T, a, check_slabs[0], len(check_slabs), a.shape[1])[:, :n]
                assert np.array_equal(got, w), "append kernel differs from the oracle"
    T.hip().sync()


def download_slabs(T, a, first, count, rows):
    """Rows [0, rows) of slabs [first, first + count) of a [slabs, cap, last] array."""
    cap, last = a.shape[1], a.shape[2]
    off = first * cap * last * a.dtype.itemsize
    full = T.hip().download(a.ptr + off, (count, cap, last), a.dtype)
    return np.ascontiguousarray(full[:, :rows])


def download_row(T, a, row):
    """Row `row` of every slab of a [slabs, cap, last] array (hipMemcpy2D)."""
    slabs, cap, last = a.shape
    out = np.empty((slabs, last), a.dtype)
    width = last * a.dtype.itemsize
    h = T.hip().h
    h.hipMemcpy2D.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                              ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int]
    h.hipMemcpy2D.restype = ctypes.c_int
    T.hip()._ok(h.hipMemcpy2D(out.ctypes.data, width, a.ptr + row * width, cap * width, width,
                              slabs, 2), "hipMemcpy2D")
    return out


def want_mlx(q, kt, vt, gs, bk, bv, scale, **kw):
    """Prefill's oracle over the mlx::dequantize'd cache (one rounding of the
    fused multiply-add), and over the secondary reading (two bf16
    roundings), printed only."""
    return tuple(O.attend_affine(q, kt, vt, gs, bk, bv, scale, dequant=d, **kw)[0]
                 for d in ("bf16", "bf16_2r"))


def check(got_bf16, want_f32, tag, secondary=None):
    """The bar in bf16 (bars.check_bf16); secondary: the other reading of
    mlx::dequantize, whose raw distance is printed."""
    check_bf16(got_bf16, want_f32, f"full-size {tag}")
    if secondary is not None:
        got = O.bf16_to_f32(got_bf16).astype(np.float64)
        print(f"[full-size {tag}] secondary reading: max_abs="
              f"{np.abs(got - secondary).max():.3e}", flush=True)


def test_config2_headline_path(T):
    B, H, HKV, D, N, GS, BITS = 32, 16, 8, 256, 32768, 64, 3
    slabs, cap, scale = B * HKV, N + 256, D ** -0.5
    print(f"[full-size] config 2: B={B} N={N} H={H}/{HKV} D={D} {BITS}-bit", flush=True)
    assert T.decode_kernel_name(H, HKV, D, GS, BITS, BITS) == "mfma"
    kc, vc = triple(T, slabs, cap, D, GS, BITS), triple(T, slabs, cap, D, GS, BITS)
    fill(T, kc, slabs, N, D, GS, BITS, cap, 11, check_slabs=list(range(HKV)))
    fill(T, vc, slabs, N, D, GS, BITS, cap, 22)
    kp, vp = tuple(a.ptr for a in kc), tuple(a.ptr for a in vc)
    news, outs = [], []
    for step in range(2):
        pos = N + step
        nk = kv_bf16((B, HKV, 1, D), 500 + step, frac=0.01, mult=10.0)
        nv = kv_bf16((B, HKV, 1, D), 600 + step, frac=0.01, mult=10.0)
        q = kv_bf16((B, H, 1, D), 700 + step)
        dk, dv, dq = T.DeviceArray.of(nk), T.DeviceArray.of(nv), T.DeviceArray.of(q)
        out = T.DeviceArray((B, H, 1, D), np.uint16)
        dummy = T.DeviceArray((1,), np.uint8)
        # A zero-byte workspace: the call must need none (one split a unit,
        # the output normalized in the kernel).
        T.decode_attend_affine_append(dq.ptr, B, H, HKV, D, GS, BITS, BITS, scale,
                                      [T.affine_seg(kp, vp, cap, pos)], dk.ptr, dv.ptr, kp + vp,
                                      cap, pos, out.ptr, dummy.ptr, 0)
        T.hip().sync()
        for trip, x in ((kc, nk), (vc, nv)):
            want = O.affine_quantize(x.reshape(slabs, 1, D), GS, BITS)
            for a, w in zip(trip, want):
                assert np.array_equal(download_row(T, a, pos), w[:, 0]), f"row {pos} differs"
        news.append((nk, nv))
        outs.append((q, out.numpy()))
    for b in (0, B - 1):
        kt = tuple(download_slabs(T, a, b * HKV, HKV, N + 2)[None] for a in kc)
        vt = tuple(download_slabs(T, a, b * HKV, HKV, N + 2)[None] for a in vc)
        for step, (q, got) in enumerate(outs):
            n = N + step + 1
            want, _, _ = O.attend_affine(q[b:b + 1], tuple(x[:, :, :n] for x in kt),
                                         tuple(x[:, :, :n] for x in vt), GS, BITS, BITS, scale)
            check(got[b:b + 1], want, f"config 2 b={b} step={step} keys={n}")


def test_config4_shared_prefix(T):
    B, H, HKV, D, P, S0, GS, BK, BV = 8, 32, 8, 128, 65536, 4096, 64, 8, 4
    cap, scale = S0 + 64, D ** -0.5
    print(f"[full-size] config 4: B={B} prefix={P} suffix={S0} bits={BK}/{BV}", flush=True)
    pk, pv = triple(T, HKV, P, D, GS, BK), triple(T, HKV, P, D, GS, BV)
    sk, sv = triple(T, B * HKV, cap, D, GS, BK), triple(T, B * HKV, cap, D, GS, BV)
    fill(T, pk, HKV, P, D, GS, BK, P, 21, check_slabs=[0, 1])
    fill(T, pv, HKV, P, D, GS, BV, P, 22)
    fill(T, sk, B * HKV, S0, D, GS, BK, cap, 23)
    fill(T, sv, B * HKV, S0, D, GS, BV, cap, 24, check_slabs=list(range(HKV, 2 * HKV)))
    nk = kv_bf16((B, HKV, 1, D), 801)
    nv = kv_bf16((B, HKV, 1, D), 802)
    q = kv_bf16((B, H, 1, D), 803)
    dk, dv, dq = T.DeviceArray.of(nk), T.DeviceArray.of(nv), T.DeviceArray.of(q)
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    pkp, pvp = tuple(a.ptr for a in pk), tuple(a.ptr for a in pv)
    skp, svp = tuple(a.ptr for a in sk), tuple(a.ptr for a in sv)
    segs = [T.affine_seg(pkp, pvp, P, P, shared=True), T.affine_seg(skp, svp, cap, S0)]
    T.decode_attend_affine_append(dq.ptr, B, H, HKV, D, GS, BK, BV, scale, segs, dk.ptr, dv.ptr,
                                  skp + svp, cap, S0, out.ptr)
    T.hip().sync()
    got = out.numpy()
    for trip, x, bits in ((sk, nk, BK), (sv, nv, BV)):
        want = O.affine_quantize(x.reshape(B * HKV, 1, D), GS, bits)
        for a, w in zip(trip, want):
            assert np.array_equal(download_row(T, a, S0), w[:, 0])
    pre_k = tuple(download_slabs(T, a, 0, HKV, P)[None] for a in pk)
    pre_v = tuple(download_slabs(T, a, 0, HKV, P)[None] for a in pv)
    for b in (0, B - 1):
        kt = tuple(np.concatenate([p, download_slabs(T, a, b * HKV, HKV, S0 + 1)[None]], axis=2)
                   for p, a in zip(pre_k, sk))
        vt = tuple(np.concatenate([p, download_slabs(T, a, b * HKV, HKV, S0 + 1)[None]], axis=2)
                   for p, a in zip(pre_v, sv))
        want, _, _ = O.attend_affine(q[b:b + 1], kt, vt, GS, BK, BV, scale)
        check(got[b:b + 1], want, f"config 4 b={b} keys={P + S0 + 1}")


def _chunk(T, B, HKV, L, D, seed):
    x = T.DeviceArray((B, HKV, L, D), np.uint16)
    T.synth_bf16(x.ptr, B * HKV * L, D, seed, 0.01, 10.0)
    return x


def test_config3_global_chunk(T):
    B, H, HKV, D, GS, BITS, CH, TOTAL = 4, 32, 8, 128, 64, 4, 2048, 16384
    scale = D ** -0.5
    print(f"[full-size] config 3 global: B={B} {TOTAL} keys in chunks of {CH}", flush=True)
    c = T.Cache(T.CACHE_AFFINE, B, HKV, D, D, GS, BITS, BITS, prealloc=True)
    ks, vs = [], []
    for c0 in range(0, TOTAL, CH):
        k, v = _chunk(T, B, HKV, CH, D, 9000 + c0), _chunk(T, B, HKV, CH, D, 19000 + c0)
        c.append(k.ptr, v.ptr, CH)
        ks.append(k)
        vs.append(v)
    T.hip().sync()
    q = kv_bf16((B, H, CH, D), 33)
    dq = T.DeviceArray.of(q)
    out = T.DeviceArray((B, H, CH, D), np.uint16)
    c.prefill_attend(dq.ptr, H, CH, scale, out.ptr)
    T.hip().sync()
    view = c.buffers()
    got = out.numpy()
    spec = [(np.uint32, D * BITS // 32), (np.uint16, D // GS), (np.uint16, D // GS)]
    kt = tuple(T.view_slot(view, i, B * HKV, dt, w).reshape(B, HKV, TOTAL, w)
               for i, (dt, w) in enumerate(spec))
    vt = tuple(T.view_slot(view, 3 + i, B * HKV, dt, w).reshape(B, HKV, TOTAL, w)
               for i, (dt, w) in enumerate(spec))
    # The cache's bytes of the first chunk equal the oracle's quantization.
    first = ks[0].numpy()
    want = O.affine_quantize(first, GS, BITS)
    assert all(np.array_equal(a[:, :, :CH], w) for a, w in zip(kt, want))
    rows = slice(CH - 32, CH)
    for b in (0, B - 1):
        wants = want_mlx(q[b:b + 1, :, rows], tuple(a[b:b + 1] for a in kt),
                         tuple(a[b:b + 1] for a in vt), GS, BITS, BITS, scale,
                         causal=True, q_start=TOTAL - 32, first_held=0)
        check(got[b:b + 1, :, rows], wants[0], f"config 3 global b={b} rows 2016-2047",
              secondary=wants[1])


def test_config3_ring_chunk(T):
    B, H, HKV, D, GS, BITS, CH, W = 4, 32, 8, 128, 64, 4, 2048, 1024
    scale = D ** -0.5
    print(f"[full-size] config 3 sliding: ring {W}, chunks of {CH}", flush=True)
    c = T.Cache(T.CACHE_AFFINE, B, HKV, D, D, GS, BITS, BITS, prealloc=True, max_size=W)
    chunks = [(_chunk(T, B, HKV, CH, D, 300 + i), _chunk(T, B, HKV, CH, D, 400 + i))
              for i in range(2)]
    host = [(k.numpy(), v.numpy()) for k, v in chunks]
    pos = 0
    for i, (k, v) in enumerate(chunks):
        view = c.append(k.ptr, v.ptr, CH)
        pos += CH
        q = kv_bf16((B, H, CH, D), 50 + i)
        dq = T.DeviceArray.of(q)
        out = T.DeviceArray((B, H, CH, D), np.uint16)
        c.prefill_attend(dq.ptr, H, CH, scale, out.ptr, window=W)
        T.hip().sync()
        n = view.n
        first = pos - n
        print(f"[full-size] ring chunk {i}: view {n} keys from {first}", flush=True)
        K = np.concatenate([h[0] for h in host[:i + 1]], axis=2)[:, :, first:pos]
        V = np.concatenate([h[1] for h in host[:i + 1]], axis=2)[:, :, first:pos]
        got = out.numpy()
        for b in (0, B - 1):
            kt = O.affine_quantize(np.ascontiguousarray(K[b:b + 1]), GS, BITS)
            vt = O.affine_quantize(np.ascontiguousarray(V[b:b + 1]), GS, BITS)
            for rows in (slice(0, 32), slice(CH - 32, CH)):
                wants = want_mlx(
                    np.ascontiguousarray(q[b:b + 1, :, rows]), kt, vt, GS, BITS, BITS, scale,
                    causal=True, q_start=pos - CH + rows.start, first_held=first, window=W)
                check(got[b:b + 1, :, rows], wants[0],
                      f"ring chunk {i} b={b} rows {rows.start}+32", secondary=wants[1])
