"""Prefill-chunk attention over codebook (TurboQuant) and bf16 caches, and
the standalone codebook dequantize, through the C ABI, against the CPU
oracle.

The reference's TurboQuant branch prefills by lloyd_max_dequantize_scaled
(bf16(centroid[c] * sigma), turboquant.rs:428-439), K_eff from the QJL signs
when the cache keeps them (qjl_apply_correction_packed), and SDPA with its
mask (gemma4_moe.rs:4546-4600), with V_dq rotated back to the original
basis first (unrotate_v_dq). The cache holds rotated rows (R x), so the
oracle attends bf16(R q) against the dequantized keys and the rotated-back
values. Bar: 2e-2 max-abs beyond half a bf16 step of the expected value
(the raw max-abs is printed; bf16 softmax weights, the reference SDPA's
operand type, move outputs by up to 2^-8 of their range) and 1e-3 mean-abs.
"""
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


def check(got_bf16, want, tag):
    check_bf16(got_bf16, want, f"cb-prefill {tag}")


def dequant(cent, codes, sigma):
    """bf16(centroid[c] * sigma), the product in f32."""
    return O.bf16_from_f32(cent.astype(np.float32)[codes] * sigma[..., None].astype(np.float32))


@pytest.mark.parametrize("bits", [3, 4, 8])
def test_codebook_dequantize_bit_exact(T, bits):
    rows, D = 777, 128
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, (rows, D)).astype(np.uint8)
    sigma = np.abs(rng.standard_normal(rows)).astype(np.float32) * 3
    _, cent = T.lloyd_max(bits)
    cent = cent.astype(np.float32)
    dc, ds, dcent = T.DeviceArray.of(codes), T.DeviceArray.of(sigma), T.DeviceArray.of(cent)
    out = T.DeviceArray((rows, D), np.uint16)
    T.codebook_dequantize(dc.ptr, ds.ptr, dcent.ptr, bits, rows, D, out.ptr)
    T.hip().sync()
    assert np.array_equal(out.numpy(), dequant(cent, codes, sigma))


@pytest.mark.parametrize("bits,qjl_words,D,G,encode", [
    (4, 0, 128, 4, 0), (3, 0, 256, 2, 0), (6, 0, 512, 8, 0),   # compress_one codes
    (4, 0, 128, 4, 1), (8, 2, 128, 2, 1), (4, 4, 64, 1, 1),   # the GPU cache's codes
])
def test_codebook_cache_prefill(T, bits, qjl_words, D, G, encode):
    # A rotating TurboQuant cache of window W: a first chunk, then a chunk
    # that wraps it (rotating_concat keeps the newest W - 1 and appends), each
    # attended causally with the window by its own queries. The cache's rows
    # are R_eff x: R x (compress_one) or x R = R^T x (the GPU cache's encode).
    B, Hkv, W = 2, 2, 192
    Hq = Hkv * G
    c = T.Cache(T.CACHE_CODEBOOK, B, Hkv, D, D, bits_k=bits, bits_v=bits, qjl_words=qjl_words,
                max_size=W, keep=0, seed=42, encode=encode)
    R = T.rotation_matrix(D, 42).astype(np.float64)
    R = R.T if encode else R  # R_eff
    m = 32 * qjl_words
    phi = T.qjl_matrix(D, max(m, 1), 43)
    _, cent = T.lloyd_max(bits)
    cent = cent.astype(np.float32)
    total = 0
    for i, L in enumerate((150, 100)):
        k = kv_bf16((B, Hkv, L, D), 80 + i, frac=0.02, mult=8.0)
        v = kv_bf16((B, Hkv, L, D), 90 + i, frac=0.02, mult=8.0)
        dk, dv = T.DeviceArray.of(k), T.DeviceArray.of(v)
        view = c.append(dk.ptr, dv.ptr, L)
        total += L
        q = kv_bf16((B, Hq, L, D), 100 + i)
        dq = T.DeviceArray.of(q)
        out = T.DeviceArray((B, Hq, L, D), np.uint16)
        print(f"[cb-prefill] bits={bits} qjl={qjl_words} D={D} G={G} chunk {i} L={L} "
              f"view={view.n}", flush=True)
        c.prefill_attend(dq.ptr, Hq, L, D ** -0.5, out.ptr, window=W)
        T.hip().sync()
        n = view.n
        bufs = c.buffers()
        kc = T.view_slot(bufs, 0, B * Hkv, np.uint8, D)[:, :n]
        ks = T.view_slot(bufs, 1, B * Hkv, np.float32, 1)[:, :n, 0]
        vi = 4 if qjl_words else 2
        vc = T.view_slot(bufs, vi, B * Hkv, np.uint8, D)[:, :n]
        vs = T.view_slot(bufs, vi + 1, B * Hkv, np.float32, 1)[:, :n, 0]
        K = dequant(cent, kc, ks).reshape(-1, D)
        if qjl_words:
            sg = T.view_slot(bufs, 2, B * Hkv, np.uint32, qjl_words)[:, :n].reshape(-1, qjl_words)
            rn = T.view_slot(bufs, 3, B * Hkv, np.float32, 1)[:, :n, 0].reshape(-1)
            K = O.qjl_apply_correction(K, sg, rn, phi[:m], m)
        K = K.reshape(B, Hkv, n, D)
        V = dequant(cent, vc, vs).reshape(B, Hkv, n, D)
        V = O.bf16_from_f32((O.bf16_to_f32(V).astype(np.float64) @ R).astype(np.float32))
        qr = O.bf16_from_f32((O.bf16_to_f32(q).astype(np.float64) @ R.T).astype(np.float32))
        want, _, _ = O.attend_bf16(qr, K, V, D ** -0.5, causal=True, q_start=total - L,
                                   first_held=total - n, window=W)
        check(out.numpy(), want, f"chunk {i}")


def test_bf16_cache_prefill(T):
    B, Hq, Hkv, D = 2, 16, 4, 128
    c = T.Cache(T.CACHE_BF16, B, Hkv, D, D)
    ks, vs = [], []
    total = 0
    for i, L in enumerate((130, 70)):
        k, v = kv_bf16((B, Hkv, L, D), 10 + i), kv_bf16((B, Hkv, L, D), 20 + i)
        ks.append(k)
        vs.append(v)
        dk, dv = T.DeviceArray.of(k), T.DeviceArray.of(v)
        c.append(dk.ptr, dv.ptr, L)
        total += L
        q = kv_bf16((B, Hq, L, D), 30 + i)
        dq = T.DeviceArray.of(q)
        out = T.DeviceArray((B, Hq, L, D), np.uint16)
        c.prefill_attend(dq.ptr, Hq, L, D ** -0.5, out.ptr)
        T.hip().sync()
        want, _, _ = O.attend_bf16(q, np.concatenate(ks, axis=2), np.concatenate(vs, axis=2),
                                   D ** -0.5, causal=True, q_start=total - L, first_held=0)
        check(out.numpy(), want, f"bf16 chunk {i}")


def test_compress_one_qjl_prefill_is_unsupported(T):
    # compress_one's QJL signs are of the original-basis residual; the
    # reference prefills with QJL only over its GPU cache's rotated-residual
    # signs, so this layout answers "unsupported" (the caller falls back).
    B, Hkv, D = 1, 2, 128
    c = T.Cache(T.CACHE_CODEBOOK, B, Hkv, D, D, bits_k=4, bits_v=4, qjl_words=2, max_size=64)
    k = T.DeviceArray.of(kv_bf16((B, Hkv, 8, D), 1))
    c.append(k.ptr, k.ptr, 8)
    q = T.DeviceArray.of(kv_bf16((B, 4, 8, D), 2))
    out = T.DeviceArray((B, 4, 8, D), np.uint16)
    with pytest.raises(T.TqkvError) as e:
        c.prefill_attend(q.ptr, 4, 8, 0.1, out.ptr)
    assert e.value.status == T.EUNSUPPORTED


@pytest.mark.parametrize("bits,qjl_words,D", [(4, 0, 128), (3, 2, 256), (8, 4, 64)])
def test_gpu_path_cache_append_and_decode(T, bits, qjl_words, D):
    # A codebook cache with the reference GPU cache's encode: its code and
    # sigma rows equal tqkv_tq_encode_gpu_path's mode 1 restated by the
    # oracle (x R, seed-42 R), its QJL rows qjl_encode_stage2 of the rotated
    # keys against their dequantized codes, and decode attends in that basis
    # (R_eff = R^T) within the bar.
    B, Hq, Hkv, W = 2, 8, 2, 512
    c = T.Cache(T.CACHE_CODEBOOK, B, Hkv, D, D, bits_k=bits, bits_v=bits, qjl_words=qjl_words,
                max_size=W, keep=0, seed=42, encode=1)
    k = kv_bf16((B, Hkv, 201, D), 41, frac=0.02, mult=8.0)
    v = kv_bf16((B, Hkv, 201, D), 42, frac=0.02, mult=8.0)
    for a, s in [(0, 200), (200, 1)]:
        dk = T.DeviceArray.of(np.ascontiguousarray(k[:, :, a:a + s]))
        dv = T.DeviceArray.of(np.ascontiguousarray(v[:, :, a:a + s]))
        c.append(dk.ptr, dv.ptr, s)
    n = 201
    R = T.rotation_matrix(D, 42)
    b, cent = T.lloyd_max(bits)
    inner = np.asarray(b[1:-1]).astype(np.float32)
    cent = cent.astype(np.float32)
    bufs = c.buffers()
    kc = T.view_slot(bufs, 0, B * Hkv, np.uint8, D)[:, :n].reshape(-1, D)
    ks = T.view_slot(bufs, 1, B * Hkv, np.float32, 1)[:, :n, 0].reshape(-1)
    vi = 4 if qjl_words else 2
    vc = T.view_slot(bufs, vi, B * Hkv, np.uint8, D)[:, :n].reshape(-1, D)
    vs = T.view_slot(bufs, vi + 1, B * Hkv, np.float32, 1)[:, :n, 0].reshape(-1)
    for x, codes, sig in ((k, kc, ks), (v, vc, vs)):
        wc, ws = O.tq_encode_gpu_path(x.reshape(-1, D), inner, R, mode=1)
        assert np.array_equal(codes, wc)
        assert np.array_equal(sig.view(np.uint32), ws.view(np.uint32))
    m = 32 * qjl_words
    phi = T.qjl_matrix(D, max(m, 1), 43)
    if qjl_words:
        # The rotated keys as the append made them (rotate_last_axis).
        dk, dR = T.DeviceArray.of(k), T.DeviceArray.of(R)
        krot = T.DeviceArray(k.shape, np.uint16)
        T.rotate_bf16(dk.ptr, B * Hkv * n, D, dR.ptr, False, krot.ptr)
        T.hip().sync()
        sg = T.view_slot(bufs, 2, B * Hkv, np.uint32, qjl_words)[:, :n].reshape(-1, qjl_words)
        rn = T.view_slot(bufs, 3, B * Hkv, np.float32, 1)[:, :n, 0].reshape(-1)
        wsg, wrn = O.qjl_encode_stage2(krot.numpy().reshape(-1, D), dequant(cent, kc, ks),
                                       phi[:m], m)
        assert np.array_equal(sg, wsg)
        assert np.array_equal(rn.view(np.uint32), wrn.view(np.uint32))
    q = kv_bf16((B, Hq, 1, D), 43)
    dq = T.DeviceArray.of(q)
    out = T.DeviceArray((B, Hq, 1, D), np.uint16)
    c.decode_attend(dq.ptr, Hq, D ** -0.5, out.ptr)
    T.hip().sync()
    Reff = R.T.astype(np.float32)
    kc4, vc4 = kc.reshape(B, Hkv, n, D), vc.reshape(B, Hkv, n, D)
    ks3, vs3 = ks.reshape(B, Hkv, n), vs.reshape(B, Hkv, n)
    if qjl_words:
        want = O.attend_codebook_qjl(q, kc4, ks3, sg.reshape(B, Hkv, n, qjl_words),
                                     rn.reshape(B, Hkv, n), vc4, vs3, cent, cent, Reff,
                                     (phi[:m].astype(np.float64) @ Reff).astype(np.float32), m,
                                     D ** -0.5)
    else:
        G = Hq // Hkv
        qr = O.bf16_to_f32(q).reshape(B, Hq, D).astype(np.float64) @ Reff.T.astype(np.float64)
        Kr = cent.astype(np.float64)[kc4] * ks3[..., None]
        Vr = cent.astype(np.float64)[vc4] * vs3[..., None]
        want = np.zeros((B, Hq, D))
        for bb in range(B):
            for h in range(Hq):
                sc = (Kr[bb, h // G] @ qr[bb, h]) * D ** -0.5
                p = np.exp(sc - sc.max())
                want[bb, h] = ((p @ Vr[bb, h // G]) / p.sum()) @ Reff.astype(np.float64)
    check(out.numpy().reshape(B, Hq, D), np.asarray(want, np.float64).reshape(B, Hq, D),
          f"gpu-path decode bits={bits} qjl={qjl_words} D={D}")
