"""The device cache object (tqkv_cache_*) through the C ABI.

1. The reference's golden plans (native_cache/golden_tests.rs:182-497) replay
   through the device cache, quantize-on-append included for the affine
   kinds, and every fetched view, buffer and counter folds into the FNV-1a
   digest the reference recorded: bit-exact growth, ring, trim, rewind.
2. Rewind refusals the plans do not reach (ring_truncate, native_cache.rs:
   304-335; the quantized legacy path :923-929).
3. Decode attention over a cache's fetched view: growing, rotating (the held
   tokens in ring order), and split into a shared prefix plus suffixes
   (keep_suffix_from + SharedPrefixKv, native_cache.rs:464-494, 2044-2051),
   against the oracle's dequantize-then-attend over the same tokens.
"""
import numpy as np
import pytest

import oracle_lib as O
from bars import check_bf16
from inputs import kv_bf16
from test_oracle_golden import RECORDED

pytestmark = pytest.mark.gpu



@pytest.fixture(scope="module")
def T():
    import tqkv
    assert tqkv.hip().device_count() > 0, "no GPU visible"
    return tqkv


# (digest dtype code, numpy dtype, last) per slot
U8, U32, F32, BF = (1, np.uint8), (2, np.uint32), (3, np.float32), (4, np.uint16)
SLOTS = {
    "full": [BF + (16,), BF + (24,)],
    "rot": [BF + (16,), BF + (24,)],
    "quant_full": [U32 + (8,), BF + (1,), BF + (1,), U32 + (16,), BF + (2,), BF + (2,)],
    "rot_quant": [U32 + (8,), BF + (1,), BF + (1,), U32 + (16,), BF + (2,), BF + (2,)],
    "tq": [U8 + (16,), F32 + (1,), U8 + (24,), F32 + (1,)],
    "tq_qjl": [U8 + (16,), F32 + (1,), U32 + (2,), F32 + (1,), U8 + (24,), F32 + (1,)],
}
H = 2  # golden_tests.rs:273


def replay(T, kind, plan, prealloc):
    events, data, max_size, keep = O.golden_tape(kind, plan)
    ring = kind not in ("full", "quant_full")
    quant = kind in ("quant_full", "rot_quant")
    slots = SLOTS[kind]
    if quant:
        cache = T.Cache(T.CACHE_AFFINE, 1, H, 64, 128, 64, 4, 4, prealloc=prealloc,
                        max_size=max_size if ring else 0, keep=keep if ring else 0)
    elif kind in ("full", "rot"):
        cache = T.Cache(T.CACHE_BF16, 1, H, 16, 24, prealloc=prealloc,
                        max_size=max_size if ring else 0, keep=keep if ring else 0)
    else:
        cache = T.Cache(T.CACHE_CODEBOOK, 1, H, 16, 24, qjl_words=2 if kind == "tq_qjl" else 0,
                        prealloc=prealloc, max_size=max_size, keep=keep)

    def arr(view, i):
        code, dt, last = slots[i]
        return T.view_slot(view, i, H, dt, last)

    def state(d):
        st = cache.state()
        has = not st.empty
        bufs = cache.buffers()

        def opt(d, i):
            if not has:
                return O.fnv_num(d, 0)
            return O.fnv_array(O.fnv_num(d, 1), slots[i][0], arr(bufs, i))

        if kind == "full":
            d = opt(opt(d, 0), 1)
            return O.fnv_num(O.fnv_num(d, st.offset), 0)
        if quant:
            for t in range(2):
                if not has:
                    d = O.fnv_num(d, 0)
                    continue
                d = O.fnv_num(d, 1)
                for i in range(3):
                    d = O.fnv_array(d, slots[3 * t + i][0], arr(bufs, 3 * t + i))
            d = O.fnv_num(d, st.offset)
            if ring:
                d = O.fnv_num(O.fnv_num(d, st.idx), st.cached_len)
            return d
        if kind == "rot":
            d = opt(opt(d, 0), 1)
        elif kind == "tq":
            for i in range(4):
                d = opt(d, i)
            d = O.fnv_num(O.fnv_num(d, 0), 0)
        else:
            for i in (0, 1, 4, 5, 2, 3):
                d = opt(d, i)
        return O.fnv_num(O.fnv_num(O.fnv_num(d, st.offset), st.idx), st.cached_len)

    d = O.FNV_OFFSET
    keepalive = []
    for op, n, at in events:
        if op == "R":
            d = state(O.fnv_num(d, 1 if cache.truncate(n) else 0))
            continue
        s = n
        if quant:
            k = data[at:at + H * s * 64 * 2].view(np.uint16).reshape(1, H, s, 64)
            v = data[at + H * s * 64 * 2:at + H * s * 192 * 2].view(np.uint16).reshape(1, H, s, 128)
            dk, dv = T.DeviceArray.of(k), T.DeviceArray.of(v)
            view = cache.append(dk.ptr, dv.ptr, s)
            keepalive = [dk, dv]
            for t in range(2):
                d = O.fnv_num(d, 1)
                for i in range(3):
                    d = O.fnv_array(d, slots[3 * t + i][0], arr(view, 3 * t + i))
        else:
            devs, p = [], at
            for code, dt, last in slots:
                nb = H * s * last * np.dtype(dt).itemsize
                devs.append(T.DeviceArray.of(data[p:p + nb].view(dt).reshape(1, H, s, last)))
                p += nb
            view = cache.update([a.ptr for a in devs], s)
            keepalive = devs
            for i in range(len(slots)):
                d = O.fnv_array(d, slots[i][0], arr(view, i))
        d = state(d)
    del keepalive
    cache.close()
    return d


@pytest.mark.parametrize("kind,plan,prealloc,want", RECORDED)
def test_device_cache_reproduces_reference_recording(T, kind, plan, prealloc, want):
    print(f"[cache-golden] {kind}/{plan} prealloc={prealloc}", flush=True)
    got = replay(T, kind, plan, prealloc)
    assert got == want, f"{got:#x} != {want:#x}"


def test_rewind_refusals(T):
    # A ring that has wrapped refuses any rewind (ring_truncate's
    # `offset > max_size` arm), but one exactly full does not.
    c = T.Cache(T.CACHE_BF16, 1, 2, 16, 16, max_size=8, keep=0)
    x = T.DeviceArray.of(kv_bf16((1, 2, 1, 16), 1))
    for _ in range(8):
        c.update([x.ptr, x.ptr], 1)
    assert c.truncate(6) and c.state().offset == 6 and c.state().idx == 6
    for _ in range(3):
        c.update([x.ptr, x.ptr], 1)  # offset 9 > 8: wrapped
    st = c.state()
    assert (st.offset, st.cached_len) == (9, 8)
    assert not c.truncate(8) and c.truncate(9) and not c.truncate(10)
    # An affine growing cache on the legacy path refuses real rewinds.
    q = T.Cache(T.CACHE_AFFINE, 1, 2, 64, 64, 64, 4, 4, prealloc=False)
    y = T.DeviceArray.of(kv_bf16((1, 2, 3, 64), 2))
    q.append(y.ptr, y.ptr, 3)
    assert not q.truncate(2) and q.truncate(3) and not q.truncate(4)
    p = T.Cache(T.CACHE_AFFINE, 1, 2, 64, 64, 64, 4, 4, prealloc=True)
    p.append(y.ptr, y.ptr, 3)
    assert p.truncate(2) and p.state().offset == 2


def check_close(got_bf16, want_f32):
    check_bf16(got_bf16, want_f32, "cache-decode")


def decode(T, cache, q, H_, scale):
    dq = T.DeviceArray.of(q)
    out = T.DeviceArray(q.shape, np.uint16)
    cache.decode_attend(dq.ptr, H_, scale, out.ptr)
    T.hip().sync()
    return out.numpy()


@pytest.mark.parametrize("bk,bv", [(4, 4), (8, 4), (3, 3)])
def test_decode_over_growing_cache(T, bk, bv):
    # Appends in uneven chunks then single tokens (crossing the 256-token
    # steps), decodes over the fetched view.
    B, Hq, Hkv, D = 2, 8, 2, 128 if bk != 3 or bv != 3 else 256
    c = T.Cache(T.CACHE_AFFINE, B, Hkv, D, D, 64, bk, bv, prealloc=True)
    ks, vs = [], []
    for i, s in enumerate([300, 1, 1, 211, 1]):
        k = kv_bf16((B, Hkv, s, D), 10 + i, frac=0.02, mult=8.0)
        v = kv_bf16((B, Hkv, s, D), 20 + i, frac=0.02, mult=8.0)
        dk, dv = T.DeviceArray.of(k), T.DeviceArray.of(v)
        c.append(dk.ptr, dv.ptr, s)
        ks.append(k)
        vs.append(v)
    K, V = np.concatenate(ks, axis=2), np.concatenate(vs, axis=2)
    assert c.state().offset == K.shape[2] and c.state().view == K.shape[2]
    q = kv_bf16((B, Hq, 1, D), 99)
    got = decode(T, c, q, Hq, D ** -0.5)
    want, _, _ = O.attend_affine(q, O.affine_quantize(K, 64, bk), O.affine_quantize(V, 64, bv),
                                 64, bk, bv, D ** -0.5)
    check_close(got, want)


def test_decode_over_rotating_cache(T):
    # A 4-bit window of 96 tokens with 4 sinks: after the ring wraps, decode
    # sees exactly the sinks plus the newest 92 tokens (in ring order).
    B, Hq, Hkv, D, W, KEEP = 1, 8, 2, 128, 96, 4
    c = T.Cache(T.CACHE_AFFINE, B, Hkv, D, D, 64, 4, 4, prealloc=True, max_size=W, keep=KEEP)
    k_all = kv_bf16((B, Hkv, 200, D), 31, frac=0.02, mult=8.0)
    v_all = kv_bf16((B, Hkv, 200, D), 32, frac=0.02, mult=8.0)
    q = kv_bf16((B, Hq, 1, D), 33)
    pos = 0
    for s in [40] + [1] * 160:
        dk = T.DeviceArray.of(np.ascontiguousarray(k_all[:, :, pos:pos + s]))
        dv = T.DeviceArray.of(np.ascontiguousarray(v_all[:, :, pos:pos + s]))
        c.append(dk.ptr, dv.ptr, s)
        pos += s
        if pos in (40, 95, 96, 97, 150, 200):
            held = list(range(pos)) if pos <= W else list(range(KEEP)) + list(range(pos - (W - KEEP), pos))
            K = np.ascontiguousarray(k_all[:, :, held])
            V = np.ascontiguousarray(v_all[:, :, held])
            got = decode(T, c, q, Hq, D ** -0.5)
            want, _, _ = O.attend_affine(q, O.affine_quantize(K, 64, 4), O.affine_quantize(V, 64, 4),
                                         64, 4, 4, D ** -0.5)
            print(f"[ring] pos={pos} held={len(held)} view={c.state().view}", flush=True)
            assert c.state().view == len(held)
            check_close(got, want)


def test_decode_over_shared_prefix(T):
    # Config-4 layout (K 8-bit / V 4-bit): every sequence prefilled with the
    # same prefix then its own suffix; keep_suffix_from drops the prefix and a
    # batch-1 prefix cache serves every row.
    B, Hq, Hkv, D, P, S = 3, 16, 4, 128, 700, 90
    pre_k = kv_bf16((1, Hkv, P, D), 41)
    pre_v = kv_bf16((1, Hkv, P, D), 42)
    suf_k = kv_bf16((B, Hkv, S, D), 43)
    suf_v = kv_bf16((B, Hkv, S, D), 44)
    prefix = T.Cache(T.CACHE_AFFINE, 1, Hkv, D, D, 64, 8, 4)
    a, b = T.DeviceArray.of(pre_k), T.DeviceArray.of(pre_v)
    prefix.append(a.ptr, b.ptr, P)
    seqs = T.Cache(T.CACHE_AFFINE, B, Hkv, D, D, 64, 8, 4)
    full_k = np.concatenate([np.broadcast_to(pre_k, (B, Hkv, P, D)), suf_k], axis=2)
    full_v = np.concatenate([np.broadcast_to(pre_v, (B, Hkv, P, D)), suf_v], axis=2)
    fk, fv = T.DeviceArray.of(np.ascontiguousarray(full_k)), T.DeviceArray.of(np.ascontiguousarray(full_v))
    seqs.append(fk.ptr, fv.ptr, P + S)
    seqs.keep_suffix_from(P)
    st = seqs.state()
    assert (st.offset, st.base_offset, st.cached_len) == (P + S, P, S)
    seqs.attach_prefix(prefix)
    q = kv_bf16((B, Hq, 1, D), 45)
    got = decode(T, seqs, q, Hq, 0.1)
    want, _, _ = O.attend_affine(q, O.affine_quantize(full_k, 64, 8), O.affine_quantize(full_v, 64, 4),
                                 64, 8, 4, 0.1)
    check_close(got, want)
    # One more token per sequence lands in the suffix.
    nk, nv = kv_bf16((B, Hkv, 1, D), 46), kv_bf16((B, Hkv, 1, D), 47)
    dk, dv = T.DeviceArray.of(nk), T.DeviceArray.of(nv)
    seqs.append(dk.ptr, dv.ptr, 1)
    got = decode(T, seqs, q, Hq, 0.1)
    full_k = np.concatenate([full_k, nk], axis=2)
    full_v = np.concatenate([full_v, nv], axis=2)
    want, _, _ = O.attend_affine(q, O.affine_quantize(full_k, 64, 8), O.affine_quantize(full_v, 64, 4),
                                 64, 8, 4, 0.1)
    check_close(got, want)
    seqs.attach_prefix(None)
    prefix.close()


def attention_f64(q, K, V, scale, G):
    """Textbook softmax attention in f64: q [B,H,D], K/V [B,Hkv,N,D]."""
    B, H, D = q.shape
    out = np.zeros((B, H, D))
    for b in range(B):
        for h in range(H):
            s = (K[b, h // G] @ q[b, h]) * scale
            p = np.exp(s - s.max())
            out[b, h] = (p @ V[b, h // G]) / p.sum()
    return out


@pytest.mark.parametrize("bits,qjl_words", [(4, 2), (3, 0), (8, 0)])
def test_codebook_cache_append_and_decode(T, bits, qjl_words):
    # A rotating TurboQuant cache: bf16 K/V compressed on append (bit-exact
    # with compress_one), then decode attention over the codes in the rotated
    # basis, un-rotated, against attention over the dequantized cache.
    B, Hq, Hkv, D, W = 2, 8, 2, 128, 1024
    c = T.Cache(T.CACHE_CODEBOOK, B, Hkv, D, D, bits_k=bits, bits_v=bits, qjl_words=qjl_words,
                max_size=W, keep=0, seed=42)
    k = kv_bf16((B, Hkv, 300, D), 61, frac=0.02, mult=8.0)
    v = kv_bf16((B, Hkv, 300, D), 62, frac=0.02, mult=8.0)
    for a, s in [(0, 200), (200, 1), (201, 99)]:
        dk = T.DeviceArray.of(np.ascontiguousarray(k[:, :, a:a + s]))
        dv = T.DeviceArray.of(np.ascontiguousarray(v[:, :, a:a + s]))
        c.append(dk.ptr, dv.ptr, s)
    st = c.state()
    assert st.view == 300 and st.offset == 300
    R = T.rotation_matrix(D, 42)
    m = 32 * qjl_words
    phi = T.qjl_matrix(D, max(m, 1), 43)
    comp = O.Compressor(D, bits, max(m, 1), R, phi[:max(m, 1)])
    bufs = c.buffers()
    kc = T.view_slot(bufs, 0, B * Hkv, np.uint8, D)[:, :300]
    ks = T.view_slot(bufs, 1, B * Hkv, np.float32, 1)[:, :300, 0]
    vi = 4 if qjl_words else 2
    vc = T.view_slot(bufs, vi, B * Hkv, np.uint8, D)[:, :300]
    vsg = T.view_slot(bufs, vi + 1, B * Hkv, np.float32, 1)[:, :300, 0]
    kf = O.bf16_to_f32(k).reshape(-1, D)
    s1, s2, rn, sc = comp.compress(kf)
    assert np.array_equal(np.stack([O.pack_codes(r, bits) for r in kc.reshape(-1, D)]), s1)
    assert np.array_equal(ks.reshape(-1).view(np.uint32), sc.view(np.uint32))
    if qjl_words:
        sg = T.view_slot(bufs, 2, B * Hkv, np.uint32, qjl_words)[:, :300].reshape(-1, qjl_words)
        assert np.array_equal(sg, s2.view(np.uint32).reshape(len(kf), -1)[:, :qjl_words])
    _, cent = T.lloyd_max(bits)
    cent = cent.astype(np.float32).astype(np.float64)
    Kr = (cent[kc] * ks[..., None]).reshape(B, Hkv, 300, D)
    Vr = (cent[vc] * vsg[..., None]).reshape(B, Hkv, 300, D)
    q = kv_bf16((B, Hq, 1, D), 63)
    qf = O.bf16_to_f32(q).reshape(B, Hq, D).astype(np.float64)
    qr = qf @ R.astype(np.float64).T  # R q per head
    if qjl_words:
        # The keys' QJL residual signs correct every score (two-stage scores).
        ksg = T.view_slot(bufs, 2, B * Hkv, np.uint32, qjl_words)[:, :300]
        krn = T.view_slot(bufs, 3, B * Hkv, np.float32, 1)[:, :300, 0]
        _, centk = T.lloyd_max(bits)
        cf = centk.astype(np.float32)
        want = O.attend_codebook_qjl(q, kc.reshape(B, Hkv, 300, D), ks.reshape(B, Hkv, 300),
                                     ksg.reshape(B, Hkv, 300, qjl_words), krn.reshape(B, Hkv, 300),
                                     vc.reshape(B, Hkv, 300, D), vsg.reshape(B, Hkv, 300), cf, cf,
                                     R, phi[:m], m, D ** -0.5).astype(np.float64)
    else:
        want = attention_f64(qr, Kr, Vr, D ** -0.5, Hq // Hkv) @ R.astype(np.float64)  # R^T o
    got_b = decode(T, c, q, Hq, D ** -0.5).reshape(B, Hq, D)
    check_bf16(got_b, want, f"codebook-decode bits={bits}")
    got = O.bf16_to_f32(got_b)
    # A coarse sanity bar against attention over the unquantized K/V (the
    # output averages many values, so codebook noise weighs more in it than
    # in any one score).
    orig = attention_f64(qf, O.bf16_to_f32(k).astype(np.float64),
                         O.bf16_to_f32(v).astype(np.float64), D ** -0.5, Hq // Hkv)
    cos = (got.ravel() @ orig.ravel()) / (np.linalg.norm(got) * np.linalg.norm(orig))
    print(f"[codebook-decode] cos_vs_unquantized={cos:.4f}", flush=True)
    assert cos > {8: 0.995, 4: 0.9, 3: 0.85}[bits]


@pytest.mark.parametrize("B,Hkv,G,D,N,bits", [(16, 8, 2, 128, 2100, 3), (32, 4, 4, 64, 1500, 4),
                                              (2, 4, 2, 256, 1300, 3), (1, 2, 8, 256, 700, 4),
                                              (1, 1, 16, 256, 333, 3)])
def test_codebook_decode_direct(T, B, Hkv, G, D, N, bits):
    """tqkv_decode_attend_codebook on codes and sigmas it is handed, against
    f64 attention over centroid * sigma in the rotated basis, rotated back;
    128 or more (batch row, KV head) units take 1024-token splits, fewer take
    512."""
    H = G * Hkv
    rng = np.random.default_rng(B * 1000 + D + bits)
    kc = rng.integers(0, 1 << bits, size=(B, Hkv, N, D), dtype=np.uint8)
    vc = rng.integers(0, 1 << bits, size=(B, Hkv, N, D), dtype=np.uint8)
    ks = rng.uniform(0.5, 2.0, size=(B, Hkv, N)).astype(np.float32)
    vs = rng.uniform(0.5, 2.0, size=(B, Hkv, N)).astype(np.float32)
    q = kv_bf16((B, H, 1, D), 71 + D)
    R = T.rotation_matrix(D, 42)
    _, cent = T.lloyd_max(bits)
    cf = cent.astype(np.float32)
    d = {n: T.DeviceArray.of(a) for n, a in
         dict(q=q, kc=kc, vc=vc, ks=ks, vs=vs, R=R, c=cf).items()}
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    wsb = T.decode_codebook_workspace_size(B, H, D, N)
    ws = T.DeviceArray((wsb,), np.uint8)
    T.decode_attend_codebook(d["q"].ptr, B, H, Hkv, D, D ** -0.5, d["R"].ptr, d["c"].ptr, bits,
                             d["c"].ptr, bits, d["kc"].ptr, d["ks"].ptr, d["vc"].ptr, d["vs"].ptr,
                             N, N, out.ptr, ws.ptr, wsb)
    T.hip().sync()
    c64 = cf.astype(np.float64)
    Kr = c64[kc] * ks[..., None]
    Vr = c64[vc] * vs[..., None]
    qr = O.bf16_to_f32(q).reshape(B, H, D).astype(np.float64) @ R.astype(np.float64).T
    want = attention_f64(qr, Kr, Vr, D ** -0.5, G) @ R.astype(np.float64)
    check_bf16(out.numpy().reshape(B, H, D), want, f"codebook-direct B={B} Hkv={Hkv} D={D}")


def test_codebook_decode_rejects_unaligned_values(T):
    """A lane loads its value codes 4 bytes at a time at D = 256: a value
    code pointer off that alignment is refused before any launch."""
    B, Hkv, H, D, N = 1, 1, 2, 256, 64
    q = T.DeviceArray((B, H, 1, D), np.uint16)
    codes = T.DeviceArray((N * D + 4,), np.uint8)
    sig = T.DeviceArray((N,), np.float32)
    R = T.DeviceArray.of(T.rotation_matrix(D, 42))
    cent = T.DeviceArray.of(T.lloyd_max(3)[1].astype(np.float32))
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    with pytest.raises(T.TqkvError) as e:
        T.decode_attend_codebook(q.ptr, B, H, Hkv, D, 1.0, R.ptr, cent.ptr, 3, cent.ptr, 3,
                                 codes.ptr, sig.ptr, codes.ptr + 1, sig.ptr, N, N, out.ptr)
    assert e.value.status == T.EINVAL_ARG


def test_codebook_decode_rejects_unaligned_keys(T):
    """Key rows are read 16 bytes a load: a key code pointer off that
    alignment is refused before any launch (values aligned)."""
    B, Hkv, H, D, N = 1, 1, 2, 128, 64
    q = T.DeviceArray((B, H, 1, D), np.uint16)
    codes = T.DeviceArray((N * D + 16,), np.uint8)
    sig = T.DeviceArray((N,), np.float32)
    R = T.DeviceArray.of(T.rotation_matrix(D, 42))
    cent = T.DeviceArray.of(T.lloyd_max(3)[1].astype(np.float32))
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    for off in (2, 8):
        with pytest.raises(T.TqkvError) as e:
            T.decode_attend_codebook(q.ptr, B, H, Hkv, D, 1.0, R.ptr, cent.ptr, 3, cent.ptr, 3,
                                     codes.ptr + off, sig.ptr, codes.ptr, sig.ptr, N, N, out.ptr)
        assert e.value.status == T.EINVAL_ARG
