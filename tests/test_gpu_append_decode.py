"""A decode step in one kernel: tqkv_cache_append_decode and
tqkv_decode_attend_affine_append, the reference's update_and_fetch of one
token followed by quantized_decode_attention over the fetched view
(gemma4_moe.rs:4081, 4125).

Each case drives two caches with the same tokens: one through the fused
entry, one through tqkv_cache_append + tqkv_cache_decode_attend. After every
step the two caches' buffers must be bit-identical (the in-kernel quantize is
mlx::quantize, as the append kernel's), and both outputs must be within the
decode bar (2e-2 max-abs, 1e-3 mean-abs) of the oracle's
dequantize-then-attend over the tokens the reference's cache holds: growing
from empty and across the 256-row growth steps, a rotating window written in
place mid-ring, a shared prefix (with an empty and a non-empty suffix), a
batch-1 prefix, and a layout the fused kernel does not serve (two calls).
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


def slots_of(c, B, Hkv, D, gs, bk, bv):
    import tqkv
    v = c.buffers()
    ng = D // gs
    spec = [(np.uint32, D * bk // 32), (np.uint16, ng), (np.uint16, ng),
            (np.uint32, D * bv // 32), (np.uint16, ng), (np.uint16, ng)]
    return [tqkv.view_slot(v, i, B * Hkv, dt, last) for i, (dt, last) in enumerate(spec)]


def same_bytes(T, a, b, shape):
    sa, sb = slots_of(a, *shape), slots_of(b, *shape)
    for i, (x, y) in enumerate(zip(sa, sb)):
        assert x.shape == y.shape and np.array_equal(x, y), f"slot {i} differs"


class Twin:
    """The same token stream through the fused entry and the two calls."""

    def __init__(self, T, B, Hkv, D, bk, bv, gs=64, **kw):
        self.T, self.shape = T, (B, Hkv, D, gs, bk, bv)
        self.fused = T.Cache(T.CACHE_AFFINE, B, Hkv, D, D, gs, bk, bv, **kw)
        self.split = T.Cache(T.CACHE_AFFINE, B, Hkv, D, D, gs, bk, bv, **kw)

    def append(self, k, v):
        dk, dv = self.T.DeviceArray.of(k), self.T.DeviceArray.of(v)
        for c in (self.fused, self.split):
            c.append(dk.ptr, dv.ptr, k.shape[2])

    def step(self, k, v, q, H, scale):
        T = self.T
        dk, dv, dq = T.DeviceArray.of(k), T.DeviceArray.of(v), T.DeviceArray.of(q)
        o1, o2 = T.DeviceArray(q.shape, np.uint16), T.DeviceArray(q.shape, np.uint16)
        self.fused.append_decode(dk.ptr, dv.ptr, dq.ptr, H, scale, o1.ptr)
        self.split.append(dk.ptr, dv.ptr, 1)
        self.split.decode_attend(dq.ptr, H, scale, o2.ptr)
        T.hip().sync()
        s1, s2 = self.fused.state(), self.split.state()
        assert (s1.offset, s1.idx, s1.cached_len, s1.view) == \
            (s2.offset, s2.idx, s2.cached_len, s2.view)
        same_bytes(T, self.fused, self.split, self.shape)
        return o1.numpy(), o2.numpy()


def check_close(got_bf16, want_f32):
    check_bf16(got_bf16, want_f32, "append-decode")


def want_of(q, K, V, gs, bk, bv, scale):
    want, _, _ = O.attend_affine(q, O.affine_quantize(K, gs, bk), O.affine_quantize(V, gs, bv),
                                 gs, bk, bv, scale)
    return want


@pytest.mark.parametrize("B,Hq,Hkv,D,bk,bv,prefill,steps,prealloc,gs", [
    (1, 32, 8, 128, 4, 4, 0, 3, True, 64),      # config 1's layout, from empty
    (2, 16, 8, 256, 3, 3, 254, 4, False, 64),   # config 2's layout, across 256 (growth copy)
    (2, 32, 8, 128, 8, 4, 500, 2, True, 64),    # config 4's widths
    (3, 8, 4, 64, 4, 8, 63, 3, True, 64),       # D = 64, mixed widths
    (1, 32, 8, 128, 6, 6, 100, 2, True, 64),    # 6-bit (MFMA kernel at D = 128)
    (2, 16, 8, 128, 2, 2, 30, 2, False, 64),    # 2-bit
    (1, 16, 8, 256, 4, 4, 100, 3, True, 32),    # group size 32 (16 A rows)
    (2, 32, 8, 128, 6, 6, 40, 2, True, 32),     # group size 32, 4 heads a KV head
    (1, 16, 8, 128, 8, 4, 70, 2, True, 128),    # group size 128
    (1, 32, 2, 128, 4, 4, 50, 2, True, 64),     # 16 heads a KV head: two launches
    (1, 64, 8, 256, 4, 4, 60, 2, True, 64),     # 8 heads at D = 256: two MFMA launches
])
def test_growing(T, B, Hq, Hkv, D, bk, bv, prefill, steps, prealloc, gs):
    assert T.decode_kernel_name(Hq, Hkv, D, gs, bk, bv) == "mfma"
    tw = Twin(T, B, Hkv, D, bk, bv, gs=gs, prealloc=prealloc)
    ks, vs = [], []
    if prefill:
        k = kv_bf16((B, Hkv, prefill, D), 1, frac=0.02, mult=8.0)
        v = kv_bf16((B, Hkv, prefill, D), 2, frac=0.02, mult=8.0)
        tw.append(k, v)
        ks.append(k)
        vs.append(v)
    scale = D ** -0.5
    for i in range(steps):
        k = kv_bf16((B, Hkv, 1, D), 10 + i, frac=0.02, mult=8.0)
        v = kv_bf16((B, Hkv, 1, D), 20 + i, frac=0.02, mult=8.0)
        q = kv_bf16((B, Hq, 1, D), 30 + i)
        ks.append(k)
        vs.append(v)
        got, ref = tw.step(k, v, q, Hq, scale)
        K, V = np.concatenate(ks, axis=2), np.concatenate(vs, axis=2)
        want = want_of(q, K, V, gs, bk, bv, scale)
        print(f"[append-decode] B={B} D={D} bits={bk}/{bv} gs={gs} step={i} keys={K.shape[2]}",
              flush=True)
        check_close(got, want)
        check_close(ref, want)


def test_rotating_in_place(T):
    # A 96-token window with 4 sinks: once it wraps, each step overwrites a
    # slot mid-ring, which the fused path leaves out of both segments.
    B, Hq, Hkv, D, W, KEEP = 2, 16, 4, 128, 96, 4
    tw = Twin(T, B, Hkv, D, 4, 4, max_size=W, keep=KEEP)
    k_all = kv_bf16((B, Hkv, 140, D), 51, frac=0.02, mult=8.0)
    v_all = kv_bf16((B, Hkv, 140, D), 52, frac=0.02, mult=8.0)
    tw.append(np.ascontiguousarray(k_all[:, :, :90]), np.ascontiguousarray(v_all[:, :, :90]))
    for pos in range(90, 140):
        q = kv_bf16((B, Hq, 1, D), 100 + pos)
        got, ref = tw.step(np.ascontiguousarray(k_all[:, :, pos:pos + 1]),
                           np.ascontiguousarray(v_all[:, :, pos:pos + 1]), q, Hq, 0.09)
        n = pos + 1
        if n in (91, 96, 97, 98, 120, 140):
            held = list(range(n)) if n <= W else list(range(KEEP)) + list(range(n - (W - KEEP), n))
            K = np.ascontiguousarray(k_all[:, :, held])
            V = np.ascontiguousarray(v_all[:, :, held])
            st = tw.fused.state()
            print(f"[append-decode ring] n={n} idx={st.idx} view={st.view}", flush=True)
            want = want_of(q, K, V, 64, 4, 4, 0.09)
            check_close(got, want)
            check_close(ref, want)
    

@pytest.mark.parametrize("B,S", [(3, 0), (3, 40), (1, 17)])
def test_shared_prefix(T, B, S):
    # Sequences share a prefix cache (B >= 2: the prefix is read once for all
    # of them); S = 0 starts from an empty suffix.
    Hq, Hkv, D, P = 16, 4, 128, 520
    pre_k = kv_bf16((1, Hkv, P, D), 61)
    pre_v = kv_bf16((1, Hkv, P, D), 62)
    suf_k = kv_bf16((B, Hkv, S, D), 63)
    suf_v = kv_bf16((B, Hkv, S, D), 64)
    prefix = T.Cache(T.CACHE_AFFINE, 1, Hkv, D, D, 64, 8, 4)
    a, b = T.DeviceArray.of(pre_k), T.DeviceArray.of(pre_v)
    prefix.append(a.ptr, b.ptr, P)
    tw = Twin(T, B, Hkv, D, 8, 4)
    full_k = np.concatenate([np.broadcast_to(pre_k, (B, Hkv, P, D)), suf_k], axis=2)
    full_v = np.concatenate([np.broadcast_to(pre_v, (B, Hkv, P, D)), suf_v], axis=2)
    tw.append(np.ascontiguousarray(full_k), np.ascontiguousarray(full_v))
    for c in (tw.fused, tw.split):
        c.keep_suffix_from(P)
        c.attach_prefix(prefix)
    for i in range(3):
        nk, nv = kv_bf16((B, Hkv, 1, D), 70 + i), kv_bf16((B, Hkv, 1, D), 80 + i)
        q = kv_bf16((B, Hq, 1, D), 90 + i)
        got, ref = tw.step(nk, nv, q, Hq, 0.1)
        full_k = np.concatenate([full_k, nk], axis=2)
        full_v = np.concatenate([full_v, nv], axis=2)
        print(f"[append-decode prefix] B={B} S={S} step={i}", flush=True)
        want = want_of(q, full_k, full_v, 64, 8, 4, 0.1)
        check_close(got, want)
        check_close(ref, want)
    for c in (tw.fused, tw.split):
        c.attach_prefix(None)
    prefix.close()


def test_layout_without_fused_kernel(T, monkeypatch):
    # The dot2 kernel does not quantize in place: the fused entry falls back
    # to the two calls (same bytes, same bar), and the kernel entry refuses.
    monkeypatch.setenv("TQKV_DECODE_KERNEL", "dot2")
    B, Hq, Hkv, D = 2, 8, 2, 128
    tw = Twin(T, B, Hkv, D, 4, 4)
    k0 = kv_bf16((B, Hkv, 70, D), 3)
    v0 = kv_bf16((B, Hkv, 70, D), 4)
    tw.append(k0, v0)
    k, v, q = kv_bf16((B, Hkv, 1, D), 5), kv_bf16((B, Hkv, 1, D), 6), kv_bf16((B, Hq, 1, D), 7)
    got, ref = tw.step(k, v, q, Hq, 0.08)
    want = want_of(q, np.concatenate([k0, k], axis=2), np.concatenate([v0, v], axis=2),
                   64, 4, 4, 0.08)
    check_close(got, want)
    check_close(ref, want)
    seg = T.AffineSeg()
    dk, dv, dq = T.DeviceArray.of(k), T.DeviceArray.of(v), T.DeviceArray.of(q)
    out = T.DeviceArray(q.shape, np.uint16)
    bufs = tw.fused.buffers()
    with pytest.raises(T.TqkvError):
        T.decode_attend_affine_append(dq.ptr, B, Hq, Hkv, D, 64, 4, 4, 0.08, [seg], dk.ptr, dv.ptr,
                                      [bufs.slot[i] for i in range(6)], bufs.cap, 0, out.ptr)


def test_kernel_entry_row_mid_buffer(T):
    # The kernel entry on raw buffers: rows [0, 37) already quantized, the new
    # row written at 37 of a 64-row slab, attended over [0, 37) + the new row;
    # the written bytes equal tqkv_affine_quantize_kv's.
    B, Hq, Hkv, D, bk, bv, CAP, N = 2, 16, 8, 256, 3, 3, 64, 37
    kr, vr, ng = D * bk // 32, D * bv // 32, D // 64
    K0 = kv_bf16((B, Hkv, N, D), 11, frac=0.01, mult=10.0)
    V0 = kv_bf16((B, Hkv, N, D), 12, frac=0.01, mult=10.0)
    k = kv_bf16((B, Hkv, 1, D), 13, frac=0.01, mult=10.0)
    v = kv_bf16((B, Hkv, 1, D), 14, frac=0.01, mult=10.0)
    q = kv_bf16((B, Hq, 1, D), 15)

    def bufs():
        return [T.DeviceArray((B * Hkv, CAP, kr), np.uint32),
                T.DeviceArray((B * Hkv, CAP, ng), np.uint16),
                T.DeviceArray((B * Hkv, CAP, ng), np.uint16),
                T.DeviceArray((B * Hkv, CAP, vr), np.uint32),
                T.DeviceArray((B * Hkv, CAP, ng), np.uint16),
                T.DeviceArray((B * Hkv, CAP, ng), np.uint16)]

    fused, plain = bufs(), bufs()
    dK0, dV0, dk, dv = (T.DeviceArray.of(x) for x in (K0, V0, k, v))
    def trip(bb, i):
        return tuple(x.ptr for x in bb[3 * i:3 * i + 3])

    for bb in (fused, plain):
        for x in bb:
            T.hip().copy_in(x.ptr, np.zeros(x.shape, x.dtype))
        T.affine_quantize_kv(dK0.ptr, dV0.ptr, B * Hkv, N, D, 64, bk, bv, trip(bb, 0),
                             trip(bb, 1), CAP, 0)
    T.affine_quantize_kv(dk.ptr, dv.ptr, B * Hkv, 1, D, 64, bk, bv, trip(plain, 0),
                         trip(plain, 1), CAP, N)
    seg = T.AffineSeg(*[x.ptr for x in fused], CAP, N, 0, 0)
    dq = T.DeviceArray.of(q)
    out = T.DeviceArray(q.shape, np.uint16)
    T.decode_attend_affine_append(dq.ptr, B, Hq, Hkv, D, 64, bk, bv, 0.0625, [seg], dk.ptr,
                                  dv.ptr, [x.ptr for x in fused], CAP, N, out.ptr)
    T.hip().sync()
    for i, (x, y) in enumerate(zip(fused, plain)):
        assert np.array_equal(x.numpy(), y.numpy()), f"buffer {i} differs"
    want = want_of(q, np.concatenate([K0, k], axis=2), np.concatenate([V0, v], axis=2),
                   64, bk, bv, 0.0625)
    check_close(out.numpy(), want)


def test_single_split_with_append(T, monkeypatch):
    # One split a unit (the headline's launch shape: no partials, the output
    # normalized in the kernel) with the new token quantized in the kernel,
    # across a growth step, against the two calls and the oracle.
    monkeypatch.setenv("TQKV_DECODE_SPLITS", "1")
    B, Hq, Hkv, D, bits = 2, 16, 8, 256, 3
    tw = Twin(T, B, Hkv, D, bits, bits, prealloc=True)
    k0 = kv_bf16((B, Hkv, 509, D), 41, frac=0.01, mult=10.0)
    v0 = kv_bf16((B, Hkv, 509, D), 42, frac=0.01, mult=10.0)
    tw.append(k0, v0)
    ks, vs = [k0], [v0]
    for i in range(4):  # rows 509-512: the last crosses the 512-row buffer
        k = kv_bf16((B, Hkv, 1, D), 43 + i, frac=0.01, mult=10.0)
        v = kv_bf16((B, Hkv, 1, D), 53 + i, frac=0.01, mult=10.0)
        q = kv_bf16((B, Hq, 1, D), 63 + i)
        ks.append(k)
        vs.append(v)
        got, ref = tw.step(k, v, q, Hq, D ** -0.5)
        K, V = np.concatenate(ks, axis=2), np.concatenate(vs, axis=2)
        print(f"[append-decode 1split] step={i} keys={K.shape[2]}", flush=True)
        want = want_of(q, K, V, 64, bits, bits, D ** -0.5)
        check_close(got, want)
        check_close(ref, want)


def test_failed_decode_leaves_cache_unchanged(T):
    # A decode step whose workspace is too small for its split partials must
    # fail before the cache counts the token: state and bytes as before, and
    # the same step then succeeds with room (tqkv_cache_append_decode).
    B, Hq, Hkv, D, bits = 1, 32, 8, 128, 4
    tw = Twin(T, B, Hkv, D, bits, bits, prealloc=True)
    k0 = kv_bf16((B, Hkv, 3000, D), 71)
    v0 = kv_bf16((B, Hkv, 3000, D), 72)
    tw.append(k0, v0)
    before = tw.fused.state()
    bytes_before = slots_of(tw.fused, B, Hkv, D, 64, bits, bits)
    k, v, q = kv_bf16((B, Hkv, 1, D), 73), kv_bf16((B, Hkv, 1, D), 74), kv_bf16((B, Hq, 1, D), 75)
    dk, dv, dq = T.DeviceArray.of(k), T.DeviceArray.of(v), T.DeviceArray.of(q)
    out = T.DeviceArray(q.shape, np.uint16)
    small = T.DeviceArray((16,), np.uint8)
    with pytest.raises(T.TqkvError) as e:
        tw.fused.append_decode(dk.ptr, dv.ptr, dq.ptr, Hq, D ** -0.5, out.ptr, small.ptr, 16)
    assert e.value.status == T.EINVAL_ARG
    T.hip().sync()
    after = tw.fused.state()
    assert (after.offset, after.idx, after.cached_len, after.view) == \
        (before.offset, before.idx, before.cached_len, before.view)
    for i, (x, y) in enumerate(zip(bytes_before, slots_of(tw.fused, B, Hkv, D, 64, bits, bits))):
        assert np.array_equal(x, y), f"slot {i} changed"
    got, ref = tw.step(k, v, q, Hq, D ** -0.5)
    want = want_of(q, np.concatenate([k0, k], axis=2), np.concatenate([v0, v], axis=2),
                   64, bits, bits, D ** -0.5)
    check_close(got, want)
    check_close(ref, want)
