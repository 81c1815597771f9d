"""tqkv_decode_attend_affine_noalloc, the decode entry that allocates nothing
(its split partials live in the library's static device scratch), against
tqkv_decode_attend_affine given a workspace of its own: outputs bit-identical
(same kernels, same split plan) and within the decode bar of the oracle, on
two calls in a row with the second smaller, for the split-and-merge path, the
shared-prefix path and the one-split path; a call whose partials would not
fit the static scratch is refused with TQKV_EINVAL_SHAPE."""
import numpy as np
import pytest

import oracle_lib as O
from inputs import kv_bf16
from test_gpu_affine import _cache, check_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def T():
    import tqkv
    assert tqkv.hip().device_count() > 0, "no GPU visible"
    return tqkv


def both(T, q, segs_host, B, H, Hkv, D, bk, bv, scale, total):
    dq = T.DeviceArray.of(q)
    segs = [T.affine_seg(tuple(a.ptr for a in k), tuple(a.ptr for a in v), cap, n, sh)
            for (k, v, cap, n, sh) in segs_host]
    o1 = T.DeviceArray((B, H, 1, D), np.uint16, np.zeros((B, H, 1, D), np.uint16))
    o2 = T.DeviceArray((B, H, 1, D), np.uint16, np.full((B, H, 1, D), 0x7FC0, np.uint16))
    wsb = T.decode_workspace_size(B, H, Hkv, D, total)
    ws = T.DeviceArray((max(wsb, 1),), np.uint8)
    T.decode_attend_affine(dq.ptr, B, H, Hkv, D, 64, bk, bv, scale, segs, o1.ptr, ws.ptr, wsb)
    T.decode_attend_affine_noalloc(dq.ptr, B, H, Hkv, D, 64, bk, bv, scale, segs, o2.ptr)
    T.hip().sync()
    return o1.numpy(), o2.numpy()


@pytest.mark.parametrize("B,H,Hkv,D,bits,sizes", [
    (1, 32, 8, 128, 4, (3000, 700)),    # config 1's layout: splits + merge
    (32, 16, 8, 256, 3, (600, 200)),    # config 2's layout: one split, no partials
    (2, 16, 4, 64, 8, (1500, 65)),
])
def test_noalloc_matches_workspace_entry(T, B, H, Hkv, D, bits, sizes):
    for i, N in enumerate(sizes):
        print(f"[noalloc] B={B} H={H}/{Hkv} D={D} bits={bits} N={N} call={i}", flush=True)
        q = kv_bf16((B, H, 1, D), 90 + i)
        k = kv_bf16((B, Hkv, N, D), 91 + i, frac=0.01, mult=10.0)
        v = kv_bf16((B, Hkv, N, D), 92 + i, frac=0.01, mult=10.0)
        (kh, kd), (vh, vd) = _cache(k, 64, bits, N + 9), _cache(v, 64, bits, N + 9)
        ref, got = both(T, q, [(kd, vd, N + 9, N, False)], B, H, Hkv, D, bits, bits, D ** -0.5,
                        N + 9)
        assert np.array_equal(got, ref), "no-allocation entry differs from the workspace entry"
        want, _, _ = O.attend_affine(q, kh, vh, 64, bits, bits, D ** -0.5)
        check_close(got, want)


def test_noalloc_holds_no_library_scratch(T):
    """What the entry is for: on a shape that splits (config 1's layout, ~32
    splits a unit, so partials and a merge) it allocates nothing: with the
    library's scratch released first, the call leaves it empty. The same
    decode through the workspace-less entry then does allocate scratch (the
    check can see an allocation)."""
    B, H, Hkv, D, bits, N = 1, 32, 8, 128, 4, 8192
    q = kv_bf16((B, H, 1, D), 301)
    k = kv_bf16((B, Hkv, N, D), 302, frac=0.01, mult=10.0)
    v = kv_bf16((B, Hkv, N, D), 303, frac=0.01, mult=10.0)
    (kh, kd), (vh, vd) = _cache(k, 64, bits, N), _cache(v, 64, bits, N)
    dq = T.DeviceArray.of(q)
    segs = [T.affine_seg(tuple(a.ptr for a in kd), tuple(a.ptr for a in vd), N, N)]
    o1 = T.DeviceArray((B, H, 1, D), np.uint16)
    o2 = T.DeviceArray((B, H, 1, D), np.uint16)
    T.hip().sync()
    T.scratch_release()
    assert T.scratch_bytes() == 0
    T.decode_attend_affine_noalloc(dq.ptr, B, H, Hkv, D, 64, bits, bits, D ** -0.5, segs, o1.ptr)
    T.hip().sync()
    assert T.scratch_bytes() == 0, "the no-allocation entry created library scratch"
    T.decode_attend_affine(dq.ptr, B, H, Hkv, D, 64, bits, bits, D ** -0.5, segs, o2.ptr)
    T.hip().sync()
    assert T.scratch_bytes() > 0, "this shape should split and use scratch"
    assert np.array_equal(o1.numpy(), o2.numpy())
    T.scratch_release()


def test_noalloc_shared_prefix(T):
    # A prefix stored once for every sequence (read once per KV head) plus
    # each sequence's suffix: prefix partials, suffix partials, one merge.
    H, Hkv, D, bk, bv = 32, 8, 128, 8, 4
    for i, (B, P, S) in enumerate(((4, 2000, 70), (2, 500, 9))):
        print(f"[noalloc shared] B={B} P={P} S={S} call={i}", flush=True)
        q = kv_bf16((B, H, 1, D), 40 + i)
        kp, vp = kv_bf16((1, Hkv, P, D), 41 + i), kv_bf16((1, Hkv, P, D), 42 + i)
        ks, vs = kv_bf16((B, Hkv, S, D), 43 + i), kv_bf16((B, Hkv, S, D), 44 + i)
        (kph, kpd), (vph, vpd) = _cache(kp, 64, bk), _cache(vp, 64, bv)
        (ksh, ksd), (vsh, vsd) = _cache(ks, 64, bk, S + 2), _cache(vs, 64, bv, S + 2)
        segs = [(kpd, vpd, P, P, True), (ksd, vsd, S + 2, S, False)]
        ref, got = both(T, q, segs, B, H, Hkv, D, bk, bv, D ** -0.5, P + S + 2)
        assert np.array_equal(got, ref)
        cat = lambda a, b: np.concatenate([np.broadcast_to(a, (B,) + a.shape[1:]), b], axis=2)
        want, _, _ = O.attend_affine(q, tuple(cat(a, b) for a, b in zip(kph, ksh)),
                                     tuple(cat(a, b) for a, b in zip(vph, vsh)), 64, bk, bv,
                                     D ** -0.5)
        check_close(got, want)


def test_noalloc_refuses_oversize(T):
    # 1,024 sequences over a shared prefix: prefix and suffix partials for
    # 32,768 query rows pass the 32 MiB static scratch; the call is refused
    # before any launch (the buffers are real, so nothing reads out of bounds).
    B, H, Hkv, D, P, S = 1024, 32, 8, 128, 64, 64
    q = T.DeviceArray((B, H, 1, D), np.uint16, np.zeros((B, H, 1, D), np.uint16))
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    kp = tuple(T.DeviceArray((Hkv, P, w), dt) for dt, w in ((np.uint32, 16), (np.uint16, 2),
                                                              (np.uint16, 2)))
    ks = tuple(T.DeviceArray((B * Hkv, S, w), dt) for dt, w in ((np.uint32, 16), (np.uint16, 2),
                                                                  (np.uint16, 2)))
    segs = [T.affine_seg(tuple(a.ptr for a in kp), tuple(a.ptr for a in kp), P, P, True),
            T.affine_seg(tuple(a.ptr for a in ks), tuple(a.ptr for a in ks), S, S)]
    with pytest.raises(T.TqkvError) as e:
        T.decode_attend_affine_noalloc(q.ptr, B, H, Hkv, D, 64, 4, 4, 0.1, segs, out.ptr)
    assert e.value.status == T.EINVAL_SHAPE
    assert "static scratch" in str(e.value)
