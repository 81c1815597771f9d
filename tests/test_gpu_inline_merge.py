"""The in-kernel merge of a split decode (TQKV_INLINE_MERGE=1: the last
workgroup of each (batch row, KV head) merges its split partials; no merge
launch) against the merge launch (the default): the same bits on split
decodes of both kernels, the dot2 kernel's two-launch head split, and the
shared-prefix path; with a workspace that starts as garbage (every partial
slot a merge reads is written first), reused call after call (the unit
counters return to zero), and with the library's own scratch. The other
decode tests check the merge launch's output against the oracle."""
import numpy as np
import pytest

import oracle_lib as O
from inputs import kv_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def T():
    import tqkv
    assert tqkv.hip().device_count() > 0, "no GPU visible"
    return tqkv


def _triple(T, x, gs, bits, cap):
    B, Hkv, N, D = x.shape
    out = []
    for a in O.affine_quantize(x, gs, bits):
        pad = np.zeros((B, Hkv, cap, a.shape[-1]), a.dtype)
        pad[:, :, :N] = a
        out.append(T.DeviceArray.of(pad))
    return tuple(out)


def _decode(T, dq, segs, B, H, Hkv, D, gs, bk, bv, ws=None, wsb=0):
    out = T.DeviceArray((B, H, 1, D), np.uint16, np.zeros((B, H, 1, D), np.uint16))
    T.decode_attend_affine(dq.ptr, B, H, Hkv, D, gs, bk, bv, D ** -0.5, segs, out.ptr,
                           None if ws is None else ws.ptr, wsb)
    T.hip().sync()
    return out.numpy()


CASES = [
    # (B, H, Hkv, D, N, bits_k, bits_v, kernel)
    (1, 32, 8, 128, 8192, 4, 4, "mfma"),    # config 1's split decode
    (2, 16, 8, 256, 3000, 3, 3, "mfma"),
    (1, 32, 8, 128, 6000, 8, 4, "dot2"),
    (1, 48, 8, 128, 5000, 3, 3, "dot2"),    # 6 heads a KV head: two launches of 3
]


@pytest.mark.parametrize("B,H,Hkv,D,N,bk,bv,kernel", CASES)
def test_inline_merge_matches_merge_launch(T, monkeypatch, B, H, Hkv, D, N, bk, bv, kernel):
    print(f"[inline-merge] B={B} H={H}/{Hkv} D={D} N={N} bits={bk}/{bv} {kernel}", flush=True)
    if kernel == "dot2":
        monkeypatch.setenv("TQKV_DECODE_KERNEL", "dot2")
    else:
        monkeypatch.delenv("TQKV_DECODE_KERNEL", raising=False)
    gs = 64
    q = kv_bf16((B, H, 1, D), 7000 + N)
    k = kv_bf16((B, Hkv, N, D), 7001 + N, frac=0.01, mult=10.0)
    v = kv_bf16((B, Hkv, N, D), 7002 + N, frac=0.01, mult=10.0)
    kt, vt = _triple(T, k, gs, bk, N), _triple(T, v, gs, bv, N)
    segs = [T.affine_seg(tuple(a.ptr for a in kt), tuple(a.ptr for a in vt), N, N)]
    dq = T.DeviceArray.of(q)
    wsb = T.decode_workspace_size(B, H, Hkv, D, N)
    monkeypatch.delenv("TQKV_INLINE_MERGE", raising=False)
    want = _decode(T, dq, segs, B, H, Hkv, D, gs, bk, bv,
                   T.DeviceArray((wsb,), np.uint8, np.zeros(wsb, np.uint8)), wsb)
    monkeypatch.setenv("TQKV_INLINE_MERGE", "1")
    garbage = T.DeviceArray((wsb,), np.uint8, np.full(wsb, 0xFF, np.uint8))
    for rep in range(3):
        got = _decode(T, dq, segs, B, H, Hkv, D, gs, bk, bv, garbage, wsb)
        assert np.array_equal(got, want), f"call {rep} with the reused workspace"
    assert np.array_equal(_decode(T, dq, segs, B, H, Hkv, D, gs, bk, bv), want), "library scratch"


def test_inline_merge_shared_prefix(T, monkeypatch):
    """The shared-prefix path: the prefix pass writes its slots, the suffix
    launch's last workgroup of each unit merges prefix and suffix slots."""
    B, H, Hkv, D, P, S, gs, bk, bv = 4, 16, 4, 128, 4096, 700, 64, 8, 4
    print(f"[inline-merge-shared] B={B} P={P} S={S}", flush=True)
    q = kv_bf16((B, H, 1, D), 7100)
    kp = kv_bf16((1, Hkv, P, D), 7101)
    vp = kv_bf16((1, Hkv, P, D), 7102)
    ks = kv_bf16((B, Hkv, S, D), 7103)
    vs = kv_bf16((B, Hkv, S, D), 7104)
    pk, pv = _triple(T, kp, gs, bk, P), _triple(T, vp, gs, bv, P)
    sk, sv = _triple(T, ks, gs, bk, S), _triple(T, vs, gs, bv, S)
    segs = [T.affine_seg(tuple(a.ptr for a in pk), tuple(a.ptr for a in pv), P, P, True),
            T.affine_seg(tuple(a.ptr for a in sk), tuple(a.ptr for a in sv), S, S)]
    dq = T.DeviceArray.of(q)
    wsb = T.decode_workspace_size(B, H, Hkv, D, P + S)
    monkeypatch.delenv("TQKV_INLINE_MERGE", raising=False)
    want = _decode(T, dq, segs, B, H, Hkv, D, gs, bk, bv)
    monkeypatch.setenv("TQKV_INLINE_MERGE", "1")
    garbage = T.DeviceArray((wsb,), np.uint8, np.full(wsb, 0xA5, np.uint8))
    for rep in range(2):
        assert np.array_equal(_decode(T, dq, segs, B, H, Hkv, D, gs, bk, bv, garbage, wsb), want)
