"""LKV2 snapshots of device caches (tqkv_lkv_export / tqkv_lkv_import) on the
GPU: every cache kind is filled through appends (crossing growth steps and
ring wrap-around), exported, read back by an independent Python reader
(struct + zlib), checked against the reference's layer layout
(gemma4_moe.rs:1617-1693, kv_disk.rs:2005-2025) and the cache's own
buffers, imported into a new cache, and then shown to be the same cache:
identical state, identical bytes, identical decode attention, and identical
behaviour under further appends.
"""
import numpy as np
import pytest

import lkv_py as L
from inputs import kv_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def T():
    import tqkv
    assert tqkv.hip().device_count() > 0, "no GPU visible"
    return tqkv


def download_slots(T, c, n_slabs):
    v = c.buffers()
    return [T.view_slot(v, i, n_slabs, np.uint8, v.row_bytes[i]) for i in range(v.n_slots)]


def fill(T, c, B, Hkv, D, chunks, seed):
    for i, s in enumerate(chunks):
        k = kv_bf16((B, Hkv, s, D), seed + 2 * i, frac=0.02, mult=8.0)
        v = kv_bf16((B, Hkv, s, D), seed + 2 * i + 1, frac=0.02, mult=8.0)
        dk, dv = T.DeviceArray.of(k), T.DeviceArray.of(v)
        c.append(dk.ptr, dv.ptr, s)
    T.hip().sync()


CASES = [
    # (name, kind, kwargs, D, chunks)
    ("bf16-growing", "BF16", {}, 64, [300, 1, 1, 2]),
    ("bf16-ring", "BF16", dict(max_size=96, keep=4), 64, [40, 70] + [1] * 30),
    ("affine-growing", "AFFINE", dict(bits_k=4, bits_v=4), 128, [300, 1, 7]),
    ("affine-k8v4", "AFFINE", dict(bits_k=8, bits_v=4), 128, [257, 1]),
    ("affine-ring", "AFFINE", dict(bits_k=3, bits_v=3, max_size=128, keep=0), 256,
     [200, 1, 1, 64] + [1] * 40),
    ("codebook-qjl", "CODEBOOK", dict(bits_k=3, bits_v=3, qjl_words=2, max_size=160), 128,
     [100, 90, 1, 1]),
    ("codebook", "CODEBOOK", dict(bits_k=4, bits_v=4, max_size=64, keep=2), 64, [50] + [1] * 30),
]

KINDS = {"Full", "Sliding", "FullQuantized", "SlidingQuantized", "SlidingTurboquant"}


def make(T, kind, kw, B, Hkv, D):
    gs = 64 if D >= 64 else 32
    return T.Cache(getattr(T, "CACHE_" + kind), B, Hkv, D, D, gs, kw.get("bits_k", 4),
                   kw.get("bits_v", 4), qjl_words=kw.get("qjl_words", 0), prealloc=True,
                   max_size=kw.get("max_size", 0), keep=kw.get("keep", 0), seed=42)


@pytest.mark.parametrize("name,kind,kw,D,chunks", CASES, ids=[c[0] for c in CASES])
def test_export_import_round_trip(T, name, kind, kw, D, chunks):
    B, Hkv, Hq = 2, 2, 4
    print(f"[lkv] {name} D={D} chunks={len(chunks)}", flush=True)
    c = make(T, kind, kw, B, Hkv, D)
    fill(T, c, B, Hkv, D, chunks, 11)
    st = c.state()
    blob = T.lkv_export([c], fingerprint="tqkv-test", created_at_unix=123, position=st.offset,
                        prefix_tokens=[7, 8, 9], last_token=10, is_deep=True)
    T.lkv_check(blob)
    m, recs = L.read(blob)  # independent parse
    assert m["model_fingerprint"] == "tqkv-test" and m["position"] == st.offset
    assert m["prefix_tokens"] == [7, 8, 9] and m["last_token"] == 10 and m["is_deep"] is True
    (lay,) = m["layers"]
    assert lay["kind"] in KINDS and lay["offset"] == st.offset
    slots = download_slots(T, c, B * Hkv)
    ring = kw.get("max_size", 0) > 0
    if ring:
        assert (lay["max_size"], lay["keep"], lay["idx"]) == (kw["max_size"], kw.get("keep", 0),
                                                                st.idx)
    rows = st.cached_len if (ring or kind != "BF16") else st.offset
    # Record payloads are exactly the cache's rows, in the reference's order.
    if kind == "BF16":
        assert lay["kind"] == ("Sliding" if ring else "Full") and lay["arrays"] == [0, 1]
        for i, (dt, shape, data) in enumerate(recs):
            assert dt == L.DTYPES["BF16"] and shape == [B, Hkv, rows, D]
            assert data == slots[i][:, :rows].tobytes()
    elif kind == "AFFINE":
        assert lay["kind"] == ("SlidingQuantized" if ring else "FullQuantized")
        assert lay["arrays"] == list(range(6)) and lay["group_size"] == 64
        assert lay["bits"] == kw["bits_k"]
        dts = ["U32", "BF16", "BF16"] * 2
        for i, (dt, shape, data) in enumerate(recs):
            assert dt == L.DTYPES[dts[i]] and shape[:3] == [B, Hkv, rows]
            assert data == slots[i].tobytes()
    else:
        qjl = kw.get("qjl_words", 0) > 0
        assert lay["kind"] == "SlidingTurboquant" and lay["bits"] == kw["bits_k"]
        assert lay["arrays"] == ([0, 1, 2, 3, 4, 5] if qjl else [0, 1, 2, 3, None, None])
        vs = 4 if qjl else 2
        order = [0, 1, vs, vs + 1] + ([2, 3] if qjl else [])
        for j, (dt, shape, data) in enumerate(recs):
            s = order[j]
            if qjl and j == 4:  # signs: bf16 +-1 [.., m] from the packed words
                m_ = 32 * kw["qjl_words"]
                assert lay["qjl_m"] == m_ and dt == L.DTYPES["BF16"] and shape == [B, Hkv, rows, m_]
                words = slots[s].view(np.uint32).reshape(B * Hkv, rows, -1)
                bits = (words[..., :, None] >> np.arange(32, dtype=np.uint32)) & 1
                want = np.where(bits.reshape(B * Hkv, rows, m_) == 1, 0x3F80, 0xBF80)
                assert data == want.astype(np.uint16).tobytes()
            else:
                assert data == slots[s].tobytes()

    c2 = T.lkv_import(blob, 0, seed=42)
    s2 = c2.state()
    assert (s2.offset, s2.idx, s2.cached_len, s2.base_offset) == (st.offset, st.idx, rows,
                                                                   st.base_offset)
    slots2 = download_slots(T, c2, B * Hkv)
    for a, b in zip(slots, slots2):
        assert np.array_equal(a[:, :rows], b[:, :rows])
    # Exporting the imported cache gives the same file.
    assert T.lkv_export([c2], fingerprint="tqkv-test", created_at_unix=123, position=st.offset,
                        prefix_tokens=[7, 8, 9], last_token=10, is_deep=True) == blob
    # Same attention, and the same cache after more appends.
    if kind != "BF16":
        q = kv_bf16((B, Hq, 1, D), 5)
        dq = T.DeviceArray.of(q)
        o1, o2 = T.DeviceArray((B, Hq, 1, D), np.uint16), T.DeviceArray((B, Hq, 1, D), np.uint16)
        c.decode_attend(dq.ptr, Hq, D ** -0.5, o1.ptr)
        c2.decode_attend(dq.ptr, Hq, D ** -0.5, o2.ptr)
        T.hip().sync()
        assert np.array_equal(o1.numpy(), o2.numpy())
    fill(T, c, B, Hkv, D, [1, 3, 1], 99)
    fill(T, c2, B, Hkv, D, [1, 3, 1], 99)
    a, b = c.state(), c2.state()
    assert (a.offset, a.idx, a.view) == (b.offset, b.idx, b.view)
    # A bf16 growing layer is stored as its view [0, offset), so its buffer
    # restarts at that length (as set_state does in the reference) and grows
    # from there; every other kind keeps its whole buffer.
    n = a.view if (kind == "BF16" and not ring) else a.cached_len
    if not (kind == "BF16" and not ring):
        assert a.cached_len == b.cached_len
    for x, y in zip(download_slots(T, c, B * Hkv), download_slots(T, c2, B * Hkv)):
        assert np.array_equal(x[:, :n], y[:, :n])


def test_multi_layer_snapshot(T):
    B, Hkv, D = 1, 2, 128
    caches = [make(T, "AFFINE", dict(bits_k=4, bits_v=4), B, Hkv, D),
              make(T, "AFFINE", dict(bits_k=4, bits_v=4, max_size=64), B, Hkv, D),
              make(T, "BF16", {}, B, Hkv, D)]
    for i, c in enumerate(caches):
        fill(T, c, B, Hkv, D, [70 + 10 * i, 1], 3 + i)
    blob = T.lkv_export(caches, fingerprint="m", position=81)
    js, nl, nr = T.lkv_manifest(blob)
    assert (nl, nr) == (3, 14)
    m, recs = L.read(blob)
    assert [x["kind"] for x in m["layers"]] == ["FullQuantized", "SlidingQuantized", "Full"]
    assert m["layers"][1]["arrays"] == list(range(6, 12)) and m["layers"][2]["arrays"] == [12, 13]
    assert "last_token" not in m
    c1 = T.lkv_import(blob, 1)
    assert c1.state().offset == caches[1].state().offset
    with pytest.raises(T.TqkvError) as e:
        T.lkv_import(blob, 3)
    assert e.value.status == T.EINVAL_ARG
    bad = bytearray(blob)
    bad[-5] ^= 1
    with pytest.raises(T.TqkvError) as e:
        T.lkv_import(bytes(bad), 0)
    assert e.value.status == T.ECORRUPT


def test_import_rejects_inconsistent_layers(T):
    # Well-formed files whose layer does not describe a cache.
    m = L.manifest("x", 0, 0, [], None, False,
                   [L.layer("FullQuantized", 4, 0, [0, 1, 2, 3, 4, 5], bits=4, group_size=64)])
    u32 = lambda n: (L.DTYPES["U32"], [1, 1, 4, n], bytes(16 * n))
    b16 = lambda n: (L.DTYPES["BF16"], [1, 1, 4, n], bytes(8 * n))
    good = [u32(16), b16(2), b16(2), u32(16), b16(2), b16(2)]
    c = T.lkv_import(L.write(m, good), 0)
    assert c.state().offset == 4 and c.state().cached_len == 4
    for bad in ([u32(15)] + good[1:],                      # packed width vs bits
                good[:5] + [(L.DTYPES["BF16"], [1, 1, 5, 2], bytes(20))],  # S differs
                good[:1] + [(L.DTYPES["F32"], [1, 1, 4, 2], bytes(32))] + good[2:]):
        with pytest.raises(T.TqkvError) as e:
            T.lkv_import(L.write(m, bad), 0)
        assert e.value.status == T.ECORRUPT
    lin = L.manifest("x", 0, 0, [], None, False, [L.layer("Linear", 0)])
    with pytest.raises(T.TqkvError) as e:
        T.lkv_import(L.write(lin, []), 0)
    assert e.value.status == T.EUNSUPPORTED


@pytest.mark.parametrize("name,kind,kw,D,chunks", CASES, ids=[c[0] for c in CASES])
def test_clone_is_an_independent_copy(T, name, kind, kw, D, chunks):
    """tqkv_cache_clone (deep_clone, native_cache.rs:1575-1610): the clone
    holds the same state and bytes, attends the same, and stays untouched
    when the source takes further appends and is destroyed."""
    B, Hkv, Hq = 2, 2, 4
    print(f"[clone] {name}", flush=True)
    c = make(T, kind, kw, B, Hkv, D)
    fill(T, c, B, Hkv, D, chunks, 21)
    c2 = c.clone()
    T.hip().sync()
    a, b = c.state(), c2.state()
    assert (a.offset, a.idx, a.cached_len, a.base_offset, a.view) == \
           (b.offset, b.idx, b.cached_len, b.base_offset, b.view)
    before = download_slots(T, c, B * Hkv)
    for x, y in zip(before, download_slots(T, c2, B * Hkv)):
        assert np.array_equal(x, y)
    if kind != "BF16":
        q = kv_bf16((B, Hq, 1, D), 5)
        dq = T.DeviceArray.of(q)
        o1, o2 = T.DeviceArray((B, Hq, 1, D), np.uint16), T.DeviceArray((B, Hq, 1, D), np.uint16)
        c.decode_attend(dq.ptr, Hq, D ** -0.5, o1.ptr)
        c2.decode_attend(dq.ptr, Hq, D ** -0.5, o2.ptr)
        T.hip().sync()
        assert np.array_equal(o1.numpy(), o2.numpy())
    fill(T, c, B, Hkv, D, [1, 5], 77)  # the source moves on
    c.close()
    for x, y in zip(before, download_slots(T, c2, B * Hkv)):
        assert np.array_equal(x, y)
    fill(T, c2, B, Hkv, D, [2], 78)  # the clone still appends
    assert c2.state().offset == a.offset + 2
