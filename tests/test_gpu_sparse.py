"""Page-sparse decode on the GPU through the C ABI (after sdpa_page_sparse,
native_attention.rs:210-329, and PageDigest, native_cache.rs:352-445),
against the CPU oracle: the digest bit-exact, the page choice a valid
top-keep of the oracle's bounds (and equal to the oracle's where no two
bounds are within the f32 summation tolerance of the cut), the attention
over the chosen pages and the tail within 2e-2 max-abs / 1e-3 mean-abs of
the oracle's over the same keys, keep >= pages identical to dense decode,
and the reference's planted-page test."""
import numpy as np
import pytest

import oracle_lib as O
from inputs import kv_bf16
from sparse_cases import PAGE, check_choice, cosine, planted
from test_gpu_affine import _cache, check_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def T():
    import tqkv
    assert tqkv.hip().device_count() > 0, "no GPU visible"
    return tqkv


def dev_ptrs(t):
    return tuple(a.ptr for a in t)


def digest_gpu(T, kd, B, Hkv, cap, D, gs, bits, pages, max_pages, cuts=()):
    kmin = T.DeviceArray((B, Hkv, max_pages, D), np.uint16,
                         np.full((B, Hkv, max_pages, D), 0x7777, np.uint16))
    kmax = T.DeviceArray((B, Hkv, max_pages, D), np.uint16,
                         np.full((B, Hkv, max_pages, D), 0x7777, np.uint16))
    edges = [0, *cuts, pages]
    for lo, hi in zip(edges[:-1], edges[1:]):
        T.page_digest_affine(dev_ptrs(kd), B * Hkv, cap, D, gs, bits, lo, hi, kmin.ptr, kmax.ptr,
                             max_pages)
    T.hip().sync()
    return kmin, kmax


@pytest.mark.parametrize("D,gs,bits", [(128, 64, 4), (256, 64, 3), (64, 32, 8), (128, 32, 6),
                                       (512, 128, 2)])
def test_digest_bit_exact_in_pieces(T, D, gs, bits):
    B, Hkv, N, cap, max_pages = 2, 3, 1000, 1100, 20
    print(f"[digest] D={D} gs={gs} bits={bits}", flush=True)
    x = kv_bf16((B, Hkv, N, D), 40 + D + bits, frac=0.02, mult=8.0)
    kh, kd = _cache(x, gs, bits, cap)
    pages = N // PAGE
    kmin, kmax = digest_gpu(T, kd, B, Hkv, cap, D, gs, bits, pages, max_pages, cuts=(6, 7))
    wmin, wmax = O.page_digest_affine(tuple(a[:, :, :N] for a in kh), gs, bits, pages)
    gmin, gmax = kmin.numpy(), kmax.numpy()
    assert np.array_equal(gmin[:, :, :pages], wmin) and np.array_equal(gmax[:, :, :pages], wmax)
    assert np.all(gmin[:, :, pages:] == 0x7777) and np.all(gmax[:, :, pages:] == 0x7777)
    # Bit-exact with the oracle's reading of mlx::dequantize (one rounding
    # of the fused multiply-add). Against the secondary reading (two bf16
    # roundings) a page's min / max moves by at most the largest difference
    # between the two readings over the page's keys at that channel (min and
    # max are 1-Lipschitz in the largest difference): the digest stays
    # within it.
    tr = tuple(a[:, :, :pages * PAGE] for a in kh)
    dq1 = O.bf16_to_f32(O.affine_dequantize(*tr, gs, bits)).astype(np.float64)
    dq2 = O.bf16_to_f32(O.affine_dequantize(*tr, gs, bits, two_roundings=True)).astype(np.float64)
    gap = np.abs(dq1 - dq2).reshape(B, Hkv, pages, PAGE, D).max(axis=3)
    pg = dq2.reshape(B, Hkv, pages, PAGE, D)
    for got, alt in ((gmin, pg.min(axis=3)), (gmax, pg.max(axis=3))):
        g = O.bf16_to_f32(got[:, :, :pages]).astype(np.float64)
        assert np.all(np.abs(g - alt) <= gap)


@pytest.mark.parametrize("pages,H,Hkv,D", [(70, 8, 2, 128), (313, 16, 8, 256), (1000, 32, 8, 128),
                                           (4096, 4, 4, 64), (9, 4, 2, 64), (1024, 8, 8, 512)])
def test_page_choice_is_a_top_keep(T, pages, H, Hkv, D):
    B = 2
    keep = min(O.sparse_keep_pages(pages), pages - 2) if pages < 64 else O.sparse_keep_pages(pages)
    print(f"[select] pages={pages} keep={keep} H={H}/{Hkv} D={D}", flush=True)
    rng = np.random.default_rng(pages + D)
    a = O.bf16_to_f32(kv_bf16((B, Hkv, pages, D), pages))
    c = a + np.abs(rng.standard_normal(a.shape)).astype(np.float32)
    kmin, kmax = O.bf16_from_f32(np.minimum(a, c)), O.bf16_from_f32(np.maximum(a, c))
    q = kv_bf16((B, H, 1, D), pages + 1)
    chosen = T.DeviceArray((B, Hkv, keep), np.int32)
    dq, dmin, dmax = T.DeviceArray.of(q), T.DeviceArray.of(kmin), T.DeviceArray.of(kmax)
    wsb = T.page_select_workspace_size(B, Hkv, pages)
    ws = T.DeviceArray((wsb,), np.uint8)
    T.page_select(dq.ptr, B, H, Hkv, D, dmin.ptr, dmax.ptr, pages, pages, keep, chosen.ptr,
                  ws.ptr, wsb)
    T.hip().sync()
    got = chosen.numpy()
    bounds = O.page_bounds(q, kmin, kmax, pages)
    check_choice(got, bounds, keep)
    want = O.select_pages(bounds, keep)
    for b in range(B):
        for h in range(Hkv):
            bd = bounds[b, h].copy()
            bd[[0, *range(pages - 4, pages)]] = np.inf
            srt = np.sort(bd)[::-1]
            if keep < pages and srt[keep - 1] - srt[keep] > 1e-4 * (1 + abs(srt[keep])):
                assert np.array_equal(got[b, h], want[b, h])


PAGE_CASES = [
    # (B, H, Hkv, D, N, pages digested, keep, bits_k, bits_v)
    (2, 32, 8, 128, 5000, 78, 20, 4, 4),    # config 1/3 layout, tail of 8 rows
    (2, 16, 8, 256, 9000, 140, 64, 3, 3),   # config 2 layout
    (1, 32, 8, 128, 4200, 60, 16, 8, 4),    # config 4 widths, tail of 360 rows
    (3, 4, 4, 64, 3000, 46, 46, 4, 4),      # every page
    (1, 16, 8, 256, 66000, 1031, 600, 3, 3),  # more than one split's page table
]


@pytest.mark.parametrize("B,H,Hkv,D,N,pages,keep,bk,bv", PAGE_CASES)
@pytest.mark.parametrize("splits", ["auto", "1"])
def test_decode_over_pages_matches_oracle(T, monkeypatch, B, H, Hkv, D, N, pages, keep, bk, bv,
                                          splits):
    if splits == "1":
        monkeypatch.setenv("TQKV_DECODE_SPLITS", "1")
    print(f"[pages] B={B} H={H}/{Hkv} D={D} N={N} pages={pages} keep={keep} bits={bk}/{bv} "
          f"splits={splits}", flush=True)
    gs, cap = 64, N + 100
    seed = N + D + keep
    q = kv_bf16((B, H, 1, D), seed)
    k = kv_bf16((B, Hkv, N, D), seed + 1, frac=0.01, mult=10.0)
    v = kv_bf16((B, Hkv, N, D), seed + 2, frac=0.01, mult=10.0)
    (kh, kd), (vh, vd) = _cache(k, gs, bk, cap), _cache(v, gs, bv, cap)
    rng = np.random.default_rng(seed)
    chosen = np.stack([np.stack([np.sort(rng.choice(pages, keep, replace=False))
                                 for _ in range(Hkv)]) for _ in range(B)]).astype(np.int32)
    dq, dc = T.DeviceArray.of(q), T.DeviceArray.of(chosen)
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    seg = T.affine_seg(dev_ptrs(kd), dev_ptrs(vd), cap, N)
    scale = 1.0 / np.sqrt(D)
    T.decode_attend_affine_pages(dq.ptr, B, H, Hkv, D, gs, bk, bv, scale, seg, dc.ptr, keep, pages,
                                 out.ptr)
    T.hip().sync()
    kt = tuple(a[:, :, :N] for a in kh)
    vt = tuple(a[:, :, :N] for a in vh)
    want, _, _ = O.attend_affine_pages(q, kt, vt, chosen, pages, N, gs, bk, bv, scale)
    check_close(out.numpy(), want)


def test_sparse_entry_end_to_end_and_dense_when_all_kept(T):
    B, H, Hkv, D, N, gs, bk, bv = 2, 16, 8, 256, 20000, 64, 3, 3
    cap, max_pages = N + 64, (N + 64) // PAGE
    q = kv_bf16((B, H, 1, D), 77)
    k = kv_bf16((B, Hkv, N, D), 78, frac=0.01, mult=10.0)
    v = kv_bf16((B, Hkv, N, D), 79, frac=0.01, mult=10.0)
    (kh, kd), (vh, vd) = _cache(k, gs, bk, cap), _cache(v, gs, bv, cap)
    pages = N // PAGE
    kmin, kmax = digest_gpu(T, kd, B, Hkv, cap, D, gs, bk, pages, max_pages)
    keep = int(T.sparse_keep_pages(pages))
    wsb = T.sparse_workspace_size(B, H, Hkv, D, N, keep)
    ws = T.DeviceArray((wsb,), np.uint8)
    dq = T.DeviceArray.of(q)
    seg = T.affine_seg(dev_ptrs(kd), dev_ptrs(vd), cap, N)
    out = T.DeviceArray((B, H, 1, D), np.uint16)
    chosen = T.DeviceArray((B, Hkv, keep), np.int32)
    scale = 1.0 / np.sqrt(D)
    print(f"[sparse] pages={pages} keep={keep}", flush=True)
    T.decode_attend_affine_sparse(dq.ptr, B, H, Hkv, D, gs, bk, bv, scale, seg, kmin.ptr,
                                  kmax.ptr, max_pages, pages, keep, out.ptr, ws.ptr, wsb,
                                  chosen_out=chosen.ptr)
    T.hip().sync()
    kt, vt = tuple(a[:, :, :N] for a in kh), tuple(a[:, :, :N] for a in vh)
    wmin, wmax = O.page_digest_affine(kt, gs, bk, pages)
    got_choice = chosen.numpy()
    check_choice(got_choice, O.page_bounds(q, wmin, wmax, pages), keep)
    want, _, _ = O.attend_affine_pages(q, kt, vt, got_choice, pages, N, gs, bk, bv, scale)
    check_close(out.numpy(), want)
    # keep >= pages: the dense decode, bit for bit.
    dense = T.DeviceArray((B, H, 1, D), np.uint16)
    T.decode_attend_affine(dq.ptr, B, H, Hkv, D, gs, bk, bv, scale, [seg], dense.ptr, ws.ptr, wsb)
    T.decode_attend_affine_sparse(dq.ptr, B, H, Hkv, D, gs, bk, bv, scale, seg, kmin.ptr,
                                  kmax.ptr, max_pages, pages, pages, out.ptr, ws.ptr, wsb)
    T.hip().sync()
    assert np.array_equal(out.numpy(), dense.numpy())


def test_planted_page_is_found(T):
    q, k, v = planted()
    B, H, Hkv, D, gs, bits = 1, 8, 2, 256, 64, 8
    n = k.shape[2]
    cap = n
    (kh, kd), (vh, vd) = _cache(k, gs, bits, cap), _cache(v, gs, bits, cap)
    pages = n // PAGE
    kmin, kmax = digest_gpu(T, kd, B, Hkv, cap, D, gs, bits, pages, pages)
    keep = 64
    wsb = T.sparse_workspace_size(B, H, Hkv, D, n, keep)
    ws = T.DeviceArray((wsb,), np.uint8)
    dq = T.DeviceArray.of(q)
    seg = T.affine_seg(dev_ptrs(kd), dev_ptrs(vd), cap, n)
    out, dense = T.DeviceArray((B, H, 1, D), np.uint16), T.DeviceArray((B, H, 1, D), np.uint16)
    chosen = T.DeviceArray((B, Hkv, keep), np.int32)
    scale = 1.0 / np.sqrt(D)
    print(f"[planted] n={n} pages={pages} keep={keep}", flush=True)
    T.decode_attend_affine_sparse(dq.ptr, B, H, Hkv, D, gs, bits, bits, scale, seg, kmin.ptr,
                                  kmax.ptr, pages, pages, keep, out.ptr, ws.ptr, wsb,
                                  chosen_out=chosen.ptr)
    T.decode_attend_affine(dq.ptr, B, H, Hkv, D, gs, bits, bits, scale, [seg], dense.ptr, ws.ptr,
                           wsb)
    T.hip().sync()
    assert all(40 in chosen.numpy()[0, j] for j in range(Hkv))
    c = cosine(O.bf16_to_f32(out.numpy()), O.bf16_to_f32(dense.numpy()))
    print(f"[planted] cos={c:.6f}", flush=True)
    assert c > 0.99
