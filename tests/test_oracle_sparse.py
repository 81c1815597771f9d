"""The page-sparse oracle on the CPU (no GPU), pinned by what fixes it:
the digest is the elementwise min / max of the dequantized pages (brute
force over the oracle's own mlx::dequantize), the bound dominates every
score of its page and equals it on a page of identical keys, the choice
pins the sink and recent pages and otherwise takes the largest bounds
(brute force), keep follows max(pages / 8, 64), and the reference's
planted-page test (native_attention.rs:1085-1140) holds."""
import numpy as np

import oracle_lib as O
from inputs import kv_bf16
from sparse_cases import PAGE, check_choice, cosine, planted


def test_digest_is_min_max_of_dequantized_pages():
    B, Hkv, cap, D, gs, bits = 2, 3, 300, 128, 64, 4
    x = kv_bf16((B, Hkv, cap, D), 5, frac=0.02, mult=8.0)
    kt = O.affine_quantize(x, gs, bits)
    pages = cap // PAGE
    kmin, kmax = O.page_digest_affine(kt, gs, bits, pages, max_pages=6)
    deq = O.bf16_to_f32(O.affine_dequantize(*kt, gs, bits))[:, :, :pages * PAGE]
    paged = deq.reshape(B, Hkv, pages, PAGE, D)
    assert np.array_equal(O.bf16_to_f32(kmin[:, :, :pages]), paged.min(axis=3))
    assert np.array_equal(O.bf16_to_f32(kmax[:, :, :pages]), paged.max(axis=3))
    assert not kmin[:, :, pages:].any() and not kmax[:, :, pages:].any()


def test_bound_dominates_its_page_and_is_tight_on_equal_keys():
    B, H, Hkv, D, gs, bits, n = 1, 8, 2, 64, 32, 8, 4 * PAGE
    x = O.bf16_to_f32(kv_bf16((B, Hkv, n, D), 7)).copy()
    x[:, :, 2 * PAGE:3 * PAGE] = x[:, :, 2 * PAGE:2 * PAGE + 1]  # page 2: one key 64 times
    kt = O.affine_quantize(O.bf16_from_f32(x), gs, bits)
    q = kv_bf16((B, H, 1, D), 8)
    kmin, kmax = O.page_digest_affine(kt, gs, bits, 4)
    bounds = O.page_bounds(q, kmin, kmax, 4)
    keys = O.bf16_to_f32(O.affine_dequantize(*kt, gs, bits)).astype(np.float64)
    qf = O.bf16_to_f32(q).astype(np.float64).reshape(B, Hkv, H // Hkv, D)
    for h in range(Hkv):
        for p in range(4):
            s = qf[0, h] @ keys[0, h, p * PAGE:(p + 1) * PAGE].T  # [G, 64]
            assert s.max() <= bounds[0, h, p] + 1e-9
            if p == 2:
                assert np.isclose(s.max(), bounds[0, h, p], rtol=1e-12, atol=1e-12)
            else:
                assert s.max() < bounds[0, h, p]


def test_select_pins_then_takes_the_largest():
    rng = np.random.default_rng(3)
    pages, keep = 100, 20
    bounds = rng.standard_normal((2, 3, pages))
    chosen = O.select_pages(bounds, keep)
    check_choice(chosen, bounds, keep, tol_rel=0.0)
    for b in range(2):
        for h in range(3):
            inner = np.arange(1, pages - 4)
            top = inner[np.argsort(-bounds[b, h, inner], kind="stable")[:keep - 5]]
            assert sorted(chosen[b, h].tolist()) == sorted([0, 96, 97, 98, 99, *top.tolist()])
    # All bounds equal: the lower pages win the ties.
    flat = O.select_pages(np.zeros((1, 1, pages)), keep)
    assert flat[0, 0].tolist() == list(range(0, keep - 4)) + [96, 97, 98, 99]
    every = O.select_pages(bounds, pages)
    assert np.array_equal(every, np.broadcast_to(np.arange(pages), (2, 3, pages)))


def test_keep_pages_closed_form():
    for pages, keep in [(1, 64), (100, 64), (512, 64), (520, 65), (1000, 125), (4096, 512)]:
        assert O.sparse_keep_pages(pages) == keep


def test_planted_page_is_found():
    q, k, v = planted()
    h, h_kv, d = 8, 2, 256
    n = k.shape[2]
    kt, vt = O.affine_quantize(k, 64, 8), O.affine_quantize(v, 64, 8)
    pages = n // PAGE
    kmin, kmax = O.page_digest_affine(kt, 64, 8, pages)
    bounds = O.page_bounds(q, kmin, kmax, pages)
    scale = 1.0 / np.sqrt(d)
    dense, _, _ = O.attend_affine(q, kt, vt, 64, 8, 8, scale)
    every = O.select_pages(bounds, pages)
    allp, _, _ = O.attend_affine_pages(q, kt, vt, every, pages, n, 64, 8, 8, scale)
    assert cosine(allp, dense) > 0.9999
    chosen = O.select_pages(bounds, 64)
    assert all(40 in chosen[0, j] for j in range(h_kv))
    sparse, _, _ = O.attend_affine_pages(q, kt, vt, chosen, pages, n, 64, 8, 8, scale)
    cut = 41 * PAGE
    without, _, _ = O.attend_affine(q, tuple(a[:, :, cut:] for a in kt),
                                    tuple(a[:, :, cut:] for a in vt), 64, 8, 8, scale)
    assert cosine(sparse, dense) > 0.99
    assert cosine(without, dense) < 0.9
