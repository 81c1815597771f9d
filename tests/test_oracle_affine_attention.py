"""The oracle's affine quantizer, masks and dequantize-then-attend against
closed forms, the reference's known answers and brute force."""
import numpy as np
import pytest

import oracle_lib as O
from oracle_lib import lib, ptr


def _bf16_normal(shape, seed, std=1.0):
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * std
    return O.bf16_from_f32(x)


def _codes(packed, bits, d):
    words = packed.reshape(-1, packed.shape[-1]).astype(np.uint64)
    rows = words.shape[0]
    # assemble the LSB-first stream as a big integer per row
    out = np.empty((rows, d), np.uint32)
    for r in range(rows):
        v = 0
        for k, w in enumerate(words[r]):
            v |= int(w) << (32 * k)
        for i in range(d):
            out[r, i] = (v >> (bits * i)) & ((1 << bits) - 1)
    return out


def test_lowbit_packing_known_answers():
    # offload/lowbit.rs:612-623, word for word: two 4-bit codes share a word
    # from the bottom up; the eleventh 3-bit code starts at bit 30 and runs
    # into the next word.
    w = np.zeros(1, np.uint32)
    O.write_code(w, 0, 4, 0xA)
    O.write_code(w, 1, 4, 0x5)
    assert w[0] == 0x5A
    w = np.zeros(2, np.uint32)
    O.write_code(w, 10, 3, 0b101)
    assert list(w) == [0b01 << 30, 0b1]
    assert O.read_code(w, 10, 3) == 0b101
    # lowbit.rs:626-640: every code of every width reads back, with the
    # same multiplicative-hash codes as the reference's test.
    for bits in (2, 3, 4, 5, 6, 8):
        n = 32 * 8
        w = np.zeros(n * bits // 32, np.uint32)
        codes = [((i * 2654435761) & 0xFFFFFFFF) >> (32 - bits) for i in range(n)]
        for i, c in enumerate(codes):
            O.write_code(w, i, bits, c)
        assert [O.read_code(w, i, bits) for i in range(n)] == codes
    # The quantizer packs with the same writer: a row alternating 0 and 7 has
    # scale -1 and bias 7 (the larger-magnitude edge), so its codes alternate
    # 7 and 0 and pack to the reference's word pattern.
    x = np.zeros((1, 64), np.float32)
    x[0, 1::2] = 7.0
    p, _, _ = O.affine_quantize(O.bf16_from_f32(x), 64, 3)
    want = np.zeros(6, np.uint32)
    for i in range(64):
        O.write_code(want, i, 3, 0 if i % 2 else 7)
    assert np.array_equal(p[0], want)


@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 8])
def test_half_way_ties_round_away_from_zero(bits):
    # A group spanning exactly [0, n_bins] has scale -1 and bias n_bins (the
    # larger-magnitude edge), so the code of w is round(n_bins - w). Values
    # k + 0.5 put every code on a tie: MLX's Metal kernel rounds half away
    # from zero (the 4-bit golden digests fix that; the kernel is one
    # template over the width), so the code is n_bins - k, where half-to-even
    # would give n_bins - k - 1 for half of them.
    top = (1 << bits) - 1
    x = np.zeros((1, 64), np.float32)
    x[0, 0], x[0, 1] = 0.0, float(top)
    ks = np.arange(62) % top
    x[0, 2:] = ks + 0.5
    p, s, b = O.affine_quantize(O.bf16_from_f32(x), 64, bits)
    assert O.bf16_to_f32(s)[0, 0] == -1.0 and O.bf16_to_f32(b)[0, 0] == float(top)
    c = _codes(p, bits, 64)[0]
    assert c[0] == top and c[1] == 0
    assert np.array_equal(c[2:], top - ks)
    even = np.rint(top - (ks + 0.5)).astype(np.int64)
    assert np.any(even != top - ks)
    p2, _, _ = O.affine_quantize(O.bf16_from_f32(x), 64, bits, round_mode=1)
    assert not np.array_equal(p2, p)


def test_dequantize_readings_differ():
    # The primary reading of mlx::dequantize (one rounding of the fused
    # multiply-add, what the reference's qwen4exp_tiny fixture records) and
    # the secondary one (two bf16 roundings) must disagree on ordinary
    # inputs, or the fixture test would not tell them apart at bf16; the
    # primary equals the exact value rounded once.
    w = _bf16_normal((256, 256), 5, std=3.0)
    for bits in (3, 4, 8):
        p, s, b = O.affine_quantize(w, 64, bits)
        one = O.affine_dequantize(p, s, b, 64, bits)
        two = O.affine_dequantize(p, s, b, 64, bits, two_roundings=True)
        assert np.mean(two != one) > 0.01
        c = _codes(p, bits, 256).reshape(256, 4, 64).astype(np.float64)
        prod = (O.bf16_to_f32(s)[..., None] * c).reshape(256, 256)
        exact = prod + np.repeat(O.bf16_to_f32(b), 64, axis=-1)
        assert np.array_equal(one, O.bf16_from_f32(exact.astype(np.float32)))
        # Two roundings: half a bf16 step of the product, then of the sum.
        ulp = lambda v: 2.0 ** (np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126))) - 7)
        bound = 0.5 * ulp(prod) + 0.5 * ulp(np.abs(exact) + 0.5 * ulp(prod))
        assert np.all(np.abs(O.bf16_to_f32(two) - exact) <= bound)


@pytest.mark.parametrize("bits", [3, 4, 8])
def test_affine_error_bound_and_edge_snapping(bits):
    w = _bf16_normal((64, 256), 11 + bits)
    p, s, b = O.affine_quantize(w, 64, bits)
    c = _codes(p, bits, 256).reshape(64, 4, 64)
    assert c.max() <= (1 << bits) - 1
    sf = O.bf16_to_f32(s)[..., None].astype(np.float64)
    bf = O.bf16_to_f32(b)[..., None].astype(np.float64)
    x = O.bf16_to_f32(w).reshape(64, 4, 64).astype(np.float64)
    # each code picks the nearest level of the grid bias + c * scale, up to
    # what bf16 storage of scale and bias moves the grid (the snapped zero
    # point can leave the far extreme outside the grid; it clips to the end)
    levels = sf * np.arange(1 << bits) + bf
    dist = np.abs(x[..., None] - levels[..., None, :])
    chosen = np.take_along_axis(dist, c[..., None].astype(np.int64), -1)[..., 0]
    slop = np.abs(sf[..., 0]) * ((1 << bits) - 1) * 2 ** -7 + np.abs(bf[..., 0]) * 2 ** -7
    assert np.all(chosen <= dist.min(-1) + slop[..., None] + 1e-9)
    # the larger-magnitude extreme is the bias (edge snapping), to bf16
    lo, hi = x.min(-1), x.max(-1)
    edge = np.where(np.abs(lo) > np.abs(hi), lo, hi)
    assert np.allclose(bf[..., 0], edge, rtol=2 ** -8)
    # and maps to code 0
    at = np.argmax(x == edge[..., None], axis=-1)
    assert np.all(np.take_along_axis(c, at[..., None], -1) == 0)


def test_affine_dequantize_matches_definition():
    # Primary: one rounding of scale * code + bias (exact in f64 here, the
    # product being exact); secondary: each operation rounded to bf16.
    w = _bf16_normal((8, 128), 3)
    p, s, b = O.affine_quantize(w, 64, 4)
    c = _codes(p, 4, 128).reshape(8, 2, 64).astype(np.float64)
    sf = O.bf16_to_f32(s)[..., None].astype(np.float64)
    bf = O.bf16_to_f32(b)[..., None].astype(np.float64)
    one = O.bf16_to_f32(O.affine_dequantize(p, s, b, 64, 4))
    assert np.array_equal(one, O.bf16_to_f32(O.bf16_from_f32((sf * c + bf).reshape(8, 128))))
    two = O.bf16_to_f32(O.affine_dequantize(p, s, b, 64, 4, two_roundings=True))
    sc = O.bf16_to_f32(O.bf16_from_f32(sf * c))
    assert np.array_equal(two, O.bf16_to_f32(O.bf16_from_f32(sc + bf)).reshape(8, 128))


@pytest.mark.parametrize("q_len,offset,window,want", [
    # native_attention.rs:690-740
    (3, 0, -1, [[1, 0, 0], [1, 1, 0], [1, 1, 1]]),
    (4, 0, 2, [[1, 0, 0, 0], [1, 1, 0, 0], [0, 1, 1, 0], [0, 0, 1, 1]]),
    (1, 3, 2, [[0, 0, 1, 1]]),
])
def test_mask_known_answers(q_len, offset, window, want):
    got = [[lib().oracle_mask_allowed(offset + i, k, window) for k in range(offset + q_len)]
           for i in range(q_len)]
    assert got == want


def _brute(q, K, V, scale, mask=None):
    B, H, Lq, D = q.shape
    Hkv = K.shape[1]
    G = H // Hkv
    out = np.zeros((B, H, Lq, D))
    lse = np.zeros((B, H, Lq))
    qf, Kf, Vf = (O.bf16_to_f32(a).astype(np.float64) for a in (q, K, V))
    for b in range(B):
        for h in range(H):
            s = scale * qf[b, h] @ Kf[b, h // G].T
            if mask is not None:
                s = np.where(mask, s, -np.inf)
            m = s.max(-1, keepdims=True)
            e = np.exp(s - m)
            out[b, h] = e @ Vf[b, h // G] / e.sum(-1, keepdims=True)
            lse[b, h] = (m + np.log(e.sum(-1, keepdims=True)))[:, 0]
    return out, lse


def test_attend_matches_brute_force_with_gqa():
    q = _bf16_normal((2, 4, 1, 32), 1)
    K = _bf16_normal((2, 2, 40, 32), 2)
    V = _bf16_normal((2, 2, 40, 32), 3)
    of, ob, lse = O.attend_bf16(q, K, V, 0.2)
    want, wl = _brute(q, K, V, 0.2)
    assert np.abs(of - want).max() < 1e-6
    assert np.abs(lse - wl).max() < 1e-5
    # a head-to-KV mapping by h % H_kv instead of h / G would not match
    Kswap = K[:, ::-1].copy()
    Vswap = V[:, ::-1].copy()
    of2, _, _ = O.attend_bf16(q, Kswap, Vswap, 0.2)
    assert np.abs(of2 - want).max() > 1e-3


def test_attend_masked_prefill_and_window():
    q = _bf16_normal((1, 2, 6, 16), 4)
    K = _bf16_normal((1, 1, 9, 16), 5)
    V = _bf16_normal((1, 1, 9, 16), 6)
    # queries at absolute 10..15, keys held from absolute 7..15, window 4
    mask = np.array([[(10 + i >= 7 + k) and (10 + i < 7 + k + 4) for k in range(9)]
                     for i in range(6)])
    of, _, _ = O.attend_bf16(q, K, V, 0.25, causal=True, q_start=10, first_held=7, window=4)
    want, _ = _brute(q, K, V, 0.25, mask)
    assert np.abs(of - want).max() < 1e-6


def test_lse_merge_equals_full_softmax():
    # native_attention.rs:174-208 (sdpa_split): blending the two segments by
    # their log-sum-exps is the softmax over the concatenation.
    q = _bf16_normal((1, 4, 1, 32), 7)
    K = _bf16_normal((1, 2, 50, 32), 8)
    V = _bf16_normal((1, 2, 50, 32), 9)
    full, _, _ = O.attend_bf16(q, K, V, 0.3)
    op, _, lp = O.attend_bf16(q, K[:, :, :20].copy(), V[:, :, :20].copy(), 0.3)
    os_, _, ls = O.attend_bf16(q, K[:, :, 20:].copy(), V[:, :, 20:].copy(), 0.3)
    m = np.maximum(lp, ls)[..., None]
    wp, ws = np.exp(lp[..., None] - m), np.exp(ls[..., None] - m)
    merged = (op * wp + os_ * ws) / (wp + ws)
    assert np.abs(merged - full).max() < 1e-5


def test_attend_affine_is_dequantize_then_attend():
    q = _bf16_normal((1, 4, 1, 128), 10)
    k = _bf16_normal((1, 2, 33, 128), 11)
    v = _bf16_normal((1, 2, 33, 128), 12)
    kt, vt = O.affine_quantize(k, 64, 4), O.affine_quantize(v, 64, 8)
    # mlx::dequantize to bf16, then attention
    of, ob, _ = O.attend_affine(q, kt, vt, 64, 4, 8, 0.1, dequant="bf16")
    Kd, Vd = O.affine_dequantize(*kt, 64, 4), O.affine_dequantize(*vt, 64, 8)
    want, _ = _brute(q, Kd, Vd, 0.1)
    assert np.abs(of - want).max() < 1e-6
    assert np.array_equal(ob, O.bf16_from_f32(of))
    # exact dequantization scale * code + bias (numpy from the unpacked codes)
    of32, _, _ = O.attend_affine(q, kt, vt, 64, 4, 8, 0.1, dequant="f32")
    def exact(t, bits):
        c = _codes(t[0], bits, 128).reshape(1, 2, 33, 2, 64).astype(np.float64)
        s = O.bf16_to_f32(t[1])[..., None].astype(np.float64)
        b = O.bf16_to_f32(t[2])[..., None].astype(np.float64)
        return (s * c + b).reshape(1, 2, 33, 128)
    Ke, Ve = exact(kt, 4), exact(vt, 8)
    qf = O.bf16_to_f32(q).astype(np.float64)
    ref = np.zeros((1, 4, 1, 128))
    for h in range(4):
        sc = 0.1 * qf[0, h] @ Ke[0, h // 2].T
        e = np.exp(sc - sc.max())
        ref[0, h] = e @ Ve[0, h // 2] / e.sum()
    assert np.abs(of32 - ref).max() < 1e-5
    assert np.abs(of32 - of).max() > 0  # the two dequantizations differ


@pytest.mark.parametrize("L,causal,window,dequant", [(1, False, -1, "f32"), (7, True, 40, "bf16"),
                                                      (5, True, -1, "f32")])
def test_cpu_baseline_port_agrees_with_the_oracle(L, causal, window, dequant):
    # The bench's CPU baseline (an f32 port of dequantize-then-attend) must
    # compute what the oracle computes: within the decode bar of the f64
    # oracle on the same cache (GQA 4, a row past the window, 3-bit keys and
    # 8-bit values), and the same bits at any thread count.
    B, H, Hkv, D, N, gs = 2, 8, 2, 128, 300, 64
    q = _bf16_normal((B, H, L, D), 71)
    kt = O.affine_quantize(_bf16_normal((B, Hkv, N, D), 72), gs, 3)
    vt = O.affine_quantize(_bf16_normal((B, Hkv, N, D), 73), gs, 8)
    kw = dict(causal=causal, q_start=N - L, first_held=0, window=window)
    got = O.attend_affine_f32(q, kt, vt, N, gs, 3, 8, D ** -0.5, threads=1, dequant=dequant, **kw)
    want, _, _ = O.attend_affine(q, kt, vt, gs, 3, 8, D ** -0.5, dequant=dequant, **kw)
    err = np.abs(O.bf16_to_f32(got).astype(np.float64) - want)
    assert err.max() <= 2e-2 and err.mean() <= 1e-3
    assert np.array_equal(got, O.attend_affine_f32(q, kt, vt, N, gs, 3, 8, D ** -0.5, threads=4,
                                                   dequant=dequant, **kw))
