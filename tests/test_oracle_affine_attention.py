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
    # offload/lowbit.rs:612-623: two 4-bit codes share a word from the bottom
    # up; the eleventh 3-bit code starts at bit 30 and runs into the next word.
    w = np.zeros((1, 64), np.uint16)
    p, s, b = O.affine_quantize(w, 64, 4)
    assert p.shape == (1, 8)
    x = np.zeros((1, 64), np.float32)
    x[0, 0], x[0, 1] = 0.0, 1.0
    x[0, 2:] = 0.5
    p, s, b = O.affine_quantize(O.bf16_from_f32(x), 64, 3)
    c = _codes(p, 3, 64)[0]
    deq = O.bf16_to_f32(O.affine_dequantize(p, s, b, 64, 3))[0]
    assert np.allclose(deq, x[0], atol=O.bf16_to_f32(s)[0, 0].__abs__() / 2 + 1e-6)
    assert c[1] in (0, 7) and c[0] in (0, 7) and c[0] != c[1]


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
    w = _bf16_normal((8, 128), 3)
    p, s, b = O.affine_quantize(w, 64, 4)
    d = O.bf16_to_f32(O.affine_dequantize(p, s, b, 64, 4))
    c = _codes(p, 4, 128).reshape(8, 2, 64).astype(np.float32)
    sc = O.bf16_to_f32(O.bf16_from_f32(O.bf16_to_f32(s)[..., None] * c))
    want = O.bf16_to_f32(O.bf16_from_f32(sc + O.bf16_to_f32(b)[..., None])).reshape(8, 128)
    assert np.array_equal(d, want)


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
