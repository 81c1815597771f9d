"""Prefill-chunk attention over affine-packed K/V on the GPU (MFMA), through
the C ABI, against the CPU oracle's dequantize-then-attend with the
dequantization the reference's prefill path uses (mlx::dequantize to bf16,
gemma4_moe.rs:2394-2399) and its absolute-position mask
(build_causal_mask_abs, native_attention.rs:545-622).

Bar: 2e-2 max-abs and 1e-3 mean-abs in bf16 (|got - RN_bf16(expected)|,
tests/bars.py), as for decode. Cases cover the reference's prefill branches
(causal aligned, sliding window over a rotating view, unmasked), GQA groups
that do not divide the 128-row block (G = 3), rows that see no key, a shared
prefix segment, every head dim the kernel takes and mixed K/V widths, and the
cache-level entry on growing and rotating caches across chunk boundaries.
The dequantize-once path (keys dequantized into scratch, then copied) must
match the in-block path bit for bit.
"""
import numpy as np
import pytest

import oracle_lib as O
from inputs import kv_bf16
from bars import check_bf16
from test_gpu_affine import _cache

pytestmark = pytest.mark.gpu

@pytest.fixture(scope="module")
def T():
    import tqkv
    assert tqkv.hip().device_count() > 0, "no GPU visible"
    return tqkv


def want_mlx(q, kh, vh, gs, bk, bv, scale, **kw):
    """The oracle over the mlx::dequantize'd cache (one rounding of the fused
    multiply-add, as the reference's fixture records MLX's kernel), and over
    the secondary reading (two bf16 roundings), printed only."""
    return tuple(O.attend_affine(q, kh, vh, gs, bk, bv, scale, dequant=d, **kw)[0]
                 for d in ("bf16", "bf16_2r"))


def check(got_bf16, wants, tag):
    """The bar in bf16 (bars.check_bf16) against the primary reading; the
    raw distance to the secondary reading is printed beside it."""
    check_bf16(got_bf16, wants[0], f"prefill {tag}")
    got = O.bf16_to_f32(got_bf16).astype(np.float64)
    print(f"[prefill {tag}] secondary reading: max_abs={np.abs(got - wants[1]).max():.3e}",
          flush=True)


def run(T, q, segs_host, B, H, Hkv, L, D, gs, bk, bv, scale, q_start, k_start, causal, window):
    dq = T.DeviceArray.of(q)
    out = T.DeviceArray((B, H, L, D), np.uint16, np.full((B, H, L, D), 0x7FC0, np.uint16))
    segs = [T.affine_seg(tuple(a.ptr for a in k), tuple(a.ptr for a in v), cap, n, sh)
            for (k, v, cap, n, sh) in segs_host]
    T.prefill_attend_affine(dq.ptr, B, H, Hkv, L, D, gs, bk, bv, scale, segs, out.ptr,
                            q_start, k_start, causal, window)
    T.hip().sync()
    return out.numpy()


PREFILL_CASES = [
    # (B, H, Hkv, D, L, N, bits_k, bits_v, gs, q_start, k_start, causal, window, scale)
    (1, 32, 8, 128, 256, 1024, 4, 4, 64, 768, 0, True, -1, 1.0),     # config 3 global layer
    (1, 32, 8, 128, 256, 383, 4, 4, 64, 1000, 873, True, 128, 1.0),  # config 3 local: ring view
    (2, 32, 8, 128, 130, 130, 4, 4, 64, 0, 0, True, 64, None),       # first chunk, window < L
    (1, 16, 8, 256, 128, 700, 3, 3, 64, 572, 0, True, -1, None),     # config 2 widths
    (2, 4, 4, 64, 200, 200, 8, 4, 32, 0, 0, True, -1, None),         # K8/V4, gs 32
    (1, 12, 4, 128, 77, 300, 5, 6, 32, 223, 0, True, -1, None),      # G = 3, ragged tiles
    (1, 8, 2, 128, 65, 300, 2, 3, 128, 0, 0, False, -1, None),       # unmasked
    (1, 8, 8, 256, 1, 333, 6, 2, 64, 332, 0, True, -1, 1.0),         # one query row
    (1, 8, 2, 128, 96, 160, 4, 4, 64, 0, 50, True, -1, None),        # rows before any key
    (1, 4, 1, 64, 300, 64, 4, 8, 64, 0, 0, True, 1, None),           # window 1: self only
    (1, 16, 2, 512, 40, 600, 4, 4, 64, 560, 0, True, -1, None),      # D = 512 (Gemma 4 global)
    (2, 8, 4, 512, 70, 300, 8, 6, 128, 230, 0, True, 100, 1.0),      # D = 512, window, 8/6-bit
    (1, 16, 2, 512, 96, 450, 3, 5, 32, 354, 0, True, -1, None),      # D = 512, 12 row blocks
    (1, 8, 2, 128, 50, 40, 4, 4, 64, 0, 0, True, -1, None),          # fewer keys than a tile
]


@pytest.mark.parametrize("B,H,Hkv,D,L,N,bk,bv,gs,q_start,k_start,causal,window,scale",
                         PREFILL_CASES)
def test_prefill_matches_dequantize_then_attend(T, B, H, Hkv, D, L, N, bk, bv, gs, q_start,
                                                k_start, causal, window, scale):
    print(f"[prefill] B={B} H={H}/{Hkv} D={D} L={L} N={N} bits={bk}/{bv} gs={gs} "
          f"q_start={q_start} k_start={k_start} causal={causal} window={window}", flush=True)
    seed = B * 7919 + H * 31 + D + L * 3 + N + bk * 11 + bv
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    q = kv_bf16((B, H, L, D), seed)
    k = kv_bf16((B, Hkv, N, D), seed + 1, frac=0.01, mult=10.0)
    v = kv_bf16((B, Hkv, N, D), seed + 2, frac=0.01, mult=10.0)
    if scale == 1.0:
        q = O.bf16_from_f32(O.bf16_to_f32(q) / np.sqrt(D))  # Gemma: q-norm'd queries, scale 1
    (kh, kd), (vh, vd) = _cache(k, gs, bk, N + 5), _cache(v, gs, bv, N + 5)
    got = run(T, q, [(kd, vd, N + 5, N, False)], B, H, Hkv, L, D, gs, bk, bv, scale, q_start,
              k_start, causal, window)
    want = want_mlx(q, kh, vh, gs, bk, bv, scale, causal=causal, q_start=q_start,
                    first_held=k_start, window=window)
    check(got, want, "chunk")
    if causal and k_start > q_start:
        # Query rows before the first key see nothing and return zeros.
        blind = k_start - q_start
        assert np.all(got[:, :, :blind] == 0)


def test_prefill_two_segments(T):
    # A shared prefix (one copy for every batch row) then per-row suffixes:
    # the keys of both enter one softmax, positions counted across both.
    B, H, Hkv, D, L, gs, bits = 2, 16, 4, 128, 96, 64, 4
    P, S = 250, 200
    q = kv_bf16((B, H, L, D), 5)
    kp = kv_bf16((1, Hkv, P, D), 6, frac=0.01, mult=10.0)
    vp = kv_bf16((1, Hkv, P, D), 7)
    ks = kv_bf16((B, Hkv, S, D), 8, frac=0.01, mult=10.0)
    vs = kv_bf16((B, Hkv, S, D), 9)
    (kph, kpd), (vph, vpd) = _cache(kp, gs, bits), _cache(vp, gs, bits)
    (ksh, ksd), (vsh, vsd) = _cache(ks, gs, bits, S + 3), _cache(vs, gs, bits, S + 3)
    scale = 1.0 / np.sqrt(D)
    got = run(T, q, [(kpd, vpd, P, P, True), (ksd, vsd, S + 3, S, False)], B, H, Hkv, L, D, gs,
              bits, bits, scale, P + S - L, 0, True, 300)
    cat = lambda a, b: np.concatenate([np.broadcast_to(a, (B,) + a.shape[1:]), b], axis=2)
    kh = tuple(cat(a, b) for a, b in zip(kph, ksh))
    vh = tuple(cat(a, b) for a, b in zip(vph, vsh))
    want = want_mlx(q, kh, vh, gs, bits, bits, scale, causal=True, q_start=P + S - L,
                    first_held=0, window=300)
    check(got, want, "two segments")


def test_prefill_sharp_softmax(T):
    # Scale 1 on unnormalized N(0,1) queries: scores spread over hundreds,
    # softmax nearly one-hot, the running maximum moves often.
    B, H, Hkv, D, L, N, gs, bits = 1, 8, 2, 128, 64, 256, 64, 4
    q = kv_bf16((B, H, L, D), 11)
    k = kv_bf16((B, Hkv, N, D), 12)
    v = kv_bf16((B, Hkv, N, D), 13)
    (kh, kd), (vh, vd) = _cache(k, gs, bits), _cache(v, gs, bits)
    got = run(T, q, [(kd, vd, N, N, False)], B, H, Hkv, L, D, gs, bits, bits, 1.0, N - L, 0,
              True, -1)
    want = want_mlx(q, kh, vh, gs, bits, bits, 1.0, causal=True, q_start=N - L, first_held=0)
    check(got, want, "sharp")


def test_prefill_rejects_bad_arguments(T):
    seg = T.affine_seg((1, 1, 1), (1, 1, 1), 8, 8)
    cases = [
        (dict(D=1024), T.EUNSUPPORTED),
        (dict(D=96), T.EUNSUPPORTED),
        (dict(bk=7), T.EUNSUPPORTED),
        (dict(gs=16), T.EUNSUPPORTED),
        (dict(window=0), T.EINVAL_ARG),
        (dict(L=0), T.EINVAL_SHAPE),
        (dict(H=6, Hkv=4), T.EINVAL_SHAPE),
    ]
    for over, status in cases:
        a = dict(B=1, H=4, Hkv=2, L=4, D=128, gs=64, bk=4, bv=4, window=-1)
        a.update(over)
        with pytest.raises(T.TqkvError) as e:
            T.prefill_attend_affine(1, a["B"], a["H"], a["Hkv"], a["L"], a["D"], a["gs"],
                                    a["bk"], a["bv"], 1.0, [seg], 1, 0, 0, True, a["window"])
        assert e.value.status == status, over


# --------------------------------------------------------- through the cache
@pytest.mark.parametrize("max_size,window", [(0, -1), (192, 192)])
def test_cache_prefill_chunks(T, max_size, window):
    """Chunks of a prompt appended into a growing cache (a global layer) or a
    ring of max_size (a sliding layer, window = max_size): after each chunk
    the view's keys end at the cache offset, and the chunk's queries attend
    causally, as forward_last_token_chunked does (gemma4_moe.rs:6172)."""
    B, H, Hkv, D, gs, bits = 2, 8, 4, 128, 64, 4
    chunks = [100, 160, 64, 1]
    total = sum(chunks)
    k_all = kv_bf16((B, Hkv, total, D), 21, frac=0.01, mult=10.0)
    v_all = kv_bf16((B, Hkv, total, D), 22)
    c = T.Cache(T.CACHE_AFFINE, B, Hkv, D, D, gs, bits, bits, prealloc=True, max_size=max_size)
    pos = 0
    for L in chunks:
        print(f"[cache-prefill] max_size={max_size} chunk at {pos} L={L}", flush=True)
        kc = np.ascontiguousarray(k_all[:, :, pos:pos + L])
        vc = np.ascontiguousarray(v_all[:, :, pos:pos + L])
        dk, dv = T.DeviceArray.of(kc), T.DeviceArray.of(vc)
        view = c.append(dk.ptr, dv.ptr, L)
        pos += L
        q = kv_bf16((B, H, L, D), 100 + pos)
        dq = T.DeviceArray.of(q)
        out = T.DeviceArray((B, H, L, D), np.uint16)
        c.prefill_attend(dq.ptr, H, L, 1.0 / np.sqrt(D), out.ptr, window=window)
        T.hip().sync()
        n = view.n
        # The view holds the newest n tokens: in order after a multi-token
        # append (rotating_concat); in ring order after a one-token append,
        # where the one query sees every held key and order does not matter.
        first = pos - n
        kh = O.affine_quantize(np.ascontiguousarray(k_all[:, :, first:pos]), gs, bits)
        vh = O.affine_quantize(np.ascontiguousarray(v_all[:, :, first:pos]), gs, bits)
        want = want_mlx(q, kh, vh, gs, bits, bits, 1.0 / np.sqrt(D), causal=True,
                        q_start=pos - L, first_held=first, window=window)
        check(out.numpy(), want, f"cache chunk L={L} view={n}")


def test_cache_prefill_rejects(T):
    c = T.Cache(T.CACHE_AFFINE, 1, 2, 128, 128, 64, 4, 4)
    k = T.DeviceArray.of(kv_bf16((1, 2, 4, 128), 1))
    c.append(k.ptr, k.ptr, 4)
    q = T.DeviceArray.of(kv_bf16((1, 4, 8, 128), 2))
    out = T.DeviceArray((1, 4, 8, 128), np.uint16)
    with pytest.raises(T.TqkvError) as e:
        c.prefill_attend(q.ptr, 4, 8, 1.0, out.ptr)  # 8 queries, 4 tokens appended
    assert e.value.status == T.EINVAL_SHAPE


@pytest.mark.parametrize("case", [0, 1, 3, 4, 5, 7, 9, 10, 12, 13])
def test_prefill_dequantize_once_is_bit_identical(T, monkeypatch, case):
    # Keys dequantized once into scratch (mlx::dequantize's bits) and then
    # copied into LDS give the same bf16 operands as dequantizing them in
    # every row block: the outputs must agree bit for bit, and with the
    # oracle to the bar.
    B, H, Hkv, D, L, N, bk, bv, gs, q_start, k_start, causal, window, scale = PREFILL_CASES[case]
    seed = 4099 + case
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    q = kv_bf16((B, H, L, D), seed)
    k = kv_bf16((B, Hkv, N, D), seed + 1, frac=0.01, mult=10.0)
    v = kv_bf16((B, Hkv, N, D), seed + 2, frac=0.01, mult=10.0)
    if scale == 1.0:
        q = O.bf16_from_f32(O.bf16_to_f32(q) / np.sqrt(D))
    (kh, kd), (vh, vd) = _cache(k, gs, bk, N + 5), _cache(v, gs, bv, N + 5)
    got = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("TQKV_PREFILL_DEQUANT_ONCE", mode)
        got[mode] = run(T, q, [(kd, vd, N + 5, N, False)], B, H, Hkv, L, D, gs, bk, bv, scale,
                        q_start, k_start, causal, window)
    assert np.array_equal(got["0"], got["1"])
    want = want_mlx(q, kh, vh, gs, bk, bv, scale, causal=causal, q_start=q_start,
                    first_held=k_start, window=window)
    check(got["1"], want, f"once case {case}")


def test_prefill_dequantize_once_two_segments_by_default(T, monkeypatch):
    # 512 positions x 4 heads = 8 row blocks a KV head: the default picks the
    # dequantize-once path; a shared prefix segment (batch stride 0) plus
    # per-row suffixes, windowed, against the in-block path and the oracle.
    monkeypatch.delenv("TQKV_PREFILL_DEQUANT_ONCE", raising=False)
    B, H, Hkv, D, L, gs, bk, bv = 2, 16, 4, 128, 512, 64, 8, 4
    P, S = 300, 600
    q = kv_bf16((B, H, L, D), 21)
    kp = kv_bf16((1, Hkv, P, D), 22, frac=0.01, mult=10.0)
    vp = kv_bf16((1, Hkv, P, D), 23)
    ks = kv_bf16((B, Hkv, S, D), 24, frac=0.01, mult=10.0)
    vs = kv_bf16((B, Hkv, S, D), 25)
    (kph, kpd), (vph, vpd) = _cache(kp, gs, bk), _cache(vp, gs, bv)
    (ksh, ksd), (vsh, vsd) = _cache(ks, gs, bk, S + 3), _cache(vs, gs, bv, S + 3)
    scale = 1.0 / np.sqrt(D)
    segs = [(kpd, vpd, P, P, True), (ksd, vsd, S + 3, S, False)]
    got = run(T, q, segs, B, H, Hkv, L, D, gs, bk, bv, scale, P + S - L, 0, True, 700)
    monkeypatch.setenv("TQKV_PREFILL_DEQUANT_ONCE", "0")
    ref = run(T, q, segs, B, H, Hkv, L, D, gs, bk, bv, scale, P + S - L, 0, True, 700)
    assert np.array_equal(got, ref)
    cat = lambda a, b: np.concatenate([np.broadcast_to(a, (B,) + a.shape[1:]), b], axis=2)
    kh = tuple(cat(a, b) for a, b in zip(kph, ksh))
    vh = tuple(cat(a, b) for a, b in zip(vph, vsh))
    want = want_mlx(q, kh, vh, gs, bk, bv, scale, causal=True, q_start=P + S - L,
                    first_held=0, window=700)
    check(got, want, "once, two segments")


@pytest.mark.parametrize("N", [1024, 1021])
def test_prefill_with_caller_workspace(T, monkeypatch, N):
    """tqkv_prefill_attend_affine_ws: with a workspace that holds the
    dequantized rows, without one (every block dequantizes), and after the
    library's scratch is released: the same bits as the library-scratch
    entry. 1021 keys end in a partial V tile (the slab pads to 1024)."""
    monkeypatch.delenv("TQKV_PREFILL_DEQUANT_ONCE", raising=False)
    B, H, Hkv, D, L, gs, bk, bv = 1, 32, 8, 128, 256, 64, 4, 4
    q = kv_bf16((B, H, L, D), 31)
    k = kv_bf16((B, Hkv, N, D), 32, frac=0.01, mult=10.0)
    v = kv_bf16((B, Hkv, N, D), 33, frac=0.01, mult=10.0)
    (_, kd), (_, vd) = _cache(k, gs, bk, N), _cache(v, gs, bv, N)
    segs_host = [(kd, vd, N, N, False)]
    scale = D ** -0.5
    want = run(T, q, segs_host, B, H, Hkv, L, D, gs, bk, bv, scale, N - L, 0, True, -1)
    T.scratch_release()
    need = T.prefill_workspace_size(B, Hkv, D, N)
    # Head dim 128 keeps V as 64-key tiles: a slab rounds up to whole tiles.
    assert need == 2 * B * Hkv * 1024 * D * 2
    assert T.prefill_workspace_size(B, Hkv, 64, N) == 2 * B * Hkv * N * 64 * 2
    dq = T.DeviceArray.of(q)
    segs = [T.affine_seg(tuple(a.ptr for a in kk), tuple(a.ptr for a in vv), c, n, sh)
            for (kk, vv, c, n, sh) in segs_host]
    for ws_bytes in (need, need - 1, 0):
        ws = T.DeviceArray((max(ws_bytes, 1),), np.uint8) if ws_bytes else None
        out = T.DeviceArray((B, H, L, D), np.uint16, np.full((B, H, L, D), 0x7FC0, np.uint16))
        T.prefill_attend_affine_ws(dq.ptr, B, H, Hkv, L, D, gs, bk, bv, scale, segs, out.ptr,
                                   None if ws is None else ws.ptr, ws_bytes, N - L, 0, True, -1)
        T.hip().sync()
        assert np.array_equal(out.numpy(), want), f"workspace of {ws_bytes} bytes"
