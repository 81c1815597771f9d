"""TurboQuant codebook format on the GPU, through the C ABI, against the
oracle's restatement of lumen-core (compressor.rs, simple.rs):

- tqkv_tq_encode is bit-exact with compress_one given the same R and Phi:
  codes, scale, residual norm and QJL sign words, f32 and bf16 inputs,
  outlier channels, an all-zero vector (the sigma < 1e-10 branch);
- the KVCache API (tqkv_kvcache_*) stores, scores and accumulates values
  bit-exactly as SimpleCache does, keeps seq_len / truncate / clear /
  memory_bytes semantics, and meets the reference's own SimpleCache bars
  (value cosine > 0.95, compression > 2x; simple.rs:151-310).
"""
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


def tables(T, dim, bits, m, seed=42):
    R = T.rotation_matrix(dim, seed)
    phi = T.qjl_matrix(dim, max(m, 1), seed + 1)
    b, c = T.lloyd_max(bits)
    return R, phi, b, c


def inputs_f32(n, dim, seed):
    x = np.random.default_rng(seed).standard_normal((n, dim)).astype(np.float32)
    x[:, np.random.default_rng(seed + 1).permutation(dim)[:max(1, dim // 50)]] *= 8.0
    x[n // 2] = 0.0  # degenerate vector: all codes 0, scale 0
    return x


@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("m", [0, 64, 100])
@pytest.mark.parametrize("bf16_in", [False, True])
def test_encode_bit_exact(T, dim, bits, m, bf16_in):
    print(f"[tq-encode] dim={dim} bits={bits} m={m} bf16={bf16_in}", flush=True)
    n = 37
    R, phi, b, c = tables(T, dim, bits, m)
    x = inputs_f32(n, dim, dim + bits + m)
    if bf16_in:
        xb = O.bf16_from_f32(x)
        x = O.bf16_to_f32(xb)
        dx = T.DeviceArray.of(xb)
    else:
        dx = T.DeviceArray.of(x)
    W = (m + 31) // 32
    dR, dphi = T.DeviceArray.of(R), T.DeviceArray.of(phi)
    db, dc = T.DeviceArray.of(b), T.DeviceArray.of(c.astype(np.float32))
    codes = T.DeviceArray((n, dim), np.uint8)
    sigma = T.DeviceArray((n,), np.float32)
    signs = T.DeviceArray((n, max(W, 1)), np.uint32, np.zeros((n, max(W, 1)), np.uint32))
    rnorm = T.DeviceArray((n,), np.float32, np.zeros(n, np.float32))
    T.tq_encode(dx.ptr, bf16_in, 1, n, dim, dR.ptr, db.ptr, dc.ptr, bits, dphi.ptr, m,
                codes.ptr, sigma.ptr, signs.ptr, rnorm.ptr)
    T.hip().sync()
    comp = O.Compressor(dim, bits, max(m, 1), R, phi[:max(m, 1)])
    s1, s2, rn, sc = comp.compress(x)
    got_codes = codes.numpy()
    packed = np.stack([O.pack_codes(got_codes[i], bits) for i in range(n)])
    assert np.array_equal(packed, s1), "codes"
    assert np.array_equal(sigma.numpy().view(np.uint32), sc.view(np.uint32)), "scale"
    assert np.all(got_codes[n // 2] == 0) and sigma.numpy()[n // 2] == 0.0
    if m > 0:
        assert np.array_equal(rnorm.numpy().view(np.uint32), rn.view(np.uint32)), "residual norm"
        words = signs.numpy()[:, :W]
        want = s2.view(np.uint32).reshape(n, -1)[:, :W]
        assert np.array_equal(words, want), "QJL signs"


def test_encode_writes_into_cache_rows(T):
    dim, bits, m = 128, 4, 64
    R, phi, b, c = tables(T, dim, bits, m)
    x = inputs_f32(2 * 5, dim, 7).reshape(2, 5, dim)
    dx = T.DeviceArray.of(x)
    dR, dphi, db, dc = (T.DeviceArray.of(a) for a in (R, phi, b, c.astype(np.float32)))
    cap = 12
    codes = T.DeviceArray((2, cap, dim), np.uint8, np.full((2, cap, dim), 0xAB, np.uint8))
    sigma = T.DeviceArray((2, cap), np.float32, np.full((2, cap), -1.0, np.float32))
    signs = T.DeviceArray((2, cap, 2), np.uint32)
    rnorm = T.DeviceArray((2, cap), np.float32)
    T.tq_encode(dx.ptr, False, 2, 5, dim, dR.ptr, db.ptr, dc.ptr, bits, dphi.ptr, m, codes.ptr,
                sigma.ptr, signs.ptr, rnorm.ptr, cap, 6)
    T.hip().sync()
    comp = O.Compressor(dim, bits, m, R, phi)
    s1, _, _, sc = comp.compress(x.reshape(-1, dim))
    got = codes.numpy()
    for i in range(2):
        for j in range(5):
            assert np.array_equal(O.pack_codes(got[i, 6 + j], bits), s1[i * 5 + j])
    assert np.all(got[:, :6] == 0xAB) and np.all(got[:, 11:] == 0xAB)
    assert np.all(sigma.numpy()[:, :6] == -1.0)


def _encode_rows(T, dim, bits, m, x_dev, bf16_in, slabs, s, cap, start, tabs, env):
    import os
    dR, dphi, db, dc = tabs
    W = max((m + 31) // 32, 1)
    codes = T.DeviceArray((slabs, cap, dim), np.uint8, np.full((slabs, cap, dim), 0xAB, np.uint8))
    sigma = T.DeviceArray((slabs, cap), np.float32, np.full((slabs, cap), -1.0, np.float32))
    signs = T.DeviceArray((slabs, cap, W), np.uint32, np.full((slabs, cap, W), 0xCDCDCDCD, np.uint32))
    rnorm = T.DeviceArray((slabs, cap), np.float32, np.full((slabs, cap), -1.0, np.float32))
    old = os.environ.get("TQKV_TQ_ENCODE_LANE")
    os.environ["TQKV_TQ_ENCODE_LANE"] = env
    try:
        T.tq_encode(x_dev.ptr, bf16_in, slabs, s, dim, dR.ptr, db.ptr, dc.ptr, bits, dphi.ptr, m,
                    codes.ptr, sigma.ptr, signs.ptr, rnorm.ptr, cap, start)
        T.hip().sync()
    finally:
        if old is None:
            del os.environ["TQKV_TQ_ENCODE_LANE"]
        else:
            os.environ["TQKV_TQ_ENCODE_LANE"] = old
    return codes.numpy(), sigma.numpy(), signs.numpy(), rnorm.numpy()


@pytest.mark.parametrize("dim,bits,m", [(64, 8, 200), (128, 3, 100), (128, 4, 64), (128, 8, 0),
                                        (64, 2, 31)])
def test_encode_lane_kernel_many_rows(T, dim, bits, m):
    """The four-lanes-per-row kernel (D <= 128) over several 128-row blocks, a
    ragged last block, slab-to-cache-row mapping, Phi longer than one LDS
    chunk (m > D): bit-exact with the oracle and with the wavefront-per-row
    kernel, rows outside [start, start + s) untouched."""
    slabs, s, cap, start = 3, 211, 240, 17
    print(f"[tq-encode-lane] dim={dim} bits={bits} m={m} rows={slabs * s}", flush=True)
    R, phi, b, c = tables(T, dim, bits, m)
    x = inputs_f32(slabs * s, dim, 1000 + dim + bits + m)
    xb = O.bf16_from_f32(x)
    x = O.bf16_to_f32(xb)
    dx = T.DeviceArray.of(xb.reshape(slabs, s, dim))
    tabs = tuple(T.DeviceArray.of(a) for a in (R, phi, b, c.astype(np.float32)))
    lane = _encode_rows(T, dim, bits, m, dx, True, slabs, s, cap, start, tabs, "1")
    wave = _encode_rows(T, dim, bits, m, dx, True, slabs, s, cap, start, tabs, "0")
    for a, w in zip(lane, wave):
        assert np.array_equal(a.view(np.uint8), w.view(np.uint8)), "lane vs wavefront kernel"
    codes, sigma, signs, rnorm = lane
    comp = O.Compressor(dim, bits, max(m, 1), R, phi[:max(m, 1)])
    s1, s2, rn, sc = comp.compress(x)
    rows = slice(start, start + s)
    got = codes[:, rows].reshape(-1, dim)
    packed = np.stack([O.pack_codes(got[i], bits) for i in range(slabs * s)])
    assert np.array_equal(packed, s1), "codes"
    assert np.array_equal(sigma[:, rows].reshape(-1).view(np.uint32), sc.view(np.uint32)), "scale"
    if m > 0:
        W = (m + 31) // 32
        assert np.array_equal(rnorm[:, rows].reshape(-1).view(np.uint32), rn.view(np.uint32))
        want = s2.view(np.uint32).reshape(slabs * s, -1)[:, :W]
        assert np.array_equal(signs[:, rows].reshape(-1, W), want), "QJL signs"
    assert np.all(codes[:, :start] == 0xAB) and np.all(codes[:, start + s:] == 0xAB)
    assert np.all(sigma[:, :start] == -1.0) and np.all(sigma[:, start + s:] == -1.0)


def test_kvcache_matches_simple_cache(T):
    dim, bits, m, layers, heads = 128, 3, 64, 2, 2
    kv = T.KVCache(dim, bits, m, 42, layers, heads)
    R, phi, _, _ = tables(T, dim, bits, m)
    comp = O.Compressor(dim, bits, m, R, phi)
    rng = np.random.default_rng(5)
    K = rng.standard_normal((40, dim)).astype(np.float32)
    V = rng.standard_normal((40, dim)).astype(np.float32)
    kv.store(1, 0, K[:25], V[:25])
    kv.store(1, 0, K[25:], V[25:])  # appends, like two store() calls
    assert kv.seq_len(1, 0) == 40 and kv.seq_len(0, 0) == 0 and kv.seq_len(1, 1) == 0
    ck, cv = comp.compress(K), comp.compress(V)
    codes, scale, signs, rn = kv.read(1, 0)
    assert np.array_equal(np.stack([O.pack_codes(r, bits) for r in codes]), ck[0])
    assert np.array_equal(scale.view(np.uint32), ck[3].view(np.uint32))
    q = rng.standard_normal(dim).astype(np.float32)
    s = kv.attend_keys(1, 0, q)
    assert np.array_equal(s.view(np.uint32), comp.scores(q, ck).view(np.uint32))
    w = np.exp(s - s.max())
    w /= w.sum()
    w[3] = 1e-12  # below the skip threshold
    out = kv.attend_values(1, 0, w)
    assert np.array_equal(out.view(np.uint32), comp.attend_values(w, cv).view(np.uint32))
    # SimpleCache bars: value reconstruction cosine > 0.95 (simple.rs:220),
    # compression over f32 > 2x (:250).
    one = np.zeros(40, np.float32)
    one[7] = 1.0
    rec = kv.attend_values(1, 0, one)
    cos = rec @ V[7] / (np.linalg.norm(rec) * np.linalg.norm(V[7]))
    assert cos > 0.95
    assert 2 * 40 * dim * 4 / kv.memory_bytes() > 2.0
    # memory_bytes is CompressedVector::size_bytes summed (config.rs:50-55):
    # 128 3-bit codes at 21 a word take 7 words (56 bytes), one u64 of QJL
    # bits, 20 bytes of fields, 80 vectors. The device holds the packed
    # words, the scale, two u32 sign words and the residual norm of each.
    assert kv.memory_bytes() == 80 * (56 + 8 + 20)
    held, reserved = kv.device_bytes()
    assert held == 80 * (56 + 4 + 8 + 4), held
    assert 2 * 40 * dim * 4 / held > 2.0 and reserved > held
    # truncate keeps the first n_keep of every head of the layer; clear empties.
    kv.store(1, 1, K[:10], V[:10])
    kv.truncate(1, 12)
    assert (kv.seq_len(1, 0), kv.seq_len(1, 1)) == (12, 10)
    assert np.array_equal(kv.attend_keys(1, 0, q).view(np.uint32), s[:12].view(np.uint32))
    kv.clear()
    assert kv.seq_len(1, 0) == 0 and kv.memory_bytes() == 0 and kv.device_bytes()[0] == 0
    with pytest.raises(T.TqkvError) as e:
        kv.store(2, 0, K[:1], V[:1])
    assert e.value.status == T.EINVAL_ARG


def test_kvcache_from_given_tables(T):
    # from_files: an external R (here the oracle's own seed-7 matrix) is
    # used as given.
    dim, bits, m = 64, 4, 32
    R = O.rotation(dim, 7)
    phi = O.qjl_matrix(dim, m, 8)
    kv = T.KVCache(dim, bits, m, 0, 1, 1, rotation=R, qjl=phi)
    x = np.random.default_rng(9).standard_normal((11, dim)).astype(np.float32)
    kv.store(0, 0, x, x)
    comp = O.Compressor(dim, bits, m, R, phi)
    s1, s2, rn, sc = comp.compress(x)
    codes, scale, signs, rnorm = kv.read(0, 0)
    assert np.array_equal(np.stack([O.pack_codes(r, bits) for r in codes]), s1)
    assert np.array_equal(signs, s2.view(np.uint32).reshape(11, -1)[:, :1])
    assert np.array_equal(rnorm.view(np.uint32), rn.view(np.uint32))


@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("transpose", [False, True])
def test_rotate_bf16(T, dim, transpose):
    """tqkv_rotate_bf16 (the GPU path's rotate_last_axis, turboquant.rs:258-267:
    y = x R, or x R^T): the four-lanes-per-row kernel (D <= 128, several blocks and a
    ragged last one) bit-identical to the block-per-row kernel, and both
    within one bf16 rounding of the f64 product."""
    import os
    rows = 333
    print(f"[rotate] dim={dim} transpose={transpose} rows={rows}", flush=True)
    R = T.rotation_matrix(dim, 42)
    xb = kv_bf16((rows, dim), 5, frac=0.02, mult=8.0)
    dx, dR = T.DeviceArray.of(xb), T.DeviceArray.of(R)
    outs = []
    for env in ("1", "0"):
        y = T.DeviceArray((rows, dim), np.uint16, np.zeros((rows, dim), np.uint16))
        old = os.environ.get("TQKV_TQ_ENCODE_LANE")
        os.environ["TQKV_TQ_ENCODE_LANE"] = env
        try:
            T.rotate_bf16(dx.ptr, rows, dim, dR.ptr, transpose, y.ptr)
            T.hip().sync()
        finally:
            if old is None:
                del os.environ["TQKV_TQ_ENCODE_LANE"]
            else:
                os.environ["TQKV_TQ_ENCODE_LANE"] = old
        outs.append(y.numpy())
    assert np.array_equal(outs[0], outs[1]), "lane vs block-per-row kernel"
    x = O.bf16_to_f32(xb).astype(np.float64)
    M = R.astype(np.float64)
    want = x @ (M.T if transpose else M)
    got = O.bf16_to_f32(outs[0]).astype(np.float64)
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-5)


# ------------------------------------------------- the GPU cache's encode
@pytest.mark.parametrize("mode,transpose", [(0, False), (1, False), (2, False), (2, True)])
@pytest.mark.parametrize("bits,D", [(4, 128), (3, 256), (8, 64), (2, 512), (6, 128)])
def test_gpu_path_encode_bit_exact(T, mode, transpose, bits, D):
    # tqkv_tq_encode_gpu_path against the oracle's restatement, rows written
    # into the middle of a larger buffer.
    slabs, s, cap, start = 3, 37, 50, 6
    print(f"[tq-gpu-path] mode={mode} transpose={transpose} bits={bits} D={D}", flush=True)
    x = O.bf16_from_f32(np.random.default_rng(D + bits + mode).standard_normal(
        (slabs, s, D)).astype(np.float32) * 3)
    R = T.rotation_matrix(D, 42)
    b, _ = T.lloyd_max(bits)
    inner = np.asarray(b[1:-1]).astype(np.float32)
    dx, dR, di = T.DeviceArray.of(x), T.DeviceArray.of(R), T.DeviceArray.of(inner)
    codes = T.DeviceArray((slabs, cap, D), np.uint8, np.full((slabs, cap, D), 0xAB, np.uint8))
    sigma = T.DeviceArray((slabs, cap), np.float32, np.full((slabs, cap), -7.0, np.float32))
    T.tq_encode_gpu_path(dx.ptr, slabs, s, D, dR.ptr, mode, transpose, di.ptr, bits, codes.ptr,
                         sigma.ptr, cap, start)
    T.hip().sync()
    wc, ws = O.tq_encode_gpu_path(x.reshape(-1, D), inner, R, mode=mode, transpose=transpose)
    gc, gs = codes.numpy(), sigma.numpy()
    assert np.array_equal(gc[:, start:start + s].reshape(-1, D), wc)
    assert np.array_equal(gs[:, start:start + s].reshape(-1).view(np.uint32), ws.view(np.uint32))
    assert np.all(gc[:, :start] == 0xAB) and np.all(gc[:, start + s:] == 0xAB)
    assert np.all(gs[:, :start] == -7.0) and np.all(gs[:, start + s:] == -7.0)


def test_gpu_path_fused_matches_rotate_then_encode(T):
    # The reference's own test of its rotate+encode kernel
    # (turboquant.rs:1385-1456), on the device outputs: [1, 8, 64, 256] bf16
    # N(0,1), 4 bits, seed-42 rotation; mode 2 against mode 1.
    D, bits, rows = 256, 4, 8 * 64
    x = O.bf16_from_f32(np.random.default_rng(0xABCDEF01).standard_normal((rows, D)).astype(
        np.float32))
    R = T.rotation_matrix(D, 42)
    b, cent = T.lloyd_max(bits)
    inner = np.asarray(b[1:-1]).astype(np.float32)
    dx, dR, di = T.DeviceArray.of(x), T.DeviceArray.of(R), T.DeviceArray.of(inner)
    out = {}
    for mode in (1, 2):
        c = T.DeviceArray((rows, D), np.uint8)
        s = T.DeviceArray((rows,), np.float32)
        T.tq_encode_gpu_path(dx.ptr, 1, rows, D, dR.ptr, mode, False, di.ptr, bits, c.ptr, s.ptr)
        T.hip().sync()
        out[mode] = (c.numpy(), s.numpy())
    (c1, s1), (c2, s2) = out[1], out[2]
    cf = cent.astype(np.float32)
    dq = lambda c, s: O.bf16_to_f32(O.bf16_from_f32(cf[c] * s[:, None]))
    sig_mse = float(np.mean((s1 - s2) ** 2))
    agree = float(np.mean(c1 == c2))
    dq_mse = float(np.mean((dq(c1, s1) - dq(c2, s2)) ** 2))
    print(f"[tq-gpu-path] sigma MSE {sig_mse:.3e}, agreement {agree:.4f}, V_dq MSE {dq_mse:.3e}",
          flush=True)
    assert sig_mse < 1e-3 and agree > 0.99 and dq_mse < 1e-2


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("dim", [1, 21, 64, 100, 128, 512])
def test_pack_codes_matches_bitpack(T, bits, dim):
    """tqkv_pack_codes / tqkv_unpack_codes against the oracle's restatement
    of bitpack::pack_codes / unpack_codes (bitpack.rs:11-52), itself pinned
    to the reference's round-trip and size tests: word for word, unused high
    bits zero, and back to the same codes."""
    n = 37
    print(f"[pack] bits={bits} dim={dim} n={n}", flush=True)
    codes = np.random.default_rng(bits * 1000 + dim).integers(0, 1 << bits, (n, dim),
                                                               dtype=np.uint8)
    pw = T.packed_words(dim, bits)
    assert pw == O.lib().oracle_packed_words(dim, bits) == -(-dim // (64 // bits))
    want = np.stack([O.pack_codes(r, bits) for r in codes])
    dc = T.DeviceArray.of(codes)
    dw = T.DeviceArray((n, pw), np.uint64, np.full((n, pw), 0xA5A5A5A5A5A5A5A5, np.uint64))
    T.pack_codes(dc.ptr, n, dim, bits, dw.ptr)
    T.hip().sync()
    assert np.array_equal(dw.numpy(), want)
    back = T.DeviceArray((n, dim), np.uint8, np.full((n, dim), 0xEE, np.uint8))
    T.unpack_codes(dw.ptr, n, dim, bits, back.ptr)
    T.hip().sync()
    assert np.array_equal(back.numpy(), codes)


def test_pack_codes_rejects_bad_shapes(T):
    assert T.packed_words(64, 0) == -1 and T.packed_words(64, 9) == -1
    assert T.packed_words(0, 3) == -1
    for bits, dim, status in [(0, 64, T.EUNSUPPORTED), (9, 64, T.EUNSUPPORTED),
                              (3, 0, T.EINVAL_SHAPE)]:
        with pytest.raises(T.TqkvError) as e:
            T.pack_codes(None, 1, dim, bits, None)
        assert e.value.status == status
    with pytest.raises(T.TqkvError) as e:
        T.pack_codes(None, 4, 64, 3, None)
    assert e.value.status == T.EINVAL_ARG
    T.pack_codes(None, 0, 64, 3, None)  # nothing to pack


@pytest.mark.parametrize("dim,bits", [(64, 2), (128, 3), (128, 4), (256, 5), (64, 8), (128, 1)])
def test_packed_estimators_match_unpacked(T, dim, bits):
    """tqkv_tq_scores_packed / tqkv_tq_values_packed read the packed words
    and give the u8-code kernels' results bit for bit (same sums, same
    order), and those equal the oracle's SimpleCache estimators."""
    n, m = 53, 0
    print(f"[packed-est] dim={dim} bits={bits} n={n}", flush=True)
    R, phi, b, c = tables(T, dim, bits, m)
    comp = O.Compressor(dim, bits, 1, R, phi[:1])
    x = inputs_f32(n, dim, 77 + bits)
    ck = comp.compress(x)
    codes = np.stack([O.unpack_codes(w, dim, bits) for w in ck[0]])
    sigma = ck[3].astype(np.float32)
    cent = c.astype(np.float32)
    dR, dcent = T.DeviceArray.of(R), T.DeviceArray.of(cent)
    dcodes, dsig = T.DeviceArray.of(codes), T.DeviceArray.of(sigma)
    dw = T.DeviceArray.of(np.ascontiguousarray(ck[0]))
    rng = np.random.default_rng(dim + bits)
    q = rng.standard_normal(dim).astype(np.float32)
    dq = T.DeviceArray.of(q)
    rq = T.DeviceArray((dim,), np.float32)
    T.tq_rotate_query(dR.ptr, dq.ptr, dim, rq.ptr)
    s_u8 = T.DeviceArray((n,), np.float32)
    s_pk = T.DeviceArray((n,), np.float32)
    T.check(T.lib().tqkv_tq_scores(rq.ptr, dcodes.ptr, dsig.ptr, dcent.ptr, dim, n, s_u8.ptr,
                                   None))
    T.tq_scores_packed(rq.ptr, dw.ptr, dsig.ptr, dcent.ptr, bits, dim, n, s_pk.ptr)
    T.hip().sync()
    a, p = s_u8.numpy(), s_pk.numpy()
    assert np.array_equal(a.view(np.uint32), p.view(np.uint32))
    assert np.array_equal(p.view(np.uint32), comp.scores(q, ck).view(np.uint32))
    w = rng.random(n).astype(np.float32)
    w[5] = 0.0
    dwt = T.DeviceArray.of(w)
    o_u8 = T.DeviceArray((dim,), np.float32)
    o_pk = T.DeviceArray((dim,), np.float32)
    T.check(T.lib().tqkv_tq_values(dR.ptr, dcodes.ptr, dsig.ptr, dcent.ptr, dwt.ptr, dim, n,
                                   o_u8.ptr, None))
    T.tq_values_packed(dR.ptr, dw.ptr, dsig.ptr, dcent.ptr, dwt.ptr, bits, dim, n, o_pk.ptr)
    T.hip().sync()
    a, p = o_u8.numpy(), o_pk.numpy()
    assert np.array_equal(a.view(np.uint32), p.view(np.uint32))
    assert np.array_equal(p.view(np.uint32), comp.attend_values(w, ck).view(np.uint32))
