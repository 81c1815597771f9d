"""The oracle's codec (lumen-core restatement) against closed forms, the
reference's known answers and thresholds, and independent numpy computations."""
import math

import numpy as np
import pytest

import oracle_lib as O
from oracle_lib import lib, ptr


# ------------------------------------------------------------------ Lloyd-Max
def test_one_bit_codebook_is_the_closed_form():
    # N(0,1), 2 levels: centroids +-sqrt(2/pi), MSE 1 - 2/pi. The A&S erf
    # approximation (|err| < 1.5e-7) bounds how close the EM lands.
    b, c, mse = O.codebook(1)
    assert abs(c[1] - math.sqrt(2 / math.pi)) < 1e-6
    assert c[0] == -c[1]
    assert b[1] == 0.0 and b[0] == -math.inf and b[2] == math.inf
    assert abs(mse - (1 - 2 / math.pi)) < 1e-6


@pytest.mark.parametrize("bits,centroids,mse_want", [
    # Max (1960), Table I, optimum quantizer for N(0,1)
    (2, [0.4528, 1.510], 0.1175),
    (3, [0.2451, 0.7560, 1.344, 2.152], 0.03454),
])
def test_codebook_matches_max_1960(bits, centroids, mse_want):
    b, c, mse = O.codebook(bits)
    n = 1 << bits
    pos = c[n // 2:]
    assert np.allclose(pos, centroids, atol=1.5e-3), pos
    assert abs(mse - mse_want) < 2e-4


def test_codebook_reference_thresholds():
    # lloyd_max.rs:216-322
    b, c, mse = O.codebook(3)
    assert mse <= 0.035
    for i in range(4):
        assert abs(c[i] + c[7 - i]) < 1e-10
    codes = np.empty(8, np.uint8)
    lib().oracle_codebook_quantize(3, ptr(np.ascontiguousarray(c)), 8, ptr(codes))
    assert list(codes) == list(range(8))
    _, _, mse4 = O.codebook(4)
    assert mse4 < 0.01


def test_codebook_empirical_mse_matches_analytic():
    b, c, mse = O.codebook(3)
    x = np.random.default_rng(123).standard_normal(100_000)
    codes = np.empty(x.size, np.uint8)
    lib().oracle_codebook_quantize(3, ptr(x), x.size, ptr(codes))
    emp = float(np.mean((x - c[codes]) ** 2))
    assert abs(emp - mse) < 0.002 and emp <= 0.036
    # the scan is a partition: searchsorted on the inner boundaries agrees
    assert np.array_equal(codes, np.searchsorted(b[1:-1], x, side="right"))


def test_codebook_boundary_ties_go_up():
    # boundaries[i] <= x < boundaries[i+1] -> code i (lloyd_max.rs:135-143)
    b, c, _ = O.codebook(3)
    xs = np.array([b[i] for i in range(1, 8)] + [np.nextafter(b[i], -np.inf) for i in range(1, 8)])
    codes = np.empty(xs.size, np.uint8)
    lib().oracle_codebook_quantize(3, ptr(xs), xs.size, ptr(codes))
    assert list(codes[:7]) == list(range(1, 8))
    assert list(codes[7:]) == list(range(0, 7))


# ------------------------------------------------------------------ bitpack
def _pack(codes, bits):
    codes = np.ascontiguousarray(codes, np.uint8)
    n = lib().oracle_packed_words(codes.size, bits)
    out = np.zeros(n, np.uint64)
    lib().oracle_pack_codes(ptr(codes), codes.size, bits, ptr(out))
    return out


def test_bitpack_known_answers():
    # bitpack.rs:54-109
    for bits, n, words in [(3, 256, 13), (2, 128, 4), (4, 64, 4)]:
        codes = (np.arange(n) % (1 << bits)).astype(np.uint8)
        packed = _pack(codes, bits)
        assert packed.size == words
        back = np.empty(n, np.uint8)
        lib().oracle_unpack_codes(ptr(packed), n, bits, ptr(back))
        assert np.array_equal(back, codes)
    assert lib().oracle_packed_words(512, 3) == 25
    # LSB first, 21 codes per word at 3 bits, top bit unused
    p = _pack(np.array([5] + [0] * 20 + [3], np.uint8), 3)
    assert p[0] == 5 and p[1] == 3
    p = _pack(np.full(21, 7, np.uint8), 3)
    assert p[0] == (1 << 63) - 1


# ------------------------------------------------------------------ rotation
def test_rotation_is_orthogonal_and_deterministic():
    # rotation.rs:153-249 thresholds
    R = O.rotation(128, 42)
    err = np.abs(R.astype(np.float64) @ R.T.astype(np.float64) - np.eye(128)).max()
    assert err < 1e-5
    assert np.array_equal(R, O.rotation(128, 42))
    assert not np.array_equal(R, O.rotation(128, 43))


def test_rotation_apply_is_sequential_f32():
    # y_i = sum_j R_ij x_j summed left to right in f32, products rounded
    # separately (rotation.rs:91-99): np.cumsum over f32 is exactly that.
    R = O.rotation(64, 7)
    x = np.random.default_rng(1).standard_normal(64).astype(np.float32)
    y = np.empty(64, np.float32)
    lib().oracle_rotation_apply(ptr(R), 64, ptr(x), ptr(y))
    want = np.array([np.cumsum((R[i] * x).astype(np.float32), dtype=np.float32)[-1]
                     for i in range(64)], np.float32)
    assert np.array_equal(y, want)
    back = np.empty(64, np.float32)
    lib().oracle_rotation_apply_inverse(ptr(R), 64, ptr(y), ptr(back))
    assert np.abs(back - x).max() < 1e-4
    assert abs(np.linalg.norm(y) - np.linalg.norm(x)) / np.linalg.norm(x) < 1e-5


# ------------------------------------------------------------------ QJL
def test_qjl_packed_len_and_last_word():
    # qjl.rs:295-320
    for m, w in [(0, 0), (1, 1), (63, 1), (64, 1), (65, 2), (128, 2), (129, 3)]:
        assert lib().oracle_qjl_packed_len(m) == w
    phi = O.qjl_matrix(32, 65, 42)
    r = np.random.default_rng(99).standard_normal(32).astype(np.float32)
    out = np.zeros(2, np.uint64)
    lib().oracle_qjl_project_and_pack(ptr(phi), 65, 32, ptr(r), ptr(out))
    assert int(out[1]) & ~1 == 0
    # bit i is sign(phi_i . r) >= 0
    dots = phi.astype(np.float64) @ r.astype(np.float64)
    bits = [(int(out[i // 64]) >> (i % 64)) & 1 for i in range(65)]
    assert bits == [int(d >= 0) for d in dots]


def test_qjl_estimator_is_unbiased():
    # qjl.rs:180-214: mean error over 2000 trials < 1.0
    dim, m = 128, 256
    phi = O.qjl_matrix(dim, m, 42)
    assert abs(phi.std() * math.sqrt(m) - 1.0) < 0.02
    rng = np.random.default_rng(99)
    err = 0.0
    for _ in range(2000):
        r = rng.standard_normal(dim).astype(np.float32)
        q = rng.standard_normal(dim).astype(np.float32)
        packed = np.zeros(lib().oracle_qjl_packed_len(m), np.uint64)
        lib().oracle_qjl_project_and_pack(ptr(phi), m, dim, ptr(r), ptr(packed))
        est = lib().oracle_qjl_estimate(ptr(phi), m, dim, ptr(q), ptr(packed),
                                        float(np.linalg.norm(r)))
        err += est - float(q @ r)
    assert abs(err / 2000) < 1.0


# ------------------------------------------------------------------ compressor
def _cos(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def _compressor(dim=128, bits=3, m=64, seed=42):
    return O.Compressor(dim, bits, m, O.rotation(dim, seed), O.qjl_matrix(dim, m, seed + 1))


def test_stage1_score_cosine():
    # compressor.rs:253-290: 3-bit stage-1 avg cosine >= 0.98
    c = _compressor()
    rng = np.random.default_rng(99)
    v = rng.standard_normal((200, 128)).astype(np.float32)
    comp = c.compress(v)
    cs = []
    for _ in range(50):
        q = rng.standard_normal(128).astype(np.float32)
        cs.append(_cos(v @ q, c.scores(q, comp)))
    assert np.mean(cs) >= 0.98


def test_two_stage_score_cosine():
    # compressor.rs:292-305: m=512 avg >= 0.99, min >= 0.95
    c = _compressor(m=512)
    rng = np.random.default_rng(99)
    v = rng.standard_normal((200, 128)).astype(np.float32)
    comp = c.compress(v)
    cs = []
    for _ in range(50):
        q = rng.standard_normal(128).astype(np.float32)
        cs.append(_cos(v @ q, c.scores(q, comp, two_stage=True)))
    assert np.mean(cs) >= 0.99 and min(cs) >= 0.95


def test_compress_one_pieces():
    # sigma = ||Rx|| / sqrt(D); codes quantize Rx/sigma; the zero vector gets
    # sigma 0 and all-zero codes (compressor.rs:67-79).
    c = _compressor(dim=64, bits=4, m=64)
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 64)).astype(np.float32)
    x[2] = 0
    s1, s2, rn, sc = c.compress(x)
    y = x[0].astype(np.float64) @ c.R.T.astype(np.float64)
    assert abs(sc[0] - np.linalg.norm(y) / 8) < 1e-5 * sc[0]
    codes = np.empty(64, np.uint8)
    lib().oracle_unpack_codes(ptr(s1[0]), 64, 4, ptr(codes))
    b, cent, _ = O.codebook(4)
    assert np.mean(codes == np.searchsorted(b[1:-1], y / sc[0], side="right")) > 0.98
    assert sc[2] == 0 and int(s1[2].sum()) == 0 and rn[2] == 0


def test_simple_cache_value_reconstruction():
    # simple.rs:151-208: value cosine > 0.95 at 3 bits, D=64
    c = _compressor(dim=64, bits=3, m=64)
    rng = np.random.default_rng(42)
    k = rng.standard_normal((10, 64)).astype(np.float32)
    v = rng.standard_normal((10, 64)).astype(np.float32)
    ck, cv = c.compress(k), c.compress(v)
    q = rng.standard_normal(64).astype(np.float32)
    s = c.scores(q, ck)
    w = np.exp(s) / np.exp(s).sum()
    assert _cos(c.attend_values(w.astype(np.float32), cv), w @ v) > 0.95
    # simple.rs:211-252: compression ratio > 2 (stage1 + stage2 + 4 + 4 + 8 + 4 bytes)
    used = (c.w1 + c.w2) * 8 + 20
    assert 64 * 4 / used > 2.0
