"""The oracle's restatement of the reference GPU cache's TurboQuant encode
(lloyd_max_quantize_stage1 and its rotate variants, turboquant.rs:398-423,
708-745), pinned where the reference pins it:

- closed form: a row of +-a (a a power of two) has sigma = a exactly and
  every y / sigma = +-1, whose code is the number of inner boundaries at or
  below +-1 of the Max (1960) 4-bit table;
- against compress_one (the bit-exact CPU path, itself pinned by the golden
  digests and known answers): with the rotation applied as R x, the codes
  agree on >= 99% of elements (they differ only where bf16(y / sigma) or the
  f32 boundaries move a value across a level) and sigma to 1e-5;
- the reference's own test of its rotate+encode kernel against
  rotate-then-encode (turboquant.rs:1385-1456): sigma MSE < 1e-3, code
  agreement > 0.99, dequantized MSE < 1e-2;
- a planted mistake (boundaries compared with < instead of <=, or y / sigma
  left in f32) changes codes that the tie cases below pin.
Parity beyond these is unpinned: MLX's reduction order for sigma is its own.
"""
import numpy as np
import pytest

import oracle_lib as O


def bf16_normal(shape, seed):
    return O.bf16_from_f32(np.random.default_rng(seed).standard_normal(shape).astype(np.float32))


def test_constant_magnitude_rows_closed_form():
    inner = O.boundaries_inner(4)
    rng = np.random.default_rng(3)
    for a in (0.25, 1.0, 8.0):
        x = (np.where(rng.random((5, 128)) < 0.5, -a, a)).astype(np.float32)
        codes, sigma = O.tq_encode_gpu_path(O.bf16_from_f32(x), inner)
        assert np.all(sigma == np.float32(a))
        up = int(np.sum(inner <= 1.0))
        down = int(np.sum(inner <= -1.0))
        assert np.all(codes == np.where(x > 0, up, down))
    # The Max (1960) 4-bit levels put +-1 in the levels just above and below
    # the middle boundary (0): codes 11 and 4 of 16.
    assert (up, down) == (11, 4)


def test_agrees_with_compress_one():
    D, bits = 128, 4
    R = O.rotation(D, 42)
    phi = O.qjl_matrix(D, 64, 43)
    x = bf16_normal((400, D), 7)
    codes, sigma = O.tq_encode_gpu_path(x, O.boundaries_inner(bits), R, mode=2, transpose=True)
    comp = O.Compressor(D, bits, 64, R, phi)
    s1, _, _, sc = comp.compress(O.bf16_to_f32(x))
    ref = np.stack([O.unpack_codes(r, D, bits) for r in s1])
    agree = np.mean(ref == codes)
    print(f"[tq-gpu-path] agreement with compress_one: {agree:.5f}")
    assert agree >= 0.99
    assert np.allclose(sigma, sc, rtol=1e-5, atol=0)


def test_reference_fused_vs_unfused_bars():
    # turboquant.rs:1385-1456 on the restatement: [1, 8, 64, 256] bf16
    # N(0,1), 4 bits, rotate-then-encode (mode 1) against rotate+encode
    # (mode 2).
    D, bits = 256, 4
    R = O.rotation(D, 42)
    x = bf16_normal((8 * 64, D), 0xABCDEF01)
    inner = O.boundaries_inner(bits)
    c1, s1 = O.tq_encode_gpu_path(x, inner, R, mode=1)
    c2, s2 = O.tq_encode_gpu_path(x, inner, R, mode=2)
    assert np.mean((s1 - s2) ** 2) < 1e-3
    assert np.mean(c1 == c2) > 0.99
    cent = O.codebook(bits)[1].astype(np.float32)
    dq = lambda c, s: O.bf16_to_f32(O.bf16_from_f32(cent[c] * s[:, None]))
    assert np.mean((dq(c1, s1) - dq(c2, s2)) ** 2) < 1e-2


def test_ties_count_boundaries_at_or_below():
    # A value landing exactly on a boundary (as f32 after bf16 rounding)
    # takes the level above it: "b <= x" counts it.
    inner = O.boundaries_inner(2)  # 3 boundaries, the middle one 0
    assert inner[1] == 0.0
    x = np.zeros((1, 64), np.float32)
    x[0, 1::2] = 1.0
    x[0, 0::4] = -1.0  # a row of -1, 0, +1 with zeros on the middle boundary
    codes, _ = O.tq_encode_gpu_path(O.bf16_from_f32(x), inner)
    zeros = codes[0][x[0] == 0.0]
    assert np.all(zeros == 2)  # boundaries -0.98, 0 at or below 0
