"""The library's host-side codebook tables (no GPU): Lloyd-Max bit-identical
to the oracle's restatement of lloyd_max.rs (which the Max 1960 tables and
the reference's thresholds pin, test_oracle_codec.py), the seeded Haar
rotation orthogonal and deterministic (rotation.rs:153-249), the QJL matrix
N(0, 1/m)."""
import numpy as np
import pytest

import oracle_lib as O


@pytest.fixture(scope="module")
def T():
    import tqkv
    return tqkv


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
def test_lloyd_max_is_bit_identical(T, bits):
    b, c = T.lloyd_max(bits)
    wb, wc, _ = O.codebook(bits)
    assert np.array_equal(b.view(np.uint64), wb.view(np.uint64))
    assert np.array_equal(c.view(np.uint64), wc.view(np.uint64))


def test_lloyd_max_three_bit_is_max_1960(T):
    _, c = T.lloyd_max(3)
    assert np.allclose(c[4:], [0.2451, 0.7560, 1.3440, 2.1520], atol=2e-3)
    with pytest.raises(T.TqkvError) as e:
        T.lloyd_max(9)
    assert e.value.status == T.EUNSUPPORTED


@pytest.mark.parametrize("dim", [16, 64, 128])
def test_rotation_is_haar_orthogonal_and_seeded(T, dim):
    R = T.rotation_matrix(dim, 42).astype(np.float64)
    assert np.abs(R @ R.T - np.eye(dim)).max() < 1e-5        # rotation.rs:153-170
    assert np.array_equal(T.rotation_matrix(dim, 42), T.rotation_matrix(dim, 42))
    assert not np.array_equal(T.rotation_matrix(dim, 42), T.rotation_matrix(dim, 43))
    x = np.random.default_rng(dim).standard_normal(dim)
    assert abs(np.linalg.norm(R @ x) - np.linalg.norm(x)) < 1e-4 * np.linalg.norm(x)
    # The same algorithm and stream as the oracle's restatement.
    assert np.array_equal(T.rotation_matrix(dim, 42), O.rotation(dim, 42))


def test_qjl_matrix(T):
    P = T.qjl_matrix(128, 512, 43)
    assert np.array_equal(P, O.qjl_matrix(128, 512, 43))
    assert abs(P.std() * np.sqrt(512) - 1.0) < 0.02 and abs(P.mean()) < 1e-3
