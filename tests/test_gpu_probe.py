"""The measurement kernels: the read probe (bandwidth.rs:73-100's sum of a
float array) against a float64 sum of the same values, and the empty launch
the bench times for the launch floor."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def T():
    import tqkv
    assert tqkv.hip().device_count() > 0, "no GPU visible"
    return tqkv


@pytest.mark.parametrize("n", [4, 1024, 4 * 257 * 256 * 8 + 12, 1 << 22])
def test_read_probe_sums_every_float(T, n):
    print(f"[read-probe] n={n}", flush=True)
    x = np.random.default_rng(n).uniform(-1.0, 1.0, n).astype(np.float32)
    dx = T.DeviceArray.of(x)
    scratch = T.DeviceArray((4096,), np.float32)
    out = T.DeviceArray((1,), np.float32, np.full(1, np.nan, np.float32))
    T.read_probe(dx.ptr, n * 4, scratch.ptr, 4096 * 4, out.ptr)
    T.hip().sync()
    got = float(out.numpy()[0])
    want = float(np.sum(x.astype(np.float64)))
    # Every partial sum of k floats in [-1, 1] is off by at most k * 2^-24
    # per addition level; the tree depth is well under 64.
    assert abs(got - want) <= 64 * 2.0 ** -24 * float(np.sum(np.abs(x))) + 1e-6


def test_read_probe_refuses_misaligned(T):
    scratch = T.DeviceArray((4096,), np.float32)
    out = T.DeviceArray((1,), np.float32)
    dx = T.DeviceArray((64,), np.float32)
    with pytest.raises(T.TqkvError):
        T.read_probe(dx.ptr, 60, scratch.ptr, 4096 * 4, out.ptr)
    with pytest.raises(T.TqkvError):
        T.read_probe(dx.ptr, 64, scratch.ptr, 4, out.ptr)


def test_empty_launch(T):
    for wg in (1, 256, 4096):
        T.empty_launch(wg)
    T.hip().sync()
    with pytest.raises(T.TqkvError):
        T.empty_launch(0)
