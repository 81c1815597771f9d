"""Seeded synthetic inputs shared by the parity tests: bf16 N(0,1) with a
fixed set of outlier channels scaled up, as BASELINE.json's configs describe."""
import numpy as np

import oracle_lib as O


def outlier_channels(dim, frac, seed):
    n = max(1, int(round(frac * dim))) if frac > 0 else 0
    return np.random.default_rng(seed ^ 0x0C0FFEE).permutation(dim)[:n]


def kv_bf16(shape, seed, frac=0.0, mult=1.0, std=1.0):
    """bf16 bit patterns of N(0, std^2) values, channels in the outlier set x mult."""
    x = np.random.default_rng(seed).standard_normal(shape).astype(np.float32) * np.float32(std)
    if frac > 0:
        x[..., outlier_channels(shape[-1], frac, seed)] *= np.float32(mult)
    return O.bf16_from_f32(x)


def grid_bf16(shape, seed):
    """The reference's golden-test inputs: bf16 of a 2^-22 grid in [-2, 2)
    (golden_tests.rs:37-45), rich in exact rounding ties."""
    r = np.random.default_rng(seed).integers(0, 1 << 24, size=shape, dtype=np.int64)
    return O.bf16_from_f32((r.astype(np.float32) / np.float32(1 << 22)) - np.float32(2.0))
