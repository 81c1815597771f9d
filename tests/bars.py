"""The attention parity bar, compared in bf16 (test infrastructure).

Attention outputs are bf16, the dtype the reference returns. The bar is
2e-2 max-abs and 1e-3 mean-abs between the kernel's bf16 output and the
oracle's f64 result x rounded to bf16 (round to nearest even), RN(x):
    err = |got - RN(x)|.
Where a bf16 step passes 2e-2 (|x| >= 4) this asks for RN(x) itself, i.e. a
correctly rounded output. No kernel that sums in another order than the
oracle can promise that: when x lies closer to a rounding boundary than the
kernel's own f32 error, either neighbour is an honest result. So the one
allowance is that narrow band: got may be the correct rounding of any x'
within REL_F32 = 2^-10 of x (relative), and the error is measured from the
nearest such value:
    err = max(0, RN(x - d) - got, got - RN(x + d)),  d = REL_F32 * |x|.
An output one bf16 step off RN(x) therefore passes only when x is within d
of the boundary between the two steps. 2^-10 is twice the unit roundoff of
the f16 weights the kernels multiply values by (2^-11); the tests print how
many outputs use the band and the raw distance to x.
"""
import numpy as np

import oracle_lib as O

MAX_ABS = 2e-2
MEAN_ABS = 1e-3
REL_F32 = 2.0 ** -10


def rn_bf16(x):
    """Values rounded to bf16 (round to nearest even), returned as f64."""
    return O.bf16_to_f32(O.bf16_from_f32(np.asarray(x, np.float32))).astype(np.float64)


def bf16_errors(got_bf16, want):
    """(err as above, |got - RN(x)|, raw |got - x|), f64 arrays of the
    output's shape."""
    got = O.bf16_to_f32(got_bf16).astype(np.float64)
    assert np.all(np.isfinite(got)), "non-finite output"
    x = np.asarray(want, np.float64)
    d = REL_F32 * np.abs(x)
    lo, hi = rn_bf16(x - d), rn_bf16(x + d)
    err = np.maximum(np.maximum(lo - got, got - hi), 0.0)
    return err, np.abs(got - rn_bf16(x)), np.abs(got - x)


def check_bf16(got_bf16, want, tag, scale=None, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    """Asserts the bar. scale: divide the errors by it first (outputs whose
    values are far outside N(0,1) are held to the bar relative to their
    magnitude). Returns (err, raw)."""
    err, strict, raw = bf16_errors(got_bf16, want)
    if scale is not None:
        err, strict, raw = err / scale, strict / scale, raw / scale
    off = int(np.count_nonzero(strict))
    band = int(np.count_nonzero((strict > max_abs) & (err <= max_abs)))
    print(f"[{tag}] bf16 err max={err.max():.3e} mean={err.mean():.3e}; |got-RN(x)| "
          f"max={strict.max():.3e} (off RN(x): {off} of {err.size}, passing by the f32 band: "
          f"{band}); raw max={raw.max():.3e} mean={raw.mean():.3e}", flush=True)
    assert err.max() <= max_abs and err.mean() <= mean_abs, tag
    return err, raw
