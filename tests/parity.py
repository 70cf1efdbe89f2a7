"""Parity bars shared by the GPU tests (imported by the test modules; no tests here).

The north-star bar: fp16 output vs the FP32 oracle, max-abs-error <= 2e-3 and mean-abs-error
<= 2e-4. `assert_parity_f16_out` applies it to the error left after the fp16 output's own final
rounding (half an fp16 spacing at |ref|): outputs above magnitude 2 (a residual stream of N(0,1)
values, or a peaked softmax returning single value rows) round by 9.8e-4 ([2, 4)) or 1.95e-3
([4, 8)) however exact the computation before that rounding, while below |o| = 1 the allowance is
at most 2.4e-4. Where |ref| < 4 the output rounding is at most 9.8e-4, so the plain bar (raw
max-abs <= max_abs) is asserted there as well: only outputs of magnitude 4 and above use the
beyond-rounding form alone.
"""
import numpy as np

import oracle

MAX_ABS = 2e-3
MEAN_ABS = 2e-4
# below this output magnitude the raw max-abs bar holds as well
PLAIN_BAR_BELOW = 4.0


def assert_parity(got, ref, max_abs=MAX_ABS, mean_abs=MEAN_ABS, label=""):
    mx, mean, _ = oracle.error_stats(got, ref)
    print(f"{label}: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert np.isfinite(got).all(), label
    assert mx <= max_abs, (label, mx)
    assert mean <= mean_abs, (label, mean)


def half_ulp_f16(x):
    """Half the fp16 spacing at |x| (the rounding error of a correctly rounded fp16 output)."""
    a = np.maximum(np.abs(np.asarray(x, np.float64)), 2.0 ** -14)
    return np.ldexp(1.0, np.floor(np.log2(a)).astype(np.int64) - 11)


def assert_parity_f16_out(got, ref, max_abs=MAX_ABS, mean_abs=MEAN_ABS, label=""):
    """The parity bar on the error beyond the fp16 output's own final rounding."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    excess = (err - half_ulp_f16(ref)).max() if err.size else 0.0
    mean = err.mean() if err.size else 0.0
    print(f"{label}: max_abs={err.max() if err.size else 0:.3e} beyond output rounding={excess:.3e} "
          f"mean_abs={mean:.3e} max|ref|={np.abs(ref).max() if ref.size else 0:.2f}", flush=True)
    assert np.isfinite(got).all(), label
    assert excess <= max_abs, (label, excess)
    small = np.abs(ref) < PLAIN_BAR_BELOW
    raw_small = err[small].max() if small.any() else 0.0
    assert raw_small <= max_abs, (label, "raw error where |ref| < 4", raw_small)
    assert mean <= mean_abs, (label, mean)
