"""The rans_ilv GPU encoder replaces x / f by a float estimate
(float32(x) * float32(1 / f), truncated) and one correction step; that is
exact only if the estimate is within one of floor(x / f).  The encoder
calls it with x < f * 2^21 (after renormalisation) and 1 <= f <= 2048.
This checks the bound with IEEE float32 arithmetic (round to nearest, as
the device's v_cvt_f32_u32 / v_mul_f32; truncation as v_cvt_u32_f32) for
every f, on random x and on x at and around multiples of f."""
import numpy as np


def test_quotient_estimate_within_one():
    rng = np.random.default_rng(1)
    for f in range(1, 2049):
        hi = f << 21
        k = rng.integers(0, 1 << 21, 600, dtype=np.uint64)
        x = np.concatenate([rng.integers(0, hi, 1500, dtype=np.uint64), k * f, k * f + f - 1, k * f + 1,
                            np.array([hi - 1, hi - f, 0, 1, 65535], np.uint64)])
        x = x[x < hi]
        rf = np.float32(1.0) / np.float32(f)
        est = (x.astype(np.float32) * rf).astype(np.float64)
        q_est = np.trunc(np.maximum(est, 0)).astype(np.int64)
        assert np.abs(q_est - (x // f).astype(np.int64)).max() <= 1, f
