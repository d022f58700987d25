"""Error bound of the branch-free rho^8 that the bf16/fp16 MFMA kernels use on waves whose scores
are all provably within |s| <= 32 (the fast-rho guard: Cauchy-Schwarz with per-block row norms,
fast_rho_safe in csrc/afa_common.h): rho = fma(t, rsqrt(t), s), t = fma(s, s, 1), then three
squarings, all in float32, with the hardware rsqrt allowed one ulp of error.  CPU only: the
float32 steps are emulated in numpy (fma as one rounding of the exact float64 result).

For s < 0 the sum cancels: t r carries a relative error eta <= 2^-25 + 1.5 * 2^-23 (the rounding
of t, halved by the square root, plus the rounding of rsqrt and its one ulp), an absolute error
|s| eta against rho(s) ~ 1/(2|s|), so rho^8 is off by about 16 s^2 eta relative, 3.4e-3 at
|s| = 32.  Outside the
guard's range that grows without bound (the reason for the guard): at |s| = 1e6 the result is
garbage of order (|s| eta)^8."""
import numpy as np

from oracle import afa_oracle as O

ETA = 2.0 ** -25 + 1.5 * 2.0 ** -23


def _fast_rho8_f32(s, rsq_ulps):
    s64 = s.astype(np.float64)
    t = (s64 * s64 + 1.0).astype(np.float32)
    r = (1.0 / np.sqrt(t.astype(np.float64))).astype(np.float32)
    r = (r.view(np.int32) + rsq_ulps).view(np.float32)
    rho = (t.astype(np.float64) * r.astype(np.float64) + s64).astype(np.float32)
    p2 = rho * rho
    p4 = p2 * p2
    return (p4 * p4).astype(np.float64)


def test_fast_rho8_relative_bound_inside_the_guard():
    """Per weight, |fast - exact| <= (16 s^2 eta + 32 * 2^-24) exact for s in [-32, 0]; the
    kernels' per-row error on rows whose scores all lie in [-32, -30] is at most 3.4e-3."""
    rng = np.random.default_rng(0)
    s = np.concatenate([-np.logspace(-4, np.log10(32.0), 400_000), -rng.uniform(0, 32, 400_000)]).astype(np.float32)
    exact = O.rho8(s.astype(np.float64))
    bound = (16 * s.astype(np.float64) ** 2 * ETA + 32 * 2.0 ** -24) * exact
    worst = 0.0
    for ulps in (-1, 0, 1):
        err = np.abs(_fast_rho8_f32(s, ulps) - exact)
        assert np.all(err <= bound)
        worst = max(worst, float((err / exact)[np.abs(s) >= 30].max()))
    assert worst <= 3.4e-3


def test_fast_rho8_positive_scores_are_relative():
    s = np.logspace(-4, 4, 200_000).astype(np.float32)
    exact = O.rho8(s.astype(np.float64))
    for ulps in (-1, 0, 1):
        rel = np.abs(_fast_rho8_f32(s, ulps) - exact) / exact
        assert rel.max() < 32 * 2.0 ** -24


def test_fast_rho8_fails_far_outside_the_guard():
    """Why the guard exists: at s = -1e6 and -1e7 the branch-free form returns weights many
    orders of magnitude above the true ~1e-51 and ~1e-59 (the advisor's 4.4e-8 and 0.31)."""
    s = np.array([-1e6, -1e7], dtype=np.float32)
    exact = O.rho8(s.astype(np.float64))
    fast = _fast_rho8_f32(s, 1)
    assert np.all(exact < 1e-50)
    assert fast[0] > 1e-9 and fast[1] > 1e-2


def test_fast_rho8_is_off_by_factors_near_minus_1500():
    """The premise of the GPU tests whose rows score near -1500: there |s| eta ~ rho(s), so most
    branch-free weights are off by more than 50% (for every rsqrt rounding), some by factors of
    100 or more, and a per-row check at 1e-2 or 3e-2 fails if the guard let that form run."""
    s = -np.linspace(1000.0, 2000.0, 20001).astype(np.float32)
    exact = O.rho8(s.astype(np.float64))
    for ulps in (-1, 0, 1):
        ratio = _fast_rho8_f32(s, ulps) / exact
        assert np.mean(np.abs(ratio - 1.0) > 0.5) > 0.5
    assert (_fast_rho8_f32(s, 1) / exact).max() > 100.0
