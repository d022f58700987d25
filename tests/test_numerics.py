"""Error bound of the branch-free rho^8 that the bf16/fp16 MFMA kernels use when the host
accepts it (fast_rho_ok in afa_capi.hip): rho = fma(t, rsqrt(t), s), t = fma(s, s, 1), then
three squarings, all in float32, with the hardware rsqrt allowed one ulp of error.  CPU only:
the float32 steps are emulated in numpy (fma as one rounding of the exact float64 result)."""
import numpy as np

from oracle import afa_oracle as O


def _fast_rho8_f32(s, rsq_ulps):
    s64 = s.astype(np.float64)
    t = (s64 * s64 + 1.0).astype(np.float32)
    r = (1.0 / np.sqrt(t.astype(np.float64))).astype(np.float32)
    r = (r.view(np.int32) + rsq_ulps).view(np.float32)
    rho = (t.astype(np.float64) * r.astype(np.float64) + s64).astype(np.float32)
    p2 = rho * rho
    p4 = p2 * p2
    return (p4 * p4).astype(np.float64)


def test_fast_rho8_bound_for_negative_scores():
    rng = np.random.default_rng(0)
    s = np.concatenate([-np.logspace(-4, 4, 400_000), -rng.uniform(0, 8, 400_000)]).astype(np.float32)
    exact = O.rho8(s.astype(np.float64))
    for ulps in (-1, 0, 1):
        err = np.abs(_fast_rho8_f32(s, ulps) - exact)
        assert np.all(err <= 32 * 2.0 ** -24 * exact + 1e-8)


def test_fast_rho8_positive_scores_are_relative():
    s = np.logspace(-4, 4, 200_000).astype(np.float32)
    exact = O.rho8(s.astype(np.float64))
    for ulps in (-1, 0, 1):
        rel = np.abs(_fast_rho8_f32(s, ulps) - exact) / exact
        assert rel.max() < 32 * 2.0 ** -24
