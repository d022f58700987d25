"""The row-restricted float64 restatements used by the full-length GPU checks
(tests/helpers.py: afa_rows_forward64, afa_rows_backward64) equal the oracle's whole-matrix
forward and backward (oracle/afa_oracle.py, pinned by the golden fixtures and by finite
differences) on the rows they compute; a planted mistake (the strict causal mask) is rejected."""
import numpy as np

from oracle import afa_oracle as O
from tests.helpers import afa_rows_backward64, afa_rows_forward64


def _inputs(L=96, D=64, seed=0):
    rng = np.random.default_rng(seed)
    return [rng.standard_normal((L, D)) for _ in range(4)]


def test_rows_forward_matches_oracle():
    q, k, v, _ = _inputs()
    out, den = O.afa_forward(q, k, v, 0.5, True, return_denominator=True)
    rows = [0, 1, 31, 32, 63, 95]
    o_r, d_r = afa_rows_forward64(q, k, v, rows)
    assert np.abs(o_r - out[rows]).max() <= 1e-12 * np.abs(out).max()
    assert np.abs(d_r - den[rows, 0]).max() <= 1e-12 * den.max()


def test_rows_backward_matches_oracle():
    q, k, v, g = _inputs(seed=1)
    out, den = O.afa_forward(q, k, v, 0.5, True, return_denominator=True)
    dq, dk, dv = O.afa_backward(q, k, v, g, 0.5, True)
    qrows, krows = [0, 5, 47, 95], [0, 1, 50, 95]
    rq, rk, rv = afa_rows_backward64(q, k, v, g, out, den[:, 0], qrows, krows)
    for got, ref in ((rq, dq[qrows]), (rk, dk[krows]), (rv, dv[krows])):
        assert np.abs(got - ref).max() <= 1e-11 * np.abs(ref).max()


def test_rows_backward_rejects_strict_mask():
    """A dk row summed over queries i > j only (the diagonal dropped) differs from the oracle."""
    q, k, v, g = _inputs(seed=2)
    out, den = O.afa_forward(q, k, v, 0.5, True, return_denominator=True)
    _, dk, _ = O.afa_backward(q, k, v, g, 0.5, True)
    j, scale = 40, 1.0 / 8.0
    s = (q[j + 1:] @ k[j]) * scale
    E = np.sum(g * out, axis=-1)
    w = O.rho8(s) / den[j + 1:, 0]
    wrong = (8.0 * scale * w / np.sqrt(1 + s * s) * (g[j + 1:] @ v[j] - E[j + 1:])) @ q[j + 1:]
    assert np.abs(wrong - dk[j]).max() > 1e-6 * np.abs(dk[j]).max()
