"""Pins the float64 OACE oracle (oracle/oace_oracle.py) with checks that do not retype its
formulas: the reference's own parity relations (fused forward = loss of the materialised
logits, the cached radial reduction = its full-vocabulary definition, chunk invariance), an
independent power-form score, a closed form, and finite differences.  Reference tests:
tests/test_pallas_oace.py:62-182."""
import math
import os

import numpy as np
import pytest

from oracle import afa_oracle as AO
from oracle import oace_oracle as O


def _case(N, d, V, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    h = rng.standard_normal((N, d)) * scale
    w = rng.standard_normal((d, V)) * scale
    t = rng.integers(0, V, size=N)
    return h, w, t


def test_octic_parts_identities():
    x = np.linspace(-40.0, 40.0, 801)
    k8, rho7, rho, r = O.octic_parts(x)
    np.testing.assert_allclose(rho * O.octic_parts(-x)[2], 1.0, rtol=1e-14)
    np.testing.assert_allclose(k8, AO.rho8(x), rtol=1e-13)
    np.testing.assert_allclose(rho7 * rho, k8, rtol=1e-14)
    np.testing.assert_allclose(r, 1.0 / np.sqrt(1.0 + x * x), rtol=1e-15)
    # rho(2)^8 = 51841 + 23184 sqrt(5) (reference tests/test_attention.py:34)
    assert abs(O.octic_parts(2.0)[0] - (51841.0 + 23184.0 * math.sqrt(5.0))) <= 1e-9 * 103682.0


@pytest.mark.parametrize("N,d,V,chunk", [(16, 32, 256, 64), (10, 20, 203, 64), (6, 12, 67, 19)])
def test_fused_forward_equals_loss_of_materialised_logits(N, d, V, chunk):
    """The reference's forward parity test (test_pallas_oace.py:62-80, rel <= 1e-6): the chunked
    Gram-based forward against fused_oace_softmax_loss on h @ w."""
    h, w, t = _case(N, d, V, seed=N + V)
    fused, rows = O.fused_linear_oace_forward(h, w, t, chunk_size=chunk)
    ref, cache = O.oace_softmax_loss(h @ w, t)
    assert abs(fused - ref) <= 1e-12 * abs(ref)
    np.testing.assert_allclose(rows["tau"], cache["tau"], rtol=1e-12)
    np.testing.assert_allclose(rows["loss"], cache["loss"], rtol=1e-11)


def test_forward_equals_power_form_score():
    """loss.py's score with p^(-1/8) and p^(7/8) by numpy powers, applied to the A-Softmax
    probabilities, equals the rho-factorised loss (model.py:193-207)."""
    h, w, t = _case(12, 24, 150, seed=3)
    fused, rows = O.fused_linear_oace_forward(h, w, t, chunk_size=40)
    _, cache = O.oace_softmax_loss(h @ w, t)
    score = O.oace_score(cache["p"], t)
    np.testing.assert_allclose(rows["loss"][:, 0], score, rtol=1e-11)
    assert abs(fused - score.mean()) <= 1e-11 * abs(fused)


@pytest.mark.parametrize("V", [1, 7, 50257])
def test_uniform_closed_form(V):
    """h = 0: every logit is 0, rho = 1, p = 1/V, loss = gamma * 64/7 * (V^(1/8) - 1)."""
    d, N = 8, 3
    h = np.zeros((N, d))
    w = np.random.default_rng(V).standard_normal((d, V))
    t = np.arange(N) % V
    fused, rows = O.fused_linear_oace_forward(h, w, t, gamma=1.5, chunk_size=4096)
    assert abs(fused - O.uniform_loss(V, gamma=1.5)) <= 1e-12 * max(1.0, O.uniform_loss(V, 1.5))
    np.testing.assert_allclose(rows["tau"], 1.0 / math.sqrt(100.0), rtol=1e-15)


def test_loss_is_minimised_by_the_target():
    """Proper score: with a dominant target logit the loss is small and positive; moving the
    target to the least likely class increases it."""
    V = 64
    z = np.zeros((1, V))
    z[0, 5] = 60.0
    good, _ = O.oace_softmax_loss(z, np.array([5]))
    bad, _ = O.oace_softmax_loss(z, np.array([6]))
    assert 0.0 < good < bad


def test_chunk_size_invariance():
    """test_pallas_oace.py:159-172: different chunkings agree to 1e-12."""
    h, w, t = _case(8, 16, 256, seed=403)
    ls = [O.fused_linear_oace_forward(h, w, t, chunk_size=c)[0] for c in (32, 64, 128, 1000)]
    for x in ls[1:]:
        assert abs(x - ls[0]) <= 1e-12 * abs(ls[0])


def test_gram_moment_equals_direct_sum():
    h, w, t = _case(5, 9, 31, seed=11)
    _, rows = O.fused_linear_oace_forward(h, w, t)
    z = h @ w
    np.testing.assert_allclose(rows["tau"][:, 0], 1.0 / np.sqrt((z * z).mean(-1) + 100.0), rtol=1e-13)


def test_radial_matches_full_vocabulary_definition():
    """test_pallas_oace.py:116-156: the radial scalar from three forward reductions equals
    mean(r * bracket * n) over the whole vocabulary."""
    h, w, t = _case(6, 12, 67, seed=405)
    _, rows = O.fused_linear_oace_forward(h, w, t, chunk_size=19)
    _, cache = O.oace_softmax_loss(h @ w, t)
    onehot = np.zeros_like(cache["n"])
    onehot[np.arange(6), t] = 1.0
    bracket = cache["p78"] - onehot * cache["p_c_inv8"] - cache["p"] * (cache["sum_p78"] - cache["p_c_inv8"])
    expected = np.mean(cache["r"] * bracket * cache["n"], axis=-1, keepdims=True)
    np.testing.assert_allclose(rows["radial"], expected, rtol=2e-13, atol=2e-13)


def _fd(f, x, i, step):
    xp = x.copy()
    xm = x.copy()
    xp[i] += step
    xm[i] -= step
    return (f(xp) - f(xm)) / (2 * step)


def test_fused_backward_matches_finite_differences():
    """dh and dW of the streamed backward against central differences of the forward."""
    h, w, t = _case(4, 6, 23, seed=402, scale=0.7)
    g = 1.3
    loss, rows = O.fused_linear_oace_forward(h, w, t, chunk_size=7)
    dh, dw = O.fused_linear_oace_backward(h, w, t, rows, g=g, chunk_size=5)
    fh = lambda x: g * O.fused_linear_oace_forward(x, w, t, chunk_size=7)[0]
    fw = lambda x: g * O.fused_linear_oace_forward(h, x, t, chunk_size=7)[0]
    for i in [(0, 0), (1, 3), (3, 5), (2, 2)]:
        assert abs(dh[i] - _fd(fh, h, i, 1e-5)) <= 1e-7 * max(1.0, np.abs(dh).max())
    for i in [(0, 0), (2, 7), (5, 22), (4, 11)]:
        assert abs(dw[i] - _fd(fw, w, i, 1e-5)) <= 1e-7 * max(1.0, np.abs(dw).max())


def test_softmax_loss_vjp_matches_finite_differences():
    rng = np.random.default_rng(7)
    z = rng.standard_normal((3, 17)) * 20.0
    t = np.array([4, 0, 16])
    _, cache = O.oace_softmax_loss(z, t)
    dz = O.oace_softmax_loss_vjp(cache, 0.8)
    f = lambda x: 0.8 * O.oace_softmax_loss(x, t)[0]
    for i in [(0, 4), (0, 5), (1, 0), (2, 16), (2, 3)]:
        assert abs(dz[i] - _fd(f, z, i, 1e-5)) <= 1e-8 * max(1.0, np.abs(dz).max())


def test_planted_sign_error_fails_the_radial_check():
    """A dropped sign in the radial expansion is caught by the full-vocabulary definition."""
    h, w, t = _case(6, 12, 67, seed=405)
    _, rows = O.fused_linear_oace_forward(h, w, t)
    _, cache = O.oace_softmax_loss(h @ w, t)
    onehot = np.zeros_like(cache["n"])
    onehot[np.arange(6), t] = 1.0
    bracket = cache["p78"] + onehot * cache["p_c_inv8"] - cache["p"] * (cache["sum_p78"] - cache["p_c_inv8"])
    wrong = np.mean(cache["r"] * bracket * cache["n"], axis=-1, keepdims=True)
    assert np.abs(wrong - rows["radial"]).max() > 1e-6


# ---------------------------------------------------------------- 40-digit golden fixtures
GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "oace_golden.npz"))


@pytest.mark.parametrize("name", ["lin_small", "lin_d32"])
def test_linear_oracle_matches_golden(name):
    """The rho-factorised oracle against the power-form score evaluated at 40 digits, and its
    analytical backward against mpmath numerical differentiation."""
    h, w, t = GOLD[f"{name}_h"], GOLD[f"{name}_w"], GOLD[f"{name}_t"]
    eps, gamma = GOLD[f"{name}_cfg"]
    loss, rows = O.fused_linear_oace_forward(h, w, t, eps_vocab=eps, gamma=gamma, chunk_size=3)
    assert abs(loss - float(GOLD[f"{name}_loss"])) <= 1e-13 * abs(float(GOLD[f"{name}_loss"]))
    np.testing.assert_allclose(rows["loss"][:, 0], GOLD[f"{name}_row_loss"], rtol=1e-12)
    np.testing.assert_allclose(rows["tau"][:, 0], GOLD[f"{name}_tau"], rtol=1e-14)
    dh, dw = O.fused_linear_oace_backward(h, w, t, rows, g=1.0, gamma=gamma, chunk_size=2)
    for got, ref in ((dh, GOLD[f"{name}_dh"]), (dw, GOLD[f"{name}_dw"])):
        assert np.abs(got - ref).max() <= 1e-10 * np.abs(ref).max()


def test_softmax_oracle_matches_golden():
    z, t = GOLD["sm_z"], GOLD["sm_t"]
    eps, gamma = GOLD["sm_cfg"]
    loss, cache = O.oace_softmax_loss(z, t, eps=eps, gamma=gamma)
    assert abs(loss - float(GOLD["sm_loss"])) <= 1e-13 * abs(float(GOLD["sm_loss"]))
    dz = O.oace_softmax_loss_vjp(cache, 1.0, gamma=gamma)
    assert np.abs(dz - GOLD["sm_dz"]).max() <= 1e-10 * np.abs(GOLD["sm_dz"]).max()
