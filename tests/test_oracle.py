"""Pinning of the CPU oracle (oracle/afa_oracle.py in float64, oracle/afa_contract.c under the
reference's fp32-accumulation contract).  CPU only.

The oracle is checked against the 40-digit mpmath fixtures in tests/golden/, the known answers
of the reference's own tests (tests/test_attention.py:28-63, tests/test_pallas_afa.py:90-224,
tests/test_ago.py:62-94 in the reference), finite differences, and invariants that a dropped
term, a wrong sign or index or a transposed operand would break.
"""
import math
import os

import numpy as np
import pytest

from oracle import afa_oracle as O
from oracle import contract as C
from tests.helpers import normwise

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "afa_golden.npz")
FWD_CASES = ["fwd_plain", "fwd_causal_valid", "fwd_nosink_causal", "fwd_tail", "fwd_rotary",
             "fwd_d64_rotary", "fwd_d128"]


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _case(gold, name):
    sink, causal, valid = gold[f"{name}_cfg"]
    rot = (gold[f"{name}_cos"], gold[f"{name}_sin"]) if f"{name}_cos" in gold else None
    return (gold[f"{name}_q"], gold[f"{name}_k"], gold[f"{name}_v"], float(sink), bool(causal),
            None if valid < 0 else int(valid), rot)


# ----------------------------------------------------------------------------- rho^8
def test_rho8_known_answer():
    # rho(2)^8 = (2 + sqrt 5)^8 = 51841 + 23184 sqrt 5 (reference tests/test_attention.py:34)
    assert O.rho8(np.array([2.0]))[0] == pytest.approx(51841 + 23184 * math.sqrt(5), rel=2e-15)
    # rho(3)^8 / rho(-3)^8 contrast, and rho(0) = 1
    r = O.rho8(np.array([3.0, -3.0, 0.0]))
    assert r[0] / r[1] > 1e5 and r[2] == 1.0


def test_rho_reciprocal_identity():
    x = np.concatenate([np.linspace(-50, 50, 2001), [1e-300, 1e3, 1e8, 1e15]])
    np.testing.assert_allclose(O.rho(x) * O.rho(-x), 1.0, rtol=4e-16 * 4, atol=0)


def test_rho8_matches_mpmath(gold):
    np.testing.assert_allclose(O.rho8(gold["rho8_x"]), gold["rho8_y"], rtol=2e-15, atol=0)


def test_rho8_negative_tail_positive_and_accurate():
    s = np.array([-1e2, -1e3, -1e4])
    w = O.rho8(s)
    assert np.all(w > 0)
    # rho(-x) = 1/rho(x), and rho(x) = x + sqrt(1+x^2) has no cancellation for x > 0
    np.testing.assert_allclose(w, 1.0 / (-s + np.sqrt(1.0 + s * s)) ** 8, rtol=1e-14)


def test_rho8_derivative_by_finite_differences():
    x = np.linspace(-4, 4, 33)
    h = 1e-6
    fd = (O.rho8(x + h) - O.rho8(x - h)) / (2 * h)
    np.testing.assert_allclose(O.rho8_derivative(x), fd, rtol=1e-7, atol=1e-9)


# ----------------------------------------------------------------------------- AFA forward
@pytest.mark.parametrize("name", FWD_CASES)
def test_afa_forward_matches_mpmath(gold, name):
    q, k, v, sink, causal, valid, rot = _case(gold, name)
    out, den = O.afa_forward(q, k, v, sink, causal, valid, rot, return_denominator=True)
    assert normwise(out, gold[f"{name}_out"]) < 1e-13
    np.testing.assert_allclose(den, gold[f"{name}_den"], rtol=1e-13)


def test_golden_fixtures_reject_planted_mistakes(gold):
    """Plausible oracle mistakes (dropped sink, transposed scores, rho^4, unscaled scores,
    off-by-one causal mask, q/k rotated in the opposite sense) all miss the fixtures."""
    q, k, v, sink, causal, valid, _ = _case(gold, "fwd_causal_valid")
    ref = gold["fwd_causal_valid_out"]
    L, D = q.shape[-2:]
    s = np.einsum("...id,...jd->...ij", q, k) / math.sqrt(D)

    def finish(w, sk=sink):
        return np.einsum("...ij,...jd->...id", w, v) / (w.sum(-1, keepdims=True) + sk)

    keep = np.tril(np.ones((L, L), bool))
    keep[:, valid:] = False
    mistakes = {
        "dropped sink": finish(np.where(keep, O.rho8(s), 0), 0.0),
        "transposed scores": finish(np.where(keep, O.rho8(np.swapaxes(s, -1, -2)), 0)),
        "rho^4": finish(np.where(keep, O.rho(s) ** 4, 0)),
        "no 1/sqrt(D)": finish(np.where(keep, O.rho8(s * math.sqrt(D)), 0)),
        "strict causal": finish(np.where(np.tril(keep, -1), O.rho8(s), 0)),
    }
    for what, bad in mistakes.items():
        assert normwise(bad, ref) > 1e-3, what
    qr, kr, vr, sk, cs, vl, (c, sn) = _case(gold, "fwd_rotary")
    bad = O.afa_forward(qr, kr, vr, sk, cs, vl, (c, -sn))
    assert normwise(bad, gold["fwd_rotary_out"]) > 1e-3


def test_afa_single_key_closed_form():
    rng = np.random.default_rng(3)
    q, k, v = rng.standard_normal((3, 1, 1, 1, 5))
    out, den = O.afa_forward(q, k, v, 0.75, return_denominator=True)
    w = O.rho8(np.array([(q * k).sum() / math.sqrt(5)]))[0]
    np.testing.assert_allclose(out[0, 0, 0], w * v[0, 0, 0] / (w + 0.75), rtol=1e-14)
    np.testing.assert_allclose(den[0, 0, 0, 0], w + 0.75, rtol=1e-14)


def test_causal_prefix_invariance_is_exact():
    rng = np.random.default_rng(4)
    q, k, v = rng.standard_normal((3, 1, 2, 40, 8))
    base = O.afa_forward(q, k, v, causal=True)
    k2, v2 = k.copy(), v.copy()
    k2[..., 25:, :] = rng.standard_normal(k2[..., 25:, :].shape) * 10
    v2[..., 25:, :] = -7.0
    pert = O.afa_forward(q, k2, v2, causal=True)
    assert np.array_equal(base[..., :25, :], pert[..., :25, :])
    assert not np.array_equal(base[..., 25:, :], pert[..., 25:, :])


def test_ring_split_additivity():
    """Partial numerators/denominators over P key shards add up to the full result
    (src/kernels/pallas_afa.py:618-662; the ring exchange is purely additive)."""
    rng = np.random.default_rng(5)
    q, k, v = rng.standard_normal((3, 2, 3, 32, 8)) * 0.7
    sink = 0.5
    full = O.afa_forward(q, k, v, sink)
    num = np.zeros_like(full)
    den = np.zeros(full.shape[:-1] + (1,))
    for p in range(4):
        ks, vs = k[..., 8 * p:8 * p + 8, :], v[..., 8 * p:8 * p + 8, :]
        o_p, d_p = O.afa_forward(q, ks, vs, 0.0, return_denominator=True)
        num += o_p * d_p
        den += d_p
    assert normwise(num / (den + sink), full) < 1e-14


@pytest.mark.parametrize("causal", [False, True])
def test_ring_oracle_equals_full_attention(causal):
    """The ring of src/kernels/pallas_afa.py:618-662 re-associates the sums of the full forward:
    for every shard count it gives the same output (a causal mask on shard-local indices, or a
    wrong shard offset, would not)."""
    rng = np.random.default_rng(15)
    q, k, v = rng.standard_normal((3, 2, 2, 32, 8)) * 0.6
    full = O.afa_forward(q, k, v, 0.5, causal=causal)
    for n in (1, 2, 4, 8):
        assert normwise(O.ring_afa(q, k, v, 0.5, causal, n), full) < 1e-13, n


def test_value_linearity_and_key_permutation():
    rng = np.random.default_rng(6)
    q, k, v, v2 = rng.standard_normal((4, 1, 2, 24, 8))
    a = O.afa_forward(q, k, 2.0 * v - 3.0 * v2)
    b = 2.0 * O.afa_forward(q, k, v) - 3.0 * O.afa_forward(q, k, v2)
    assert normwise(a, b) < 1e-13
    perm = rng.permutation(24)
    c = O.afa_forward(q, k[..., perm, :], v[..., perm, :])
    assert normwise(c, O.afa_forward(q, k, v)) < 1e-13


def test_valid_len_equals_truncated_keys():
    rng = np.random.default_rng(7)
    q, k, v = rng.standard_normal((3, 1, 1, 20, 8))
    a = O.afa_forward(q, k, v, valid_len=13)
    b = O.afa_forward(q, k[..., :13, :], v[..., :13, :])
    assert normwise(a, b) < 1e-15


# ----------------------------------------------------------------------------- AFA backward
def test_afa_backward_matches_mpmath(gold):
    q, k, v, g = gold["bwd_q"], gold["bwd_k"], gold["bwd_v"], gold["bwd_g"]
    sink, causal, _ = gold["bwd_cfg"]
    dq, dk, dv = O.afa_backward(q, k, v, g, float(sink), bool(causal))
    for got, key in ((dq, "bwd_dq"), (dk, "bwd_dk"), (dv, "bwd_dv")):
        assert normwise(got, gold[key]) < 1e-12, key


@pytest.mark.parametrize("causal,valid", [(False, None), (True, None), (True, 9)])
def test_afa_backward_finite_differences(causal, valid):
    rng = np.random.default_rng(8)
    q, k, v, g = rng.standard_normal((4, 1, 2, 12, 4)) * 0.8
    grads = O.afa_backward(q, k, v, g, 0.5, causal, valid)
    h = 1e-6
    for which, grad in enumerate(grads):
        fd = np.zeros_like(grad)
        args = [q, k, v]
        it = np.nditer(args[which], flags=["multi_index"])
        for _ in it:
            idx = it.multi_index
            plus = [a.copy() for a in args]
            minus = [a.copy() for a in args]
            plus[which][idx] += h
            minus[which][idx] -= h
            fp = (O.afa_forward(*plus, 0.5, causal, valid) * g).sum()
            fm = (O.afa_forward(*minus, 0.5, causal, valid) * g).sum()
            fd[idx] = (fp - fm) / (2 * h)
        assert normwise(grad, fd) < 1e-7


# ----------------------------------------------------------------------------- A-Softmax
@pytest.mark.parametrize("n", [1, 3, 7, 64])
def test_asoftmax_matches_mpmath(gold, n):
    sink, eps = gold[f"asm_{n}_cfg"]
    y = O.asoftmax(gold[f"asm_{n}_x"], float(sink), float(eps))
    np.testing.assert_allclose(y, gold[f"asm_{n}_y"], rtol=1e-13, atol=1e-300)


def test_asoftmax_jacobian_at_zero():
    # d p / d z at z = 0 with sink 0 is [[2,-2],[-2,2]]; through AVN at x = 0 it is that / sqrt(eps)
    # (reference tests/test_attention.py:37-53)
    eps = 1e-5
    x = np.zeros(2)
    J = np.stack([O.asoftmax_vjp(x, np.eye(2)[i], 0.0, eps) for i in range(2)])
    np.testing.assert_allclose(J * math.sqrt(eps), [[2, -2], [-2, 2]], rtol=1e-12)


@pytest.mark.parametrize("n", [1, 64, 4096])
def test_asoftmax_simplex_extremes(n):
    rng = np.random.default_rng(n)
    x = rng.choice([-1e15, 1e15], size=(3, n))
    for sink in (0.0, 0.5, 1.0):
        p = O.asoftmax(x, sink)
        assert np.all(np.isfinite(p)) and np.all(p >= 0)
        assert np.all(p.sum(-1) <= 1 + 1e-12)
        if sink == 0.0:
            np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-12)


def test_asoftmax_vjp_by_finite_differences():
    rng = np.random.default_rng(9)
    x, g = rng.standard_normal((2, 3, 10)) * 1.5
    got = O.asoftmax_vjp(x, g, 0.5, 1e-5)
    h = 1e-6
    fd = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        fd[idx] = ((O.asoftmax(xp, 0.5) - O.asoftmax(xm, 0.5)) * g).sum() / (2 * h)
    assert normwise(got, fd) < 1e-7


# ----------------------------------------------------------------------------- Cayley rotary
@pytest.mark.parametrize("name", ["cayley_default", "cayley_c3"])
def test_cayley_tables_match_closed_form(gold, name):
    cos, sin = gold[f"{name}_cos"], gold[f"{name}_sin"]
    c, s = O.cayley_tables(2 * cos.shape[1], cos.shape[0], freqs=gold[f"{name}_freqs"])
    np.testing.assert_allclose(c, cos, rtol=0, atol=1e-13)
    np.testing.assert_allclose(s, sin, rtol=0, atol=1e-13)


def test_cayley_default_frequencies(gold):
    np.testing.assert_allclose(O.default_freqs(8), gold["cayley_default_freqs"], rtol=1e-15)


def test_cayley_det_orthogonality_norm_and_shift():
    """det R = c^2 + s^2 = 1, R^T R = I, norm conservation to L = 8192, and shift
    equivariance <R_m q, R_n k> = <q, R_(n-m) k> (reference tests/test_ago.py:62-94)."""
    D, L = 64, 8192
    c, s = O.cayley_tables(D, L, freqs=10000.0 ** (-2.0 * np.arange(D // 2) / D))
    np.testing.assert_allclose(c * c + s * s, 1.0, atol=1e-15)
    rng = np.random.default_rng(10)
    x = rng.standard_normal((1, L, D))
    xr = O.rotate_pairs(x, c, s)
    np.testing.assert_allclose(np.linalg.norm(xr, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-12)
    q, k = rng.standard_normal((2, D))
    for m, n in ((0, 5), (100, 105), (4000, 4005), (3, 4095)):
        qm = O.rotate_pairs(np.broadcast_to(q, (L, D)), c, s)[m]
        kn = O.rotate_pairs(np.broadcast_to(k, (L, D)), c, s)[n]
        k0 = O.rotate_pairs(np.broadcast_to(k, (L, D)), c, s)[n - m]
        assert abs(qm @ kn - q @ k0) < 1e-6


def test_rotation_pair_layout():
    # (x0, x1) -> (c x0 - s x1, s x0 + c x1) on consecutive (even, odd) features
    x = np.array([[[1.0, 2.0, 3.0, 4.0]]])
    c, s = np.array([[0.6, 0.0]]), np.array([[0.8, 1.0]])
    np.testing.assert_allclose(O.rotate_pairs(x, c, s), [[[0.6 - 1.6, 0.8 + 1.2, -4.0, 3.0]]])


# ----------------------------------------------------------------------------- C contract oracle
@pytest.mark.parametrize("name", FWD_CASES)
def test_contract_fp64_matches_mpmath(oracle_lib, gold, name):
    q, k, v, sink, causal, valid, rot = _case(gold, name)
    out, den = C.afa_fwd(q, k, v, C.DT_F64, sink, causal, valid, rot)
    assert normwise(out, gold[f"{name}_out"]) < 1e-13
    np.testing.assert_allclose(den, gold[f"{name}_den"], rtol=1e-13)


@pytest.mark.parametrize("name", FWD_CASES)
def test_contract_fp32_and_bf16_near_mpmath(oracle_lib, gold, name):
    q, k, v, sink, causal, valid, rot = _case(gold, name)
    out32, _ = C.afa_fwd(q, k, v, C.DT_F32, sink, causal, valid, rot)
    assert normwise(out32, gold[f"{name}_out"]) < 1e-5
    qb, kb, vb = (C.bf16_bits(a) for a in (q, k, v))
    outb, _ = C.afa_fwd(qb, kb, vb, C.DT_BF16, sink, causal, valid, rot)
    assert normwise(C.bf16_to_f32(outb), gold[f"{name}_out"]) < 2e-2


def test_contract_c1_fp32_vs_fp64(oracle_lib):
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((1, 4, 256, 64)) for _ in range(3))
    ref = O.afa_forward(q, k, v, 0.5)
    out, _ = C.afa_fwd(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), C.DT_F32, 0.5)
    assert normwise(out, ref) < 1e-5


@pytest.mark.parametrize("causal", [False, True])
def test_contract_tile_size_invariance(oracle_lib, causal):
    rng = np.random.default_rng(11)
    q, k, v = (rng.standard_normal((1, 2, 128, 16)) for _ in range(3))
    outs = [C.afa_fwd(q, k, v, C.DT_F64, 0.5, causal, None, None, bq, bk)[0]
            for bq, bk in ((128, 128), (32, 64), (16, 16), (64, 32))]
    for o in outs[1:]:
        assert normwise(o, outs[0]) < 1e-14
    f = [C.afa_fwd(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32), C.DT_F32, 0.5,
                   causal, None, None, bq, bk)[0] for bq, bk in ((128, 128), (32, 16))]
    assert normwise(f[1], f[0]) < 2e-6


def test_contract_rotary_fp64_matches_numpy(oracle_lib):
    rng = np.random.default_rng(12)
    q, k, v = (rng.standard_normal((2, 1, 48, 8)) for _ in range(3))
    c, s = O.cayley_tables(8, 48, freqs=10000.0 ** (-2.0 * np.arange(4) / 8))
    out, den = C.afa_fwd(q, k, v, C.DT_F64, 0.5, True, 40, (c, s), 16, 16)
    ref, rden = O.afa_forward(q, k, v, 0.5, True, 40, (c, s), return_denominator=True)
    assert normwise(out, ref) < 1e-13
    np.testing.assert_allclose(den, rden, rtol=1e-13)


def test_contract_rho8_f32_accuracy(oracle_lib):
    x = np.concatenate([np.linspace(-60, 60, 4001), [-1e4, -1e3, 1e3, 1e4]]).astype(np.float32)
    got = C.rho8_f32(x).astype(np.float64)
    ref = O.rho8(x.astype(np.float64))
    np.testing.assert_allclose(got, ref, rtol=3e-6)


def test_contract_bf16_and_f16_rounding_bits(oracle_lib):
    import torch
    rng = np.random.default_rng(13)
    x = np.concatenate([rng.standard_normal(4096).astype(np.float32) * 100,
                        np.array([0.0, -0.0, 1.0, 65504.0, 65520.0, 1e-8, 3.0e38, -3.4e38,
                                  np.inf, -np.inf], dtype=np.float32)])
    # exact ties: halfway between two bf16 / fp16 neighbours round to even
    ties = (np.arange(1, 513, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, ties + np.float32(0)])
    tb = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(C.bf16_bits(x), tb)
    with np.errstate(over="ignore"):
        f16 = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(C.f16_bits(x), f16)


def test_contract_backward_fp32_vs_fp64(oracle_lib):
    rng = np.random.default_rng(14)
    q, k, v, g = (rng.standard_normal((1, 2, 64, 16)).astype(np.float32) for _ in range(4))
    out, den = C.afa_fwd(q, k, v, C.DT_F32, 0.5, True)
    dq, dk, dv = C.afa_bwd(q, k, v, out, den, g, C.DT_F32, True)
    rq, rk, rv = O.afa_backward(q, k, v, g, 0.5, True)
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        assert normwise(got, ref) < 1e-5
