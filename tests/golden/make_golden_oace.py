"""Write tests/golden/oace_golden.npz: small fixtures for the OACE loss head.

The reference ships no golden vectors for this path and its JAX code cannot run here.  The
expected values are computed from the definitions in 40-digit mpmath arithmetic, independently
of oracle/ (float64 numpy) and of the rho factorisation the kernels use:

  logits .......... z = h W (src/kernels/pallas_oace.py:130-131)
  AVN ............. tau = 1/sqrt(mean_v z^2 + eps), x = tau z (:122, model.py:181-183)
  A-Softmax ....... p_v = rho(x_v)^8 / sum_u rho(x_u)^8, rho(x) = x + sqrt(1 + x^2)
  score ........... gamma (8 p_t^(-1/8) + 8/7 sum_v p_v^(7/8) - 64/7), the proper power score for
                    alpha = 1/8 with integer targets (src/loss.py:37-68), evaluated with mpmath
                    powers; the loss is its mean over rows
  gradients ....... mpmath numerical differentiation of the loss (mpmath.diff, central)

Inputs are rounded once to bfloat16-representable values, so the same fixture checks fp64, fp32,
bf16 and fp16 runs (exact inputs for all).

    python tests/golden/make_golden_oace.py
"""
from __future__ import annotations

import os

import mpmath as mp
import numpy as np

from make_golden import bf16_exact

mp.mp.dps = 40
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "oace_golden.npz")


def row_loss_mp(z, t, eps, gamma):
    V = len(z)
    tau = 1 / mp.sqrt(sum(x * x for x in z) / V + eps)
    xs = [tau * x for x in z]
    w = [(x + mp.sqrt(1 + x * x)) ** 8 for x in xs]
    S = sum(w)
    p = [wi / S for wi in w]
    loss = gamma * (8 * p[t] ** mp.mpf(-0.125) + mp.mpf(8) / 7 * sum(pi ** mp.mpf(0.875) for pi in p) - mp.mpf(64) / 7)
    return loss, tau


def logits_mp(H, W):
    N, d = len(H), len(H[0])
    V = len(W[0])
    return [[sum(H[n][k] * W[k][v] for k in range(d)) for v in range(V)] for n in range(N)]


def mean_loss_mp(Z, T, eps, gamma):
    ls = [row_loss_mp(Z[n], T[n], eps, gamma) for n in range(len(Z))]
    return sum(l for l, _ in ls) / len(Z), ls


def to_mp(a):
    return [[mp.mpf(float(x)) for x in row] for row in a]


def linear_case(fx, name, N, d, V, eps, gamma, seed, scale):
    rng = np.random.default_rng(seed)
    h = bf16_exact(rng.standard_normal((N, d)) * scale)
    w = bf16_exact(rng.standard_normal((d, V)) * scale)
    t = rng.integers(0, V, size=N)
    H, W = to_mp(h), to_mp(w)
    loss, rows = mean_loss_mp(logits_mp(H, W), list(t), eps, gamma)

    def with_h(i, j):
        def f(e):
            H2 = [row[:] for row in H]
            H2[i][j] += e
            return mean_loss_mp(logits_mp(H2, W), list(t), eps, gamma)[0]
        return f

    def with_w(i, j):
        def f(e):
            W2 = [row[:] for row in W]
            W2[i][j] += e
            return mean_loss_mp(logits_mp(H, W2), list(t), eps, gamma)[0]
        return f

    dh = np.array([[float(mp.diff(with_h(i, j), 0)) for j in range(d)] for i in range(N)])
    dw = np.array([[float(mp.diff(with_w(i, j), 0)) for j in range(V)] for i in range(d)])
    fx[f"{name}_h"], fx[f"{name}_w"], fx[f"{name}_t"] = h, w, t
    fx[f"{name}_cfg"] = np.array([eps, gamma])
    fx[f"{name}_loss"] = np.array(float(loss))
    fx[f"{name}_row_loss"] = np.array([float(l) for l, _ in rows])
    fx[f"{name}_tau"] = np.array([float(tau) for _, tau in rows])
    fx[f"{name}_dh"], fx[f"{name}_dw"] = dh, dw


def softmax_case(fx, name, N, V, eps, gamma, seed, scale):
    rng = np.random.default_rng(seed)
    z = bf16_exact(rng.standard_normal((N, V)) * scale)
    t = rng.integers(0, V, size=N)
    Z = to_mp(z)
    loss, rows = mean_loss_mp(Z, list(t), eps, gamma)

    def with_z(i, j):
        def f(e):
            Z2 = [row[:] for row in Z]
            Z2[i][j] += e
            return mean_loss_mp(Z2, list(t), eps, gamma)[0]
        return f

    dz = np.array([[float(mp.diff(with_z(i, j), 0)) for j in range(V)] for i in range(N)])
    fx[f"{name}_z"], fx[f"{name}_t"] = z, t
    fx[f"{name}_cfg"] = np.array([eps, gamma])
    fx[f"{name}_loss"] = np.array(float(loss))
    fx[f"{name}_row_loss"] = np.array([float(l) for l, _ in rows])
    fx[f"{name}_dz"] = dz


def main():
    fx = {}
    linear_case(fx, "lin_small", N=3, d=4, V=7, eps=0.5, gamma=2.0, seed=11, scale=1.0)
    linear_case(fx, "lin_d32", N=3, d=32, V=7, eps=100.0, gamma=2.0, seed=12, scale=2.0)
    softmax_case(fx, "sm", N=3, V=9, eps=100.0, gamma=1.5, seed=13, scale=12.0)
    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT}: {len(fx)} arrays")


if __name__ == "__main__":
    main()
