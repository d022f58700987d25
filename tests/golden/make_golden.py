"""Write tests/golden/afa_golden.npz: small AFA / A-Softmax / Cayley-rotary fixtures.

The reference ships no golden vectors for this path and its JAX code cannot run here, so the
expected outputs are computed from the definitions in 40-digit mpmath arithmetic, independently
of oracle/ (which uses float64 numpy and a C restatement):

  rho(s)^8 ........ rho(s) = s + sqrt(1 + s^2), evaluated directly at 40 digits
                    (src/kernels/pallas_afa.py:32-49)
  AFA forward ..... out_i = sum_j w_ij v_j / (sum_j w_ij + Omega), w_ij = rho(q_i.k_j / sqrt(D))^8,
                    causal j <= i, keys j >= valid_len dropped (src/kernels/pallas_afa.py:97-151)
  AFA backward .... mpmath numerical differentiation of the forward (mpmath.diff, central)
  A-Softmax ....... z = x / sqrt(mean(x^2) + eps), p = rho(z)^8 / (sum rho(z)^8 + Omega)
                    (src/attention.py:59-67)
  Cayley tables ... closed form c_m = cos(2 m atan w), s_m = sin(2 m atan w), which the
                    recurrence of src/attention.py:189-203 reproduces in exact arithmetic

Inputs are drawn with numpy's default_rng and rounded once to bfloat16-representable values, so
the same fixture checks fp64, fp32 and bf16 runs (exact inputs for all three).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import mpmath as mp
import numpy as np

mp.mp.dps = 40
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "afa_golden.npz")


def bf16_exact(x):
    """Round float64 values to the nearest bfloat16 (ties to even) and return them as float64."""
    f = np.asarray(x, dtype=np.float32)
    b = f.view(np.uint32).astype(np.uint64)
    b = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return b.astype(np.uint32).view(np.float32).astype(np.float64)


def rho8_mp(s):
    r = s + mp.sqrt(1 + s * s)
    return r ** 8


def afa_mp(q, k, v, sink, causal, valid_len, rot=None):
    """Returns (out, den) as float64 arrays for q, k, v of shape (B, H, L, D)."""
    B, H, L, D = q.shape
    out = np.zeros((B, H, L, D))
    den = np.zeros((B, H, L, 1))
    inv = 1 / mp.sqrt(D)
    for b in range(B):
        for h in range(H):
            Q = [[mp.mpf(float(x)) for x in row] for row in q[b, h]]
            K = [[mp.mpf(float(x)) for x in row] for row in k[b, h]]
            V = [[mp.mpf(float(x)) for x in row] for row in v[b, h]]
            if rot is not None:
                Q = [rotate_mp(Q[m], rot[0][m], rot[1][m]) for m in range(L)]
                K = [rotate_mp(K[m], rot[0][m], rot[1][m]) for m in range(L)]
            for i in range(L):
                num = [mp.mpf(0)] * D
                tot = mp.mpf(0)
                for j in range(L):
                    if (causal and j > i) or (valid_len is not None and j >= valid_len):
                        continue
                    s = mp.fsum(Q[i][d] * K[j][d] for d in range(D)) * inv
                    w = rho8_mp(s)
                    tot += w
                    num = [num[d] + w * V[j][d] for d in range(D)]
                d_tot = tot + mp.mpf(sink)
                out[b, h, i] = [float(x / d_tot) for x in num]
                den[b, h, i, 0] = float(d_tot)
    return out, den


def rotate_mp(x, c, s):
    y = list(x)
    for p in range(len(x) // 2):
        x0, x1 = x[2 * p], x[2 * p + 1]
        y[2 * p] = c[p] * x0 - s[p] * x1
        y[2 * p + 1] = s[p] * x0 + c[p] * x1
    return y


def cayley_mp(freqs, L):
    """40-digit closed-form tables (lists of mpf rows) and their float64 images."""
    th = [2 * mp.atan(mp.mpf(float(w))) for w in freqs]
    c = [[mp.cos(m * t) for t in th] for m in range(L)]
    s = [[mp.sin(m * t) for t in th] for m in range(L)]
    as_np = lambda t: np.array([[float(x) for x in row] for row in t])
    return c, s, as_np(c), as_np(s)


def asoftmax_mp(x, sink, eps):
    n = len(x)
    X = [mp.mpf(float(t)) for t in x]
    tau = 1 / mp.sqrt(mp.fsum(t * t for t in X) / n + mp.mpf(eps))
    w = [rho8_mp(tau * t) for t in X]
    S = mp.fsum(w) + mp.mpf(sink)
    return [t / S for t in w]


def main():
    rng = np.random.default_rng(20260101)
    fx = {}

    # rho^8 at known points, including the far negative tail (tests/test_pallas_afa.py:90-96)
    xs = np.array([-1e4, -1e3, -1e2, -30.0, -3.0, -1.0, -0.25, -1e-3, 0.0, 1e-3, 0.25, 1.0, 2.0,
                   3.0, 30.0, 1e2, 1e3, 1e4])
    fx["rho8_x"] = xs
    fx["rho8_y"] = np.array([float(rho8_mp(mp.mpf(float(t)))) for t in xs])

    def draw(shape, scale):
        return bf16_exact(rng.standard_normal(shape) * scale)

    # AFA forward cases: (name, shape, scale, sink, causal, valid_len, rotary freqs)
    cases = [
        ("fwd_plain", (1, 2, 12, 8), 1.0, 0.5, False, None, None),
        ("fwd_causal_valid", (1, 1, 16, 16), 1.0, 1.0, True, 11, None),
        ("fwd_nosink_causal", (2, 1, 8, 4), 1.0, 0.0, True, None, None),
        ("fwd_tail", (1, 1, 10, 8), 6.0, 0.5, False, None, None),
        ("fwd_rotary", (1, 1, 10, 8), 1.0, 0.5, True, None,
         10000.0 ** (-2.0 * np.arange(4) / 8)),
        ("fwd_d64_rotary", (1, 2, 20, 64), 1.0, 0.5, True, 17,
         10000.0 ** (-2.0 * np.arange(32) / 64)),
        ("fwd_d128", (1, 1, 9, 128), 1.0, 0.5, False, None, None),
    ]
    for name, shape, scale, sink, causal, valid, freqs in cases:
        q, k, v = draw(shape, scale), draw(shape, scale), draw(shape, 1.0)
        rot = None
        if freqs is not None:
            cm, sm, cn, sn = cayley_mp(freqs, shape[2])
            rot = (cm, sm)
            fx[f"{name}_freqs"] = np.asarray(freqs, dtype=np.float64)
            fx[f"{name}_cos"], fx[f"{name}_sin"] = cn, sn
        out, den = afa_mp(q, k, v, sink, causal, valid, rot)
        fx[f"{name}_q"], fx[f"{name}_k"], fx[f"{name}_v"] = q, k, v
        fx[f"{name}_out"], fx[f"{name}_den"] = out, den
        fx[f"{name}_cfg"] = np.array([sink, float(causal), -1.0 if valid is None else float(valid)])

    # AFA backward: gradient of sum(g * out) by 40-digit numerical differentiation
    shape = (1, 1, 6, 4)
    q, k, v, g = (draw(shape, 1.0) for _ in range(4))
    sink, causal = 0.5, True
    fx["bwd_q"], fx["bwd_k"], fx["bwd_v"], fx["bwd_g"] = q, k, v, g
    fx["bwd_cfg"] = np.array([sink, float(causal), -1.0])
    L, D = shape[2], shape[3]

    def loss_of(arrs):
        Q, K, V = arrs
        inv = 1 / mp.sqrt(D)
        tot = mp.mpf(0)
        for i in range(L):
            num = [mp.mpf(0)] * D
            den_ = mp.mpf(sink)
            for j in range(i + 1):
                w = rho8_mp(mp.fsum(Q[i][d] * K[j][d] for d in range(D)) * inv)
                den_ += w
                num = [num[d] + w * V[j][d] for d in range(D)]
            tot += mp.fsum(mp.mpf(float(g[0, 0, i, d])) * num[d] / den_ for d in range(D))
        return tot

    base = [[[mp.mpf(float(x)) for x in row] for row in a[0, 0]] for a in (q, k, v)]
    grads = []
    for which in range(3):
        gr = np.zeros(shape)
        for i in range(L):
            for d in range(D):
                def f(t, which=which, i=i, d=d):
                    arrs = [[list(r) for r in a] for a in base]
                    arrs[which][i][d] = t
                    return loss_of(arrs)
                gr[0, 0, i, d] = float(mp.diff(f, base[which][i][d]))
        grads.append(gr)
    fx["bwd_dq"], fx["bwd_dk"], fx["bwd_dv"] = grads

    # A-Softmax rows of several lengths and sinks (src/attention.py:53-91)
    for n, sink in ((1, 0.5), (3, 0.0), (7, 1.0), (64, 0.5)):
        x = draw((n,), 2.0)
        fx[f"asm_{n}_x"] = x
        fx[f"asm_{n}_y"] = np.array([float(t) for t in asoftmax_mp(x, sink, 1e-5)])
        fx[f"asm_{n}_cfg"] = np.array([sink, 1e-5])

    # Cayley tables: default parameters (src/attention.py:180-187) and C3's t_i
    dim, L = 8, 64
    pairs = dim // 2
    alpha = (mp.sqrt(10000) - 1) / (pairs - 1)
    wdef = np.array([float(1 / (1 + alpha * i) ** 2) for i in range(pairs)])
    for name, w in (("cayley_default", wdef), ("cayley_c3", 10000.0 ** (-2.0 * np.arange(pairs) / dim))):
        _, _, cn, sn = cayley_mp(w, L)
        fx[f"{name}_freqs"], fx[f"{name}_cos"], fx[f"{name}_sin"] = w, cn, sn

    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT}: {len(fx)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
