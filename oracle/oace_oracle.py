"""Float64 oracle for the fused Linear + OACE loss head and the OACE softmax loss.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this file;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.

Restates, in float64 numpy and independently of the reference's code:

  octic_parts ................... src/kernels/pallas_oace.py:38-56 (two-branch rho, rho^7, rho^8, r)
  oace_softmax_loss (+VJP) ...... src/model.py:180-240 (fused_oace_softmax_loss over given logits)
  fused_linear_oace_forward ..... src/kernels/pallas_oace.py:59-209 (vocabulary-chunked forward,
                                  Gram second moment, three forward reductions, target capture)
  fused_linear_oace_backward .... src/kernels/pallas_oace.py:212-269 (streamed dz, dW, dh)
  oace_score .................... src/loss.py:37-68 (proper power score for alpha = 1/8 from
                                  probabilities, with numpy powers instead of the rho factorization)

Pinning (tests/test_oracle_oace.py):
  octic_parts        rho(x) rho(-x) = 1; rho^8 against the AFA oracle's rho8; rho^7 rho = rho^8
  forward            equals oace_softmax_loss of the materialised logits (the reference's own
                     parity test, pallas_oace tests :62-80); equals oace_score of the A-Softmax
                     probabilities (power form p^(-1/8), p^(7/8) by numpy); closed form at h = 0
                     (uniform p): loss = gamma * 64/7 * (V^(1/8) - 1); chunk-size invariance;
                     Gram second moment equal to the direct sum of squared logits
  radial             equals the full-vocabulary definition (pallas_oace tests :116-156)
  backward           central finite differences of the forward (float64) for dh and dW; the
                     softmax-loss VJP by finite differences of oace_softmax_loss
"""
from __future__ import annotations

import math

import numpy as np

__all__ = ["octic_parts", "oace_softmax_loss", "oace_softmax_loss_vjp", "fused_linear_oace_forward",
           "fused_linear_oace_backward", "oace_score", "ROW_FIELDS"]

# Per-row values the forward caches for the backward, in this order (pallas_oace.py:189-202).
ROW_FIELDS = ("tau", "inv_S", "S_eighth", "sum_p78", "p_c_inv8", "radial", "loss")


def octic_parts(s):
    """(k8, rho7, rho, r) of s: r = 1/sqrt(1+s^2); rho = s + (1+s^2) r for s >= 0 and
    r / (1 - s r) for s < 0 (no cancellation); k8 = rho^8, rho7 = rho^7 (pallas_oace.py:38-56)."""
    s = np.asarray(s, dtype=np.float64)
    rad = 1.0 + s * s
    r = 1.0 / np.sqrt(rad)
    u = s * r
    rho = np.where(s < 0, r / np.where(s < 0, 1.0 - u, 1.0), s + rad * r)
    k2 = rho * rho
    k4 = k2 * k2
    return k4 * k4, rho * k2 * k4, rho, r


def _rows_from_logits(z, targets, eps, gamma):
    """Per-row OACE quantities from materialised logits z (N, V) (model.py:180-210)."""
    z = np.asarray(z, dtype=np.float64)
    V = z.shape[-1]
    tau = 1.0 / np.sqrt(np.sum(z * z, axis=-1, keepdims=True) / V + eps)
    n = z * tau
    k8, rho7, rho, r = octic_parts(n)
    inv_S = 1.0 / np.sum(k8, axis=-1, keepdims=True)
    S8 = inv_S ** -0.125
    p = k8 * inv_S
    p78 = S8 * inv_S * rho7
    sum_p78 = np.sum(p78, axis=-1, keepdims=True)
    rho_c = np.take_along_axis(rho, np.asarray(targets)[:, None], axis=-1)
    p_c_inv8 = S8 / rho_c
    loss = gamma * (8.0 * p_c_inv8 + (8.0 / 7.0) * sum_p78 - 64.0 / 7.0)
    return dict(n=n, tau=tau, p=p, p78=p78, r=r, sum_p78=sum_p78, p_c_inv8=p_c_inv8, inv_S=inv_S,
                S_eighth=S8, loss=loss)


def oace_softmax_loss(logits, targets, eps=100.0, gamma=2.0):
    """Mean OACE loss of the AVN-normalised A-Softmax over the last axis (model.py:180-210).
    Returns (loss, cache) with the per-row values of the VJP."""
    z = np.asarray(logits, dtype=np.float64)
    shape = z.shape
    z2 = z.reshape(-1, shape[-1])
    t = np.asarray(targets).reshape(-1)
    c = _rows_from_logits(z2, t, eps, gamma)
    c["targets"] = t
    c["shape"] = shape
    return float(np.mean(c["loss"])), c


def oace_softmax_loss_vjp(cache, g, gamma=2.0):
    """d loss / d logits (model.py:213-226): bracket = p78 - onehot p_c^-1/8 - p (sum_p78 - p_c^-1/8);
    radial = mean(r bracket n); dx = tau c (r bracket - radial n), c = 8 gamma g / N."""
    n, p, p78, r, t = cache["n"], cache["p"], cache["p78"], cache["r"], cache["targets"]
    V = n.shape[-1]
    onehot = np.zeros_like(n)
    onehot[np.arange(n.shape[0]), t] = 1.0
    diff = cache["sum_p78"] - cache["p_c_inv8"]
    bracket = p78 - onehot * cache["p_c_inv8"] - p * diff
    rb = r * bracket
    radial = np.sum(rb * n, axis=-1, keepdims=True) / V
    c = 8.0 * gamma / float(t.size) * g
    return ((cache["tau"] * c) * (rb - radial * n)).reshape(cache["shape"])


def fused_linear_oace_forward(h, w, targets, eps_vocab=100.0, gamma=2.0, chunk_size=4096):
    """Vocabulary-chunked fused forward (pallas_oace.py:59-209).  h (..., d), w (d, V).

    The second moment sum_v z_v^2 comes from the Gram matrix W W^T (d x d) as in the reference;
    the vocabulary pass accumulates sum k8, sum rho7, sum (r n) k8, sum (r n) rho7 and captures
    rho and r n at the target.  Returns (mean loss, per-row dict of ROW_FIELDS)."""
    h = np.asarray(h, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    d, V = w.shape
    hf = h.reshape(-1, d)
    t = np.asarray(targets).reshape(-1)
    N = hf.shape[0]
    if chunk_size <= 0:
        raise ValueError("chunk_size must be positive")
    gram = w @ w.T
    ss = np.sum((hf @ gram) * hf, axis=-1, keepdims=True)
    tau = 1.0 / np.sqrt(ss / V + eps_vocab)
    acc = np.zeros((N, 4))
    rho_t = np.zeros((N, 1))
    rn_t = np.zeros((N, 1))
    for c0 in range(0, V, chunk_size):
        c1 = min(c0 + chunk_size, V)
        n = (hf @ w[:, c0:c1]) * tau
        k8, rho7, rho, r = octic_parts(n)
        rn = r * n
        acc[:, 0] += k8.sum(-1)
        acc[:, 1] += rho7.sum(-1)
        acc[:, 2] += (rn * k8).sum(-1)
        acc[:, 3] += (rn * rho7).sum(-1)
        inside = (t >= c0) & (t < c1)
        idx = np.clip(t - c0, 0, c1 - c0 - 1)
        rho_t[inside, 0] = rho[inside, idx[inside]]
        rn_t[inside, 0] = rn[inside, idx[inside]]
    inv_S = 1.0 / acc[:, :1]
    S8 = inv_S ** -0.125
    scale = S8 * inv_S
    sum_p78 = scale * acc[:, 1:2]
    p_c_inv8 = S8 / rho_t
    diff = sum_p78 - p_c_inv8
    radial = (scale * acc[:, 3:4] - rn_t * p_c_inv8 - diff * inv_S * acc[:, 2:3]) / V
    loss = gamma * (8.0 * p_c_inv8 + (8.0 / 7.0) * sum_p78 - 64.0 / 7.0)
    rows = dict(tau=tau, inv_S=inv_S, S_eighth=S8, sum_p78=sum_p78, p_c_inv8=p_c_inv8, radial=radial,
                loss=loss)
    return float(np.mean(loss)), rows


def fused_linear_oace_backward(h, w, targets, rows, g=1.0, gamma=2.0, chunk_size=4096):
    """Streamed backward (pallas_oace.py:212-269): per chunk, recompute n = (h w_c) tau,
    dz = tau c (r bracket - radial n) with c = 8 gamma g / N, then dW_c = h^T dz and
    dh += dz w_c^T.  Returns (dh shaped like h, dW shaped like w)."""
    h = np.asarray(h, dtype=np.float64)
    w = np.asarray(w, dtype=np.float64)
    d, V = w.shape
    hf = h.reshape(-1, d)
    t = np.asarray(targets).reshape(-1)
    N = hf.shape[0]
    tau, inv_S, S8 = rows["tau"], rows["inv_S"], rows["S_eighth"]
    diff = rows["sum_p78"] - rows["p_c_inv8"]
    c = 8.0 * gamma / float(N) * g
    dh = np.zeros_like(hf)
    dw = np.zeros_like(w)
    for c0 in range(0, V, chunk_size):
        c1 = min(c0 + chunk_size, V)
        n = (hf @ w[:, c0:c1]) * tau
        k8, rho7, _, r = octic_parts(n)
        onehot = (t[:, None] == np.arange(c0, c1)[None, :]).astype(np.float64)
        bracket = S8 * inv_S * rho7 - onehot * rows["p_c_inv8"] - k8 * inv_S * diff
        dz = tau * c * (r * bracket - rows["radial"] * n)
        dw[:, c0:c1] = hf.T @ dz
        dh += dz @ w[:, c0:c1].T
    return dh.reshape(h.shape), dw


def oace_score(p, targets, gamma=2.0):
    """Per-row proper power score of probabilities p for integer targets (loss.py:37-68):
    gamma (8 p_y^(-1/8) + 8/7 sum p^(7/8) - 64/7), evaluated with numpy powers."""
    p = np.asarray(p, dtype=np.float64)
    t = np.asarray(targets)
    py = np.take_along_axis(p, t[:, None], axis=-1)[:, 0]
    return gamma * (8.0 * py ** -0.125 + (8.0 / 7.0) * np.sum(p ** 0.875, axis=-1) - 64.0 / 7.0)


def uniform_loss(V, gamma=2.0):
    """Closed form at uniform probabilities (all logits equal): gamma * 64/7 * (V^(1/8) - 1)."""
    return gamma * 64.0 / 7.0 * (math.pow(V, 0.125) - 1.0)
