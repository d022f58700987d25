"""Float64 oracle for the Algebraic FlashAttention (AFA) hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this file;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.

Every function restates the mathematics of the reference path in float64 numpy,
written independently of the reference's code.  Citations point into the
reference repository (tasmaikeni13/algebraic-intelligence):

  rho8 / octic weight .......... src/kernels/pallas_afa.py:32-49, src/attention.py:18-26
                                 (oracle form: tests/reference_attention.py:5-13)
  AFA forward .................. src/kernels/pallas_afa.py:52-151 (kernel), :267-327 (exact),
                                 :330-406 (tiled); tests/reference_attention.py:44-59
  ring AFA (per device, hop) .. src/kernels/pallas_afa.py:618-662 (distributed_ring_afa)
  AFA backward (VJP) ........... src/kernels/pallas_afa.py:409-522
  A-Softmax (+VJP) ............. src/attention.py:53-91, src/primitives.py:56-79;
                                 tests/reference_attention.py:16-36
  Cayley rotary tables ......... src/attention.py:155-204; tests/reference_ago.py:21-53
  pairwise rotation ............ src/attention.py:142-152, :207-240

Pinning (what checks each function; the tests live in tests/test_oracle.py):
  rho8            known answer rho(2)^8 = 51841 + 23184*sqrt(5); rho(x)*rho(-x) = 1;
                  50-digit mpmath evaluation; derivative 8*rho^8/sqrt(1+x^2) by finite differences
  afa_forward     50-digit mpmath brute force on tiny inputs; scale invariance; causal prefix
                  invariance; split-K (ring) additivity; L=1 closed form
  ring_afa        equals afa_forward for every shard count, causal and not (the hops only
                  re-associate the sums); one shard reduces to afa_forward itself
  afa_backward    central finite differences of afa_forward (float64)
  asoftmax        Jacobian at 0 = [[2,-2],[-2,2]] (sink 0); simplex bounds; VJP by finite differences;
                  mpmath brute force
  cayley tables   closed form c_m = cos(2 m atan w), s_m = sin(2 m atan w) (checker-side trig);
                  det = 1, orthogonality, norm conservation
  rotate_pairs    orthogonality (norm preserved), R(w)^T R(w) = I, composition R_m^T R_n = R_{n-m}
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "rho", "rho8", "rho8_derivative", "afa_forward", "ring_afa", "afa_backward", "afa_flops",
    "asoftmax", "asoftmax_vjp", "cayley_base", "cayley_tables", "default_freqs",
    "rotate_pairs", "ago_apply",
]


# --------------------------------------------------------------------------- rho / rho^8
def rho(x):
    """rho(x) = x + sqrt(1 + x^2), evaluated without cancellation.

    For x < 0 the conjugate form 1 / (sqrt(1+x^2) - x) is used (both terms positive),
    mirroring the two-branch evaluation of src/kernels/pallas_afa.py:39-46.
    """
    x = np.asarray(x, dtype=np.float64)
    root = np.sqrt(1.0 + x * x)
    out = np.empty_like(x)
    pos = x >= 0
    out[pos] = x[pos] + root[pos]
    out[~pos] = 1.0 / (root[~pos] - x[~pos])
    return out


def rho8(x):
    """rho(x)^8 by three squarings (src/kernels/pallas_afa.py:47-49)."""
    r = rho(x)
    r2 = r * r
    r4 = r2 * r2
    return r4 * r4


def rho8_derivative(x):
    """d/dx rho(x)^8 = 8 rho(x)^8 / sqrt(1+x^2) (src/attention.py:39-41)."""
    x = np.asarray(x, dtype=np.float64)
    return 8.0 * rho8(x) / np.sqrt(1.0 + x * x)


# --------------------------------------------------------------------------- AFA forward
def _mask(Lq, Lk, causal, valid_len):
    """Kept (query, key) pairs: key j <= query i when causal, j < valid_len when given.
    Lk may differ from Lq (a key shard, as in src/kernels/pallas_afa.py:618-662)."""
    keep = np.ones((Lq, Lk), dtype=bool)
    if causal:
        keep &= np.arange(Lk)[None, :] <= np.arange(Lq)[:, None]
    if valid_len is not None:
        keep[:, valid_len:] = False
    return keep


def afa_forward(q, k, v, sink_omega=0.5, causal=False, valid_len=None, rotary=None,
                return_denominator=False):
    """Untiled float64 AFA forward.

    out_i = sum_j w_ij v_j / (sum_j w_ij + Omega),  w_ij = rho(s_ij)^8,
    s_ij = (q_i . k_j) / sqrt(D), with j <= i when causal and j < valid_len when given
    (src/kernels/pallas_afa.py:104-151).  ``rotary=(c, s)`` first rotates q and k with the
    Cayley tables (the model applies this before attention, src/model.py:262-264).
    Returns out (and d = sum_j w_ij + Omega with shape (..., L, 1) when requested).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    if rotary is not None:
        c, s = rotary
        q = rotate_pairs(q, c, s)
        k = rotate_pairs(k, c, s)
    D = q.shape[-1]
    scores = np.einsum("...id,...jd->...ij", q, k) / np.sqrt(D)
    w = rho8(scores)
    w = np.where(_mask(q.shape[-2], k.shape[-2], causal, valid_len), w, 0.0)
    num = np.einsum("...ij,...jd->...id", w, v)
    den = w.sum(axis=-1, keepdims=True) + sink_omega
    out = num / den
    if return_denominator:
        return out, den
    return out


def ring_afa(q, k, v, sink_omega=0.5, causal=False, num_devices=16):
    """The ring of src/kernels/pallas_afa.py:618-662 in float64, every device in turn.

    q, k, v: (..., L, D) with L = num_devices * shard_len; device d holds rows
    [d * shard_len, (d + 1) * shard_len) of each.  At hop h device d holds key/value shard
    kv = (d - h) mod n and adds p = rho(q_d k_kv^T / sqrt(D))^8 to its sums: o += p v_kv,
    den += sum_j p.  causal: p is kept where the global column index <= the global row index
    and the whole tile is dropped when kv > d (which the index rule already implies).
    out_d = o / (den + sink_omega); the devices' outputs are returned side by side.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    n = num_devices
    L, D = q.shape[-2], q.shape[-1]
    S = L // n
    out = np.empty_like(q)
    rows = np.arange(S)[:, None]
    cols = np.arange(S)[None, :]
    for d in range(n):
        qd = q[..., d * S:(d + 1) * S, :]
        o = np.zeros_like(qd)
        den = np.zeros(qd.shape[:-1] + (1,))
        for hop in range(n):
            kv = (d - hop) % n
            kd, vd = k[..., kv * S:(kv + 1) * S, :], v[..., kv * S:(kv + 1) * S, :]
            p = rho8(np.einsum("...id,...jd->...ij", qd, kd) / np.sqrt(D))
            if causal:
                p = np.where((cols + kv * S <= rows + d * S) & (kv <= d), p, 0.0)
            o += np.einsum("...ij,...jd->...id", p, vd)
            den += p.sum(axis=-1, keepdims=True)
        out[..., d * S:(d + 1) * S, :] = o / (den + sink_omega)
    return out


def afa_flops(B, H, L, D, causal):
    """Algorithmic FLOPs of one forward: 4*B*H*D*N_pairs (QK^T + PV over unmasked pairs)."""
    pairs = L * (L + 1) // 2 if causal else L * L
    return 4 * B * H * D * pairs


# --------------------------------------------------------------------------- AFA backward
def afa_backward(q, k, v, g, sink_omega=0.5, causal=False, valid_len=None):
    """Float64 VJP of afa_forward with respect to (q, k, v), derived by the quotient rule.

    With N_i = sum_j w_ij v_j and S_i = sum_j w_ij + Omega, out_i = N_i / S_i:
      d out_i / d w_ij = (v_j - out_i) / S_i
      dL/dw_ij = (g_i . v_j - g_i . out_i) / S_i
      dL/ds_ij = dL/dw_ij * 8 w_ij / sqrt(1 + s_ij^2)
      dq_i = scale * sum_j dL/ds_ij k_j,  dk_j = scale * sum_i dL/ds_ij q_i,
      dv_j = sum_i w_ij g_i / S_i.
    The reference computes the same quantity from cached (out, d) in
    src/kernels/pallas_afa.py:451-517; this restatement works from the definitions.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    L, D = q.shape[-2], q.shape[-1]
    scale = 1.0 / np.sqrt(D)
    scores = np.einsum("...id,...jd->...ij", q, k) * scale
    keep = _mask(L, L, causal, valid_len)
    w = np.where(keep, rho8(scores), 0.0)
    S = w.sum(axis=-1, keepdims=True) + sink_omega
    out = np.einsum("...ij,...jd->...id", w, v) / S
    gv = np.einsum("...id,...jd->...ij", g, v)
    go = np.sum(g * out, axis=-1, keepdims=True)
    dw = (gv - go) / S
    ds = np.where(keep, dw * 8.0 * w / np.sqrt(1.0 + scores * scores), 0.0)
    dq = np.einsum("...ij,...jd->...id", ds, k) * scale
    dk = np.einsum("...ij,...id->...jd", ds, q) * scale
    dv = np.einsum("...ij,...id->...jd", w / S, g)
    return dq, dk, dv


# --------------------------------------------------------------------------- A-Softmax
def asoftmax(x, sink_omega=0.5, eps=1e-5):
    """AVN-normalised octic attention over the last axis (src/attention.py:59-67).

    z = x / sqrt(mean(x^2) + eps);  p = rho(z)^8 / (sum rho(z)^8 + Omega).
    """
    x = np.asarray(x, dtype=np.float64)
    tau = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    w = rho8(x * tau)
    return w / (w.sum(axis=-1, keepdims=True) + sink_omega)


def asoftmax_vjp(x, g, sink_omega=0.5, eps=1e-5):
    """VJP of asoftmax by explicit chain rule through AVN and the sink-normalised quotient.

    Let z = tau x, tau = (mean(x^2)+eps)^(-1/2), w = rho(z)^8, S = sum w + Omega, p = w/S.
    dL/dw_j = g_j / S - (g . w) / S^2;  dL/dz_j = dL/dw_j * rho8'(z_j);
    dz_j/dx_m = tau delta_jm - x_j tau^3 x_m / n.
    """
    x = np.asarray(x, dtype=np.float64)
    g = np.asarray(g, dtype=np.float64)
    n = x.shape[-1]
    tau = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    z = x * tau
    w = rho8(z)
    S = w.sum(axis=-1, keepdims=True) + sink_omega
    dw = g / S - np.sum(g * w, axis=-1, keepdims=True) / (S * S)
    dz = dw * rho8_derivative(z)
    return tau * dz - x * tau ** 3 * np.sum(x * dz, axis=-1, keepdims=True) / n


# --------------------------------------------------------------------------- AGO (Cayley rotary)
def default_freqs(dim, base=10000.0):
    """Default Cayley parameters w_k = 1/(1 + alpha k)^2, alpha = (sqrt(base)-1)/max(D/2-1, 1)
    (src/attention.py:180-187)."""
    pairs = dim // 2
    kk = np.arange(pairs, dtype=np.float64)
    alpha = (np.sqrt(base) - 1.0) / max(float(pairs - 1), 1.0)
    return 1.0 / (1.0 + alpha * kk) ** 2


def cayley_base(w):
    """Cayley map of the skew matrix [[0,-w],[w,0]]: c = (1-w^2)/(1+w^2), s = 2w/(1+w^2)."""
    w = np.asarray(w, dtype=np.float64)
    return (1.0 - w * w) / (1.0 + w * w), 2.0 * w / (1.0 + w * w)


def cayley_tables(dim, max_seq_len, freqs=None, base=10000.0):
    """(c, s) tables of shape (max_seq_len, dim/2): row 0 = (1, 0), row m+1 = R(w) row m
    renormalised to unit length (src/attention.py:189-203)."""
    if dim <= 0 or dim % 2:
        raise ValueError("dim must be a positive even integer")
    if max_seq_len <= 0:
        raise ValueError("max_seq_len must be a positive integer")
    w = default_freqs(dim, base) if freqs is None else np.asarray(freqs, dtype=np.float64)
    cb, sb = cayley_base(w)
    c = np.empty((max_seq_len, dim // 2))
    s = np.empty((max_seq_len, dim // 2))
    c[0], s[0] = 1.0, 0.0
    for m in range(1, max_seq_len):
        cn = cb * c[m - 1] - sb * s[m - 1]
        sn = sb * c[m - 1] + cb * s[m - 1]
        inv = 1.0 / np.sqrt(cn * cn + sn * sn)
        c[m], s[m] = cn * inv, sn * inv
    return c, s


def rotate_pairs(x, c, s):
    """Rotate consecutive (even, odd) feature pairs of x (..., L, D) by position-indexed
    (c, s) rows (src/attention.py:142-152).  c, s have shape (>=L, D/2)."""
    x = np.asarray(x, dtype=np.float64)
    L = x.shape[-2]
    c = np.asarray(c, dtype=np.float64)[:L]
    s = np.asarray(s, dtype=np.float64)[:L]
    x0 = x[..., 0::2]
    x1 = x[..., 1::2]
    out = np.empty_like(x)
    out[..., 0::2] = c * x0 - s * x1
    out[..., 1::2] = s * x0 + c * x1
    return out


def ago_apply(q, k, c, s, seq_axis):
    """apply_ago_rotations for an explicit sequence axis (src/attention.py:207-240)."""
    q = np.moveaxis(np.asarray(q, dtype=np.float64), seq_axis, -2)
    k = np.moveaxis(np.asarray(k, dtype=np.float64), seq_axis, -2)
    qr = np.moveaxis(rotate_pairs(q, c, s), -2, seq_axis)
    kr = np.moveaxis(rotate_pairs(k, c, s), -2, seq_axis)
    return qr, kr
