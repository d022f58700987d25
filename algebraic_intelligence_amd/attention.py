"""Octic attention primitives on MI355X: the call surface of src/attention.py.

octic_kernel / algebraic_softmax / CayleyRotary / build_cayley_rotary_matrix /
apply_ago_rotations with the reference's names, argument meanings and errors
(tasmaikeni13/algebraic-intelligence, src/attention.py), on torch tensors on a HIP device.
Every computation runs in the gfx950 kernels of libafa_hip.so (include/afa.h).
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from . import _lib

__all__ = [
    "octic_kernel", "algebraic_softmax", "CayleyRotary", "build_cayley_rotary_matrix",
    "apply_ago_rotations", "rotate_tensor",
]


def _float_input(x) -> torch.Tensor:
    if not isinstance(x, torch.Tensor):
        x = torch.as_tensor(x)
    if not x.is_floating_point():
        raise TypeError("expected a floating point array")
    return x


# ------------------------------------------------------------------------------------ octic
class _Octic(torch.autograd.Function):
    """rho(x)^8 with the cached VJP 8 r rho^8 g (src/attention.py:29-44)."""

    @staticmethod
    def forward(ctx, x):
        dev = _lib.require_device(x)
        xc = x.contiguous()
        y = torch.empty_like(xc)
        with torch.cuda.device(dev):
            rc = _lib.lib().octic_fwd(_lib.dtype_code(x.dtype), xc.numel(), _lib.ptr(xc), _lib.ptr(y),
                                      _lib.stream_ptr(dev))
        _lib.check(rc, "octic_fwd")
        ctx.save_for_backward(xc)
        return y

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        dev = x.device
        gc = g.to(x.dtype).contiguous()
        dx = torch.empty_like(x)
        with torch.cuda.device(dev):
            rc = _lib.lib().octic_bwd(_lib.dtype_code(x.dtype), x.numel(), _lib.ptr(x), _lib.ptr(gc),
                                      _lib.ptr(dx), _lib.stream_ptr(dev))
        _lib.check(rc, "octic_bwd")
        return dx.to(g.dtype)


def octic_kernel(x) -> torch.Tensor:
    """rho(x)^8 via exactly three squarings after evaluating rho (src/attention.py:47-50),
    with rho(x) = x + sqrt(1+x^2) evaluated in its cancellation-free two-branch form and the
    arithmetic promoted to fp32 (fp64 stays fp64); the result has the input dtype."""
    return _Octic.apply(_float_input(x))


def _vmu_octic_kernel(s: torch.Tensor) -> torch.Tensor:
    """Elementwise rho(s)^8 of src/kernels/pallas_afa.py:32-49 (same function as octic_kernel)."""
    return octic_kernel(s)


# the differentiable octic weight under the reference's private name (src/attention.py:34-44)
_octic = octic_kernel


def _kernel(z):
    """(rho(z)^8, r) with r = rsqrt(1 + z^2), from one evaluation (src/attention.py:18-26): the
    octic weight and the factor of its VJP 8 r rho^8 g.  Both come back in the accumulation type,
    fp32 (fp64 for fp64 z), which is the type the reference's callers hand it (_accumulate,
    src/primitives.py:17-21).  Not differentiable, as in the reference, whose custom VJPs use r
    instead."""
    z = _float_input(z)
    dev = _lib.require_device(z)
    zc = z.contiguous()
    acc = _lib.accum_dtype(z.dtype)
    k = torch.empty(zc.shape, dtype=acc, device=dev)
    r = torch.empty(zc.shape, dtype=acc, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.lib().octic_fwd_r(_lib.dtype_code(z.dtype), zc.numel(), _lib.ptr(zc), _lib.ptr(k), _lib.ptr(r),
                                    _lib.stream_ptr(dev))
    _lib.check(rc, "octic_fwd_r")
    return k, r


# ------------------------------------------------------------------------------ A-Softmax
class _ASoftmax(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, sink_omega, eps):
        dev = _lib.require_device(x)
        xc = x.contiguous()
        cols = xc.shape[-1]
        rows = xc.numel() // cols
        y = torch.empty_like(xc)
        with torch.cuda.device(dev):
            rc = _lib.lib().asoftmax_fwd(_lib.dtype_code(x.dtype), rows, cols, _lib.ptr(xc), _lib.ptr(y),
                                         float(sink_omega), float(eps), _lib.stream_ptr(dev))
        _lib.check(rc, "asoftmax_fwd")
        ctx.save_for_backward(xc)
        ctx.cfg = (sink_omega, eps)
        return y

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        sink_omega, eps = ctx.cfg
        gc = g.to(x.dtype).contiguous()
        dx = torch.empty_like(x)
        cols = x.shape[-1]
        with torch.cuda.device(x.device):
            rc = _lib.lib().asoftmax_bwd(_lib.dtype_code(x.dtype), x.numel() // cols, cols, _lib.ptr(x),
                                         _lib.ptr(gc), _lib.ptr(dx), float(sink_omega), float(eps),
                                         _lib.stream_ptr(x.device))
        _lib.check(rc, "asoftmax_bwd")
        return dx.to(g.dtype), None, None


def algebraic_softmax(scores, sink_omega: float = 0.5, eps: float = 1e-5) -> torch.Tensor:
    """AVN-bounded octic attention over the last axis (src/attention.py:53-91):
    p = rho(z)^8 / (sum rho(z)^8 + sink_omega), z = x / sqrt(mean(x^2) + eps).
    Differentiable (cached VJP of src/attention.py:75-82)."""
    if not 0 <= float(sink_omega) < float("inf"):
        raise ValueError("sink_omega must be finite and nonnegative")
    if not 0 < float(eps) < float("inf"):
        raise ValueError("eps must be finite and positive")
    x = _float_input(scores)
    if x.ndim == 0 or x.shape[-1] == 0:
        raise ValueError("AVN needs a nonempty feature axis")
    if x.numel() == 0:
        return x.clone()
    return _ASoftmax.apply(x, float(sink_omega), float(eps))


# ------------------------------------------------------------------------------------- AGO
class CayleyRotary(NamedTuple):
    """Precomputed Cayley rotation parameters (src/attention.py:94-107): unpack as (c, s) or
    use .c, .s, .matrix."""

    c: torch.Tensor
    s: torch.Tensor

    @property
    def matrix(self) -> torch.Tensor:
        """2x2 rotation blocks [[c, -s], [s, c]] of shape (..., 2, 2)."""
        row0 = torch.stack([self.c, -self.s], dim=-1)
        row1 = torch.stack([self.s, self.c], dim=-1)
        return torch.stack([row0, row1], dim=-2)


def build_cayley_rotary_matrix(dim: int, max_seq_len: int, freqs=None, base: float = 10000.0,
                               dtype: torch.dtype = torch.float32, device=None) -> CayleyRotary:
    """Cayley rotary tables (src/attention.py:155-204), built by the table kernel.

    The recurrence runs in fp32 (fp64 when dtype is float64) and the tables are cast to dtype.
    ``freqs`` are the Cayley parameters w_k in (0, 1] (shape (dim/2,)); the default is
    w_k = 1/(1 + alpha k)^2.  ``device`` defaults to the current HIP device.
    """
    if dim <= 0 or dim % 2 != 0:
        raise ValueError("dim must be a positive even integer")
    if max_seq_len <= 0:
        raise ValueError("max_seq_len must be a positive integer")
    pairs = dim // 2
    if freqs is not None and tuple(torch.as_tensor(freqs).shape) != (pairs,):
        raise ValueError(f"freqs must have shape ({pairs},), got {tuple(torch.as_tensor(freqs).shape)}")
    if device is None:
        if not torch.cuda.is_available():
            raise RuntimeError("the Cayley table kernel runs on the GPU, and no HIP device is visible")
        device = torch.device("cuda", torch.cuda.current_device())
    device = torch.device(device)
    calc = torch.float64 if dtype == torch.float64 else torch.float32
    f = None if freqs is None else torch.as_tensor(freqs, dtype=calc, device=device).contiguous()
    _lib.require_device(torch.empty(0, device=device))
    c = torch.empty((max_seq_len, pairs), dtype=calc, device=device)
    s = torch.empty_like(c)
    with torch.cuda.device(device):
        rc = _lib.lib().ago_build_tables(_lib.dtype_code(calc), dim, max_seq_len, _lib.ptr(f), float(base),
                                         _lib.ptr(c), _lib.ptr(s), _lib.stream_ptr(device))
    _lib.check(rc, "ago_build_tables")
    return CayleyRotary(c.to(dtype), s.to(dtype))


def _extract_cs(rotary_params):
    """(c, s) from a CayleyRotary, a (c, s) pair, a (..., 2, 2) matrix stack or a (..., 2)
    stack (src/attention.py:110-120)."""
    if isinstance(rotary_params, (tuple, list)) and len(rotary_params) >= 2:
        return rotary_params[0], rotary_params[1]
    if hasattr(rotary_params, "c") and hasattr(rotary_params, "s"):
        return rotary_params.c, rotary_params.s
    if hasattr(rotary_params, "shape"):
        if rotary_params.ndim >= 4 and tuple(rotary_params.shape[-2:]) == (2, 2):
            return rotary_params[..., 0, 0], rotary_params[..., 1, 0]
        if rotary_params.ndim >= 3 and rotary_params.shape[-1] == 2:
            return rotary_params[..., 0], rotary_params[..., 1]
    raise TypeError(f"Unsupported rotary parameters type: {type(rotary_params)}")


def _infer_seq_axis(shape, param_len):
    """Sequence-axis inference of src/attention.py:123-134 (_align_param)."""
    ndim = len(shape)
    if ndim == 2:
        return 0
    if ndim == 3:
        return 1
    if ndim == 4:
        if shape[1] <= param_len and shape[1] > shape[2]:
            return 1
        return 2 if shape[2] <= param_len else 1
    return ndim - 2


def _rotate_launch(x, c, s, seq_axis):
    dev = _lib.require_device(x, c, s)
    xc = x.contiguous()
    seq = xc.shape[seq_axis]
    outer = 1
    for n in xc.shape[:seq_axis]:
        outer *= n
    inner = 1
    for n in xc.shape[seq_axis + 1:-1]:
        inner *= n
    y = torch.empty_like(xc)
    cc, sc = c.contiguous(), s.contiguous()
    with torch.cuda.device(dev):
        rc = _lib.lib().ago_rotate(_lib.dtype_code(x.dtype), outer, seq, inner, xc.shape[-1], _lib.ptr(xc),
                                   _lib.ptr(y), _lib.dtype_code(cc.dtype), _lib.ptr(cc), _lib.ptr(sc),
                                   cc.shape[0], _lib.stream_ptr(dev))
    _lib.check(rc, "ago_rotate")
    return y


class _Rotate(torch.autograd.Function):
    """Pairwise rotation; its VJP rotates the cotangent by the transpose (angle negated)."""

    @staticmethod
    def forward(ctx, x, c, s, seq_axis):
        ctx.cfg = (c, s, seq_axis)
        return _rotate_launch(x, c, s, seq_axis)

    @staticmethod
    def backward(ctx, g):
        c, s, seq_axis = ctx.cfg
        return _rotate_launch(g.contiguous(), c, -s, seq_axis), None, None, None


def rotate_tensor(x: torch.Tensor, c: torch.Tensor, s: torch.Tensor, seq_axis: int) -> torch.Tensor:
    """Rotate (even, odd) feature pairs of x by the table rows of its sequence axis
    (src/attention.py:142-152); c and s are (>= L, D/2) tables."""
    if x.shape[-1] % 2 != 0:
        raise ValueError(f"Feature dimension must be even, got {x.shape[-1]}")
    c = _lib.table_2d(c, x.shape[-1])
    s = _lib.table_2d(s, x.shape[-1])
    if c.shape[0] < x.shape[seq_axis]:
        raise ValueError("rotary tables are shorter than the sequence")
    return _Rotate.apply(_float_input(x), c, s, seq_axis % x.ndim)


def _align_param(param, q_shape, seq_axis=None):
    """The first seq_len rows of a (positions, D/2) table, shaped to broadcast against the
    (..., D/2) feature pairs of a q_shape tensor: size seq_len on the sequence axis, D/2 last, 1
    elsewhere (src/attention.py:123-139; the model aligns its tables this way before
    _rotate_tensor, src/model.py:355-357).  A view of param, no copy."""
    q_shape = tuple(q_shape)
    ndim = len(q_shape)
    if seq_axis is None:
        seq_axis = _infer_seq_axis(q_shape, param.shape[0])
    seq_len = q_shape[seq_axis]
    shape = [1] * (ndim - 1) + [q_shape[-1] // 2]
    shape[seq_axis] = seq_len
    return param[:seq_len].reshape(shape)


def _rotate_tensor(x, c, s):
    """Rotate (even, odd) feature pairs of x by tables that broadcast against its (..., D/2)
    pairs (src/attention.py:142-152), as the model calls it on (B, H, T, D) q and k with tables
    from _align_param (src/model.py:263-264).  The tables may vary along one leading axis, the
    sequence axis, and are cast to x's dtype before the rotation, as the reference casts them.
    Runs ago_rotate; differentiable with respect to x."""
    x = _float_input(x)
    if x.ndim < 1 or x.shape[-1] % 2 != 0:
        raise ValueError(f"Feature dimension must be even, got {tuple(x.shape)}")
    pairs = x.shape[-1] // 2
    c = torch.as_tensor(c, device=x.device)
    s = torch.as_tensor(s, device=x.device)
    if c.shape != s.shape or c.ndim < 1 or c.ndim > x.ndim or c.shape[-1] != pairs:
        raise ValueError(f"rotary tables of shapes {tuple(c.shape)} and {tuple(s.shape)} do not broadcast "
                         f"against the feature pairs of {tuple(x.shape)}")
    lead = (1,) * (x.ndim - c.ndim) + tuple(c.shape[:-1])
    axes = [ax for ax, n in enumerate(lead) if n != 1]
    if len(axes) > 1 or any(n != 1 and n != x.shape[ax] for ax, n in enumerate(lead)):
        raise ValueError(f"rotary tables of shape {tuple(c.shape)} must vary along at most one axis of "
                         f"{tuple(x.shape)}, its sequence axis")
    if axes:
        seq_axis = axes[0]
        rows_c, rows_s = c.reshape(x.shape[seq_axis], pairs), s.reshape(x.shape[seq_axis], pairs)
    else:
        # one row for every position: the table is repeated along axis -2 (a copy of its rows)
        seq_axis = x.ndim - 2 if x.ndim >= 2 else 0
        n = x.shape[seq_axis] if x.ndim >= 2 else 1
        rows_c = c.reshape(1, pairs).expand(n, pairs).contiguous()
        rows_s = s.reshape(1, pairs).expand(n, pairs).contiguous()
        if x.ndim == 1:
            return _Rotate.apply(x.reshape(1, -1), rows_c, rows_s, 0).reshape(x.shape)
    return _Rotate.apply(x, rows_c, rows_s, seq_axis)


def apply_ago_rotations(q, k, rotary_params=None, seq_axis=None):
    """Apply AGO Cayley rotations to q and k (src/attention.py:207-240); returns (q_rot, k_rot)
    in the input dtypes."""
    if q.shape != k.shape:
        raise ValueError(f"q and k shapes must match, got {tuple(q.shape)} and {tuple(k.shape)}")
    dim = q.shape[-1]
    if dim % 2 != 0:
        raise ValueError(f"Feature dimension must be even, got {dim}")
    ndim = q.ndim
    if rotary_params is None:
        if seq_axis is None:
            seq_axis = 0 if ndim == 2 else 1 if ndim == 3 else (1 if q.shape[1] > q.shape[2] else 2)
        rotary_params = build_cayley_rotary_matrix(dim, q.shape[seq_axis], dtype=q.dtype, device=q.device)
    c_raw, s_raw = _extract_cs(rotary_params)
    c_raw = torch.as_tensor(c_raw, device=q.device)
    s_raw = torch.as_tensor(s_raw, device=q.device)
    if seq_axis is None:
        seq_axis = _infer_seq_axis(tuple(q.shape), c_raw.shape[0])
    return rotate_tensor(q, c_raw, s_raw, seq_axis), rotate_tensor(k, c_raw, s_raw, seq_axis)
