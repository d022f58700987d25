"""Algebraic FlashAttention on MI355X: the call surface of src/kernels/pallas_afa.py.

Same names, argument meanings, defaults and ValueError checks as the reference module
(tasmaikeni13/algebraic-intelligence, src/kernels/pallas_afa.py), on torch tensors that live on
a HIP device.  Every function launches the gfx950 kernels of libafa_hip.so through the C ABI in
include/afa.h; there is no CPU implementation behind them.

Beyond the reference signatures, the forward entry points take ``rotary_params`` (a
CayleyRotary or a (c, s) pair of (>= L, D/2) tables): q and k are then rotated inside the
kernel at tile load, which fuses the model's ``_rotate_tensor`` calls (src/model.py:262-264).

``block_q`` / ``block_k`` are validated exactly as the reference does, but they do not change
the computation: the kernels pick their own tiles, and the additive accumulation makes the
result independent of the tiling (src/kernels/pallas_afa.py tests, test_additive_tile_associativity).
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple, Union

import torch

from . import _lib
from ._lib import table_2d
from .attention import _vmu_octic_kernel  # noqa: F401  (src/kernels/pallas_afa.py:32-49 defines it here)

__all__ = [
    "pallas_afa_forward", "tiled_afa_forward", "exact_afa_reference", "exact_afa_with_denominator",
    "tiled_afa_backward", "pallas_afa", "algebraic_flash_attention", "distributed_ring_afa",
    "sharded_pallas_afa",
]


def _finite_nonneg(x) -> bool:
    return 0.0 <= float(x) < float("inf")


def _rotary_tables(rotary_params, q: torch.Tensor):
    """(c, s) device tables in the kernel's table type: fp32, or fp64 for fp64 inputs."""
    if rotary_params is None:
        return None, None, 0
    if isinstance(rotary_params, (tuple, list)) and len(rotary_params) >= 2:
        c, s = rotary_params[0], rotary_params[1]
    elif hasattr(rotary_params, "c") and hasattr(rotary_params, "s"):
        c, s = rotary_params.c, rotary_params.s
    else:
        raise TypeError(f"Unsupported rotary parameters type: {type(rotary_params)}")
    tdt = torch.float64 if q.dtype == torch.float64 else torch.float32
    D = q.shape[-1]
    c = table_2d(torch.as_tensor(c, device=q.device), D)
    s = table_2d(torch.as_tensor(s, device=q.device), D)
    if c.shape != s.shape:
        raise ValueError(f"rotary tables must match, got {tuple(c.shape)} and {tuple(s.shape)}")
    return c.to(tdt).contiguous(), s.to(tdt).contiguous(), c.shape[0]


def _strides(*ts):
    """12 element strides (b, h, l per tensor); head_dim must be contiguous."""
    out = []
    for t in ts:
        out.extend(t.stride()[:3])
    return (ctypes.c_int64 * 12)(*out)


def _prep(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def _launch_fwd(q, k, v, sink_omega, causal, valid_seq_len, rotary_params, flags,
                want_denominator):
    c, s, rot_len = _rotary_tables(rotary_params, q)  # shape checks first, as the reference's
    dev = _lib.require_device(q, k, v)
    dt = _lib.dtype_code(q.dtype)
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError(f"q, k and v must share a dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    q, k, v = _prep(q), _prep(k), _prep(v)
    B, H, L, D = q.shape
    out = torch.empty((B, H, L, D), dtype=q.dtype, device=dev)
    den = torch.empty((B, H, L, 1), dtype=_lib.accum_dtype(q.dtype), device=dev) if want_denominator else None
    with torch.cuda.device(dev):
        # the workspace comes from torch's caching allocator, so the library allocates nothing
        ws_bytes = _lib.lib().afa_fwd_workspace_size(dt, B, H, L, D, int(c is not None))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
        rc = _lib.lib().afa_fwd(
            dt, B, H, L, D, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _strides(q, k, v, out),
            _lib.ptr(out), _lib.ptr(den), _lib.ptr(c), _lib.ptr(s), rot_len, float(sink_omega),
            int(bool(causal)), 0 if valid_seq_len is None else int(valid_seq_len), flags,
            _lib.ptr(ws), ws_bytes, _lib.stream_ptr(dev))
    _lib.check(rc, "afa_fwd")
    return out, den


def afa_kernel(*refs, **config):
    """The reference's tile body (src/kernels/pallas_afa.py:52-151) takes Pallas-TPU memory refs
    and runs only inside pallas_call.  Here the tile loop is the HIP kernels of libafa_hip.so
    (afa_fwd_d64_kernel, afa_fwd_pipe_kernel, afa_fwd_mfma_kernel, afa_fwd_f32_kernel), which
    pallas_afa_forward launches; this name lets modules that import it load, and calling it
    raises."""
    raise NotImplementedError(
        "afa_kernel is the Pallas-TPU tile body; on MI355X the tile loop runs inside libafa_hip.so: "
        "call pallas_afa_forward (or tiled_afa_forward) with the whole q, k, v")


def pallas_afa_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    sink_omega: float = 0.5,
    causal: bool = False,
    block_q: int = 128,
    block_k: int = 128,
    valid_seq_len: Optional[int] = None,
    interpret: Optional[bool] = None,
    return_denominator: bool = False,
    *,
    rotary_params=None,
) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """Fused AFA forward (src/kernels/pallas_afa.py:154-264).

    Returns out (q.dtype) or (out, d) with d = sum_j rho(s_ij)^8 + sink_omega of shape
    (B, H, L, 1) in fp32 (fp64 for fp64 inputs).  ``interpret`` is accepted for signature
    compatibility; the reference uses it to pick the Pallas interpreter off-TPU, and here the
    HIP kernel runs either way.
    """
    del interpret
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must all have shape (batch, heads, sequence, dimension)")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q, k, and v shapes must match, got {tuple(q.shape)}, {tuple(k.shape)}, and {tuple(v.shape)}")
    if not _finite_nonneg(sink_omega):
        raise ValueError("sink_omega must be finite and nonnegative")
    if block_q <= 0 or block_k <= 0:
        raise ValueError("block_q and block_k must be positive")
    batch_size, num_heads, seq_len, head_dim = q.shape
    if head_dim <= 0:
        raise ValueError("head dimension must be positive")
    if head_dim > 128 and head_dim % 128 != 0:
        raise ValueError("head dimensions above 128 must be divisible by 128")
    if seq_len % block_q != 0 or seq_len % block_k != 0:
        raise ValueError(
            f"seq_len ({seq_len}) must be divisible by block_q ({block_q}) and block_k ({block_k})"
        )
    if valid_seq_len is not None and not 0 < valid_seq_len <= seq_len:
        raise ValueError("valid_seq_len must be in [1, seq_len]")
    out, den = _launch_fwd(q, k, v, sink_omega, causal, valid_seq_len, rotary_params, 0,
                           return_denominator)
    return (out, den) if return_denominator else out


def tiled_afa_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    sink_omega: float = 0.5,
    causal: bool = False,
    block_q: int = 128,
    block_k: int = 128,
    valid_seq_len: Optional[int] = None,
    return_denominator: bool = False,
    *,
    rotary_params=None,
) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """Tiled additive AFA (src/kernels/pallas_afa.py:330-406): the same function as
    pallas_afa_forward, with the reference's own argument checks."""
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, and v must have the same four-dimensional shape")
    if not _finite_nonneg(sink_omega):
        raise ValueError("sink_omega must be finite and nonnegative")
    if block_q <= 0 or block_k <= 0:
        raise ValueError("block_q and block_k must be positive")
    seq_len = q.shape[2]
    if seq_len % block_q != 0 or seq_len % block_k != 0:
        raise ValueError("sequence length must be divisible by both tile dimensions")
    if valid_seq_len is not None and not 0 < valid_seq_len <= seq_len:
        raise ValueError("valid_seq_len must be in [1, seq_len]")
    out, den = _launch_fwd(q, k, v, sink_omega, causal, valid_seq_len, rotary_params, 0,
                           return_denominator)
    return (out, den) if return_denominator else out


def exact_afa_reference(q, k, v, sink_omega: float = 0.5, causal: bool = False) -> torch.Tensor:
    """Untiled reference contract (src/kernels/pallas_afa.py:267-297): q * scale rounded to
    q.dtype before the dot, row sum of P cast to v.dtype, out = O * (1 / (D + sink)).

    For bf16/fp16 inputs every op is rounded to the input dtype as the reference's JAX program
    types it: the scale itself, the scores, each step of rho^8, the P V product, the row sum,
    D + sink, its reciprocal and the product.  The summation orders, which the program leaves
    to XLA, are fixed by the kernel (8 fma chains per score added pairwise, key order for the
    P V product and the row sum).
    """
    return exact_afa_with_denominator(q, k, v, sink_omega, causal)[0]


def exact_afa_with_denominator(q, k, v, sink_omega: float = 0.5, causal: bool = False):
    """(out, d_total) of the untiled contract (src/kernels/pallas_afa.py:300-327); d_total is
    returned in v.dtype, as the reference sums P after casting it to v.dtype."""
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, and v must have the same four-dimensional shape")
    if not _finite_nonneg(sink_omega):
        raise ValueError("sink_omega must be finite and nonnegative")
    out, den = _launch_fwd(q, k, v, sink_omega, causal, None, None, _lib.FLAG_EXACT_REF, True)
    return out, den.to(v.dtype)


def tiled_afa_backward(
    q, k, v, out, d_total, g_out, sink_omega: float = 0.5, causal: bool = False,
    block_q: int = 128, block_k: int = 128, valid_seq_len: Optional[int] = None, *,
    rotary_params=None,
):
    """Analytical AFA backward (src/kernels/pallas_afa.py:409-522): (dq, dk, dv) in the input
    dtypes.  With ``rotary_params`` the forward rotated q and k in-kernel and dq, dk are with
    respect to the unrotated inputs."""
    del block_q, block_k
    dev = _lib.require_device(q, k, v, out, d_total, g_out)
    dt = _lib.dtype_code(q.dtype)
    B, H, L, D = q.shape
    q, k, v, out, g_out = (t.contiguous() for t in (q, k, v, out, g_out))
    d_total = d_total.to(_lib.accum_dtype(q.dtype)).contiguous()
    dq, dk, dv = (torch.empty_like(t) for t in (q, k, v))
    c, s, rot_len = _rotary_tables(rotary_params, q)
    ws_bytes = _lib.lib().afa_bwd_workspace_size(dt, B, H, L, D, int(c is not None))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.lib().afa_bwd(
            dt, B, H, L, D, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(d_total),
            _lib.ptr(g_out), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(c), _lib.ptr(s),
            rot_len, float(sink_omega), int(bool(causal)),
            0 if valid_seq_len is None else int(valid_seq_len), 0, _lib.ptr(ws), ws_bytes,
            _lib.stream_ptr(dev))
    _lib.check(rc, "afa_bwd")
    return dq, dk, dv


class _PallasAFA(torch.autograd.Function):
    """Custom VJP of pallas_afa (src/kernels/pallas_afa.py:532-615): the forward keeps
    (q, k, v, out, d_total) and the backward is the analytical tiled_afa_backward."""

    @staticmethod
    def forward(ctx, q, k, v, sink_omega, causal, valid_seq_len, rotary_params):
        out, den = _launch_fwd(q, k, v, sink_omega, causal, valid_seq_len, rotary_params, 0, True)
        ctx.save_for_backward(q, k, v, out, den)
        ctx.cfg = (sink_omega, causal, valid_seq_len, rotary_params)
        return out

    @staticmethod
    def backward(ctx, g):
        q, k, v, out, den = ctx.saved_tensors
        sink_omega, causal, valid_seq_len, rotary_params = ctx.cfg
        dq, dk, dv = tiled_afa_backward(q, k, v, out, den, g, sink_omega, causal,
                                        valid_seq_len=valid_seq_len, rotary_params=rotary_params)
        return dq, dk, dv, None, None, None, None


def pallas_afa(
    q, k, v, sink_omega: float = 0.5, causal: bool = False, block_q: int = 128,
    block_k: int = 128, valid_seq_len: Optional[int] = None, *, rotary_params=None,
) -> torch.Tensor:
    """Differentiable fused AFA (src/kernels/pallas_afa.py:579-615)."""
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, and v must have the same four-dimensional shape")
    if not _finite_nonneg(sink_omega):
        raise ValueError("sink_omega must be finite and nonnegative")
    if block_q <= 0 or block_k <= 0:
        raise ValueError("block_q and block_k must be positive")
    seq_len = q.shape[2]
    if seq_len % block_q != 0 or seq_len % block_k != 0:
        raise ValueError(
            f"seq_len ({seq_len}) must be divisible by block_q ({block_q}) and block_k ({block_k})"
        )
    if valid_seq_len is not None and not 0 < valid_seq_len <= seq_len:
        raise ValueError("valid_seq_len must be in [1, seq_len]")
    return _PallasAFA.apply(q, k, v, float(sink_omega), bool(causal), valid_seq_len, rotary_params)


def algebraic_flash_attention(
    q, k, v, sink_omega: float = 0.5, causal: bool = False, block_q: int = 128,
    block_k: int = 128, *, rotary_params=None,
) -> torch.Tensor:
    """Unified entry point for any sequence length (src/kernels/pallas_afa.py:695-739).

    The reference pads L up to lcm(block_q, block_k), masks the padded keys with
    valid_seq_len and slices the padded queries off.  The HIP kernels take any L directly and
    give the same values without the padded copies: padded keys carry zero weight and padded
    queries are never stored.
    """
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, and v must have the same four-dimensional shape")
    if block_q <= 0 or block_k <= 0:
        raise ValueError("block_q and block_k must be positive")
    if not _finite_nonneg(sink_omega):
        raise ValueError("sink_omega must be finite and nonnegative")
    if q.shape[-1] > 128 and q.shape[-1] % 128 != 0:
        raise ValueError("head dimensions above 128 must be divisible by 128")
    return _PallasAFA.apply(q, k, v, float(sink_omega), bool(causal), None, rotary_params)


def _device_major(t: torch.Tensor, n: int) -> torch.Tensor:
    """(B, H, n * S, D) contiguous -> the (n, B * H, S, D) view whose batch axis is the shard."""
    B, H, L, D = t.shape
    S = L // n
    return t.as_strided((n, B * H, S, D), (S * D, L * D, D, 1), t.storage_offset())


def _ring_forward(q, k, v, sink_omega, causal, n, want_total):
    """The ring's hops and final division (see distributed_ring_afa); returns (out, d_total) with
    d_total = row sums + sink_omega as (B, H, L, 1) in the accumulation type when asked for."""
    dev = _lib.require_device(q, k, v)
    dt = _lib.dtype_code(q.dtype)
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError(f"q, k and v must share a dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    B, H, L, D = q.shape
    S = L // n
    qd, kd, vd = (_device_major(t.contiguous(), n) for t in (q, k, v))
    acc = torch.empty((B, H, L, D), dtype=_lib.accum_dtype(q.dtype), device=dev)
    den = torch.empty((n, B * H, S), dtype=acc.dtype, device=dev)
    out = torch.empty((B, H, L, D), dtype=q.dtype, device=dev)
    total = torch.empty((B, H, L, 1), dtype=acc.dtype, device=dev) if want_total else None
    accd = _device_major(acc, n)
    L_ = _lib.lib()
    with torch.cuda.device(dev):
        stream = _lib.stream_ptr(dev)
        ws_bytes = max(L_.afa_fwd_workspace_size(dt, m, B * H, S, D, 0) for m in range(1, n + 1))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
        if causal or n == 1:
            kr, vr = kd, vd
        else:
            # non-causal hops wrap round the ring (device d reads shard (d - hop) mod n): with the
            # shard sequence stored twice, shard d - hop + n sits at index d - hop + n, and every
            # hop is one call over all devices
            kr, vr = torch.cat((kd, kd)), torch.cat((vd, vd))
        # the hops' views differ only in their first shard: the strides are shared and the base
        # pointers advance by one shard per device, so each hop is one C call
        strides = _strides(qd, kr, vr, accd)
        qp, kp, vp, ap, dp, wp = (t.data_ptr() for t in (qd, kr, vr, accd, den, ws if ws is not None else den))
        esz = q.element_size()
        shard, kshard = S * D * esz, kr.stride(0) * esz
        ashard, dshard = S * D * acc.element_size(), B * H * S * den.element_size()
        fwd = L_.afa_fwd

        def hop_call(d0, d1, kv0, diag, flags=_lib.FLAG_ACCUMULATE):
            # devices d0 .. d1-1 against key/value shards kv0 .. kv0 + d1 - d0 - 1
            rc = fwd(dt, d1 - d0, B * H, S, D, qp + d0 * shard, kp + kv0 * kshard, vp + kv0 * kshard, strides,
                     ap + d0 * ashard, dp + d0 * dshard, None, None, 0, 0.0, int(diag), 0, flags,
                     wp if ws_bytes else None, ws_bytes, stream)
            _lib.check(rc, "afa_fwd")

        hop_call(0, n, 0, causal, _lib.FLAG_PARTIAL)  # every device against its own shard
        for hop in range(1, n):
            if causal:
                hop_call(hop, n, 0, False)  # devices d >= hop read the earlier shard d - hop
            else:
                hop_call(0, n, n - hop, False)  # device d reads shard d - hop + n of the doubled run
        # the finish runs over the same device-major views; d_total of (device, bh, row) sits at
        # bh * L + device * S + row of the (B, H, L) array
        st = (ctypes.c_int64 * 9)(S * D, L * D, D, S * D, L * D, D, S, L, 1)
        rc = L_.afa_ring_finish(dt, n, B * H, S, D, _lib.ptr(acc), _lib.ptr(den), st, float(sink_omega),
                                _lib.ptr(out), _lib.ptr(total), stream)
    _lib.check(rc, "afa_ring_finish")
    return out, total


class _RingAFA(torch.autograd.Function):
    """distributed_ring_afa with a gradient.  The ring only re-associates the sums of the full
    attention, so its gradient is the full attention's: the analytical tiled_afa_backward on the
    ring's output and total denominator (src/kernels/pallas_afa.py:409-522)."""

    @staticmethod
    def forward(ctx, q, k, v, sink_omega, causal, n):
        out, total = _ring_forward(q, k, v, sink_omega, causal, n, True)
        ctx.save_for_backward(q, k, v, out, total)
        ctx.cfg = (sink_omega, causal)
        return out

    @staticmethod
    def backward(ctx, g):
        q, k, v, out, total = ctx.saved_tensors
        sink_omega, causal = ctx.cfg
        dq, dk, dv = tiled_afa_backward(q, k, v, out, total, g, sink_omega, causal)
        return dq, dk, dv, None, None, None


def distributed_ring_afa(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    sink_omega: float = 0.5,
    causal: bool = False,
    axis_name: str = "devices",
    num_devices: int = 16,
) -> torch.Tensor:
    """Ring AFA over ``num_devices`` sequence shards (src/kernels/pallas_afa.py:618-662).

    The reference runs once per device inside a mesh: device d holds query shard d, the key and
    value shards travel round the ring, and hop h adds rho(s)^8-weighted sums of shard
    (d - h) mod n to fp32 accumulators; out = o / (d + sink_omega) after n hops.  Here, on one
    GPU, q, k and v are the whole (B, H, L, D) arrays, L = num_devices * shard_len, device d's
    shard being rows [d * shard_len, (d + 1) * shard_len), and the result is the devices' outputs
    side by side.  A hop is one afa_fwd call over every device's pair at once: the devices are the
    batch axis of strided views (non-causal: over the key/value shards stored twice in a row, so
    that the shards a hop wraps round to follow on), and no shard moves between hops.  Hop 0
    stores the sums (AFA_FLAG_PARTIAL, so the accumulators need no clearing), every later hop adds
    to them (AFA_FLAG_ACCUMULATE).  causal: hop 0 pairs each shard with itself under the causal
    mask, and at hop h > 0 only devices d >= h hold an earlier shard; the later ones (masked whole
    in the reference) are not computed.  The accumulators are fp32 (fp64 for fp64 inputs); the
    final division is afa_ring_finish.  Differentiable, as the reference's JAX function is: the
    gradient is the full attention's (tiled_afa_backward on the ring's output and denominator).
    ``axis_name`` is accepted for signature compatibility.
    """
    del axis_name
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("q, k, and v must all have shape (batch, heads, sequence, dimension)")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q, k, and v shapes must match, got {tuple(q.shape)}, {tuple(k.shape)}, and {tuple(v.shape)}")
    if not _finite_nonneg(sink_omega):
        raise ValueError("sink_omega must be finite and nonnegative")
    n = int(num_devices)
    L = q.shape[2]
    if n <= 0 or L % n != 0:
        raise ValueError(f"seq_len ({L}) must split into num_devices ({num_devices}) equal shards")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        return _RingAFA.apply(q, k, v, float(sink_omega), bool(causal), n)
    return _ring_forward(q, k, v, float(sink_omega), bool(causal), n, False)[0]


def _mesh_axes(mesh) -> dict:
    """Axis sizes of a mesh: None (one device), a mapping {axis: size}, or an object with a
    ``shape`` mapping (a JAX Mesh exposes its axis sizes that way)."""
    if mesh is None:
        return {}
    shape = mesh if isinstance(mesh, dict) else getattr(mesh, "shape", None)
    if not isinstance(shape, dict):
        raise TypeError(f"mesh must be None, a mapping of axis sizes, or have a .shape mapping, got {type(mesh)}")
    return {str(k): int(v) for k, v in shape.items()}


def sharded_pallas_afa(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    mesh=None,
    sink_omega: float = 0.5,
    causal: bool = False,
    block_q: int = 128,
    block_k: int = 128,
) -> torch.Tensor:
    """Batch over the mesh's 'data' axis, heads over 'fsdp' (src/kernels/pallas_afa.py:665-692).

    The reference places q, k and v with NamedSharding(mesh, P("data", "fsdp", None, None)) and
    runs the differentiable pallas_afa on every shard.  (b, h) pairs are independent, so the
    result is pallas_afa of the whole arrays; on this one GPU every shard lives on the same device
    and one call computes them all.  The shard shapes are checked as the placement would: batch
    divisible by the 'data' axis size and heads by 'fsdp'.
    """
    axes = _mesh_axes(mesh)
    if q.ndim == 4:
        B, H = q.shape[0], q.shape[1]
        if B % axes.get("data", 1) != 0:
            raise ValueError(f"batch ({B}) must be divisible by the 'data' axis size ({axes['data']})")
        if H % axes.get("fsdp", 1) != 0:
            raise ValueError(f"heads ({H}) must be divisible by the 'fsdp' axis size ({axes['fsdp']})")
    return pallas_afa(q, k, v, sink_omega=sink_omega, causal=causal, block_q=block_q, block_k=block_k)


def afa_flops(batch: int, heads: int, seq_len: int, head_dim: int, causal: bool) -> int:
    """Algorithmic FLOPs of one forward: 4 B H D N_pairs (QK^T + PV over unmasked pairs),
    N_pairs = L^2 or L(L+1)/2 (scripts/run_phase6_tpu.py:236 for the non-causal form)."""
    pairs = seq_len * (seq_len + 1) // 2 if causal else seq_len * seq_len
    return 4 * batch * heads * head_dim * pairs
