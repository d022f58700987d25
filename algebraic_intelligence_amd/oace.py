"""OACE loss head on MI355X: the call surface of src/kernels/pallas_oace.py and of
fused_oace_softmax_loss (src/model.py:180-240), tasmaikeni13/algebraic-intelligence.

fused_linear_oace(h, w_vocab, targets, eps_vocab=100.0, gamma=2.0, chunk_size=4096) is the mean
octic algebraic cross-entropy of the AVN-normalised A-Softmax of z = h @ w_vocab, differentiable
with the reference's analytical backward.  On the bf16/fp16 path the logits (rows, vocab) are
materialised only when they fit 256 MB (fp32, in the call's workspace, reused by the backward);
larger problems recompute them.  Every computation runs in the gfx950 kernels of libafa_hip.so
(include/afa.h).
"""
from __future__ import annotations

import math

import torch

from . import _lib

__all__ = ["fused_linear_oace", "fused_linear_oace_forward", "fused_linear_oace_backward",
           "fused_oace_softmax_loss"]

OACE_W_DV, OACE_W_VD = 0, 1
ROW_FIELDS = 8
FLAG_WT_READY = 0x10
FLAG_Z_READY = 0x20
FLAG_RECOMPUTE_Z = 0x40


def _check_scalars(chunk_size=None, gamma=None):
    if chunk_size is not None and (not isinstance(chunk_size, int) or chunk_size <= 0):
        raise ValueError("chunk_size must be a positive integer")
    if gamma is not None and not (0.0 < float(gamma) < math.inf):
        raise ValueError("gamma must be finite and strictly positive")


def _w_operand(w: torch.Tensor):
    """(tensor whose storage the kernel reads, layout, ldw) for a (d_model, vocab) weight: the
    output head as stored (row-major), or the transposed view of a row-major (vocab, d_model)
    tied embedding, read without a copy."""
    d, V = w.shape
    if w.stride(1) == 1 and w.stride(0) >= V:
        return w, OACE_W_DV, w.stride(0)
    if w.stride(0) == 1 and w.stride(1) >= d:
        return w, OACE_W_VD, w.stride(1)
    w = w.contiguous()
    return w, OACE_W_DV, V


def _rows2d(h: torch.Tensor, d: int) -> torch.Tensor:
    hf = h.reshape(-1, d)
    if hf.stride(1) != 1:
        hf = hf.contiguous()
    return hf


def fused_linear_oace_forward(h, w_vocab, targets, eps_vocab: float = 100.0, gamma: float = 2.0,
                              chunk_size: int = 4096, *, flags: int = 0):
    """Loss and cache (src/kernels/pallas_oace.py:59-209).  h (..., d_model), w_vocab
    (d_model, vocab), targets h.shape[:-1] integer class indices.  The loss is in the
    accumulation dtype (fp32; fp64 for fp64 inputs), as the reference's mean."""
    _check_scalars(chunk_size, gamma)
    dev = _lib.require_device(h, w_vocab)
    if w_vocab.dtype != h.dtype:
        raise TypeError(f"h and w_vocab must share a dtype, got {h.dtype} and {w_vocab.dtype}")
    if w_vocab.dim() != 2 or h.shape[-1] != w_vocab.shape[0]:
        raise ValueError(f"w_vocab must be (d_model, vocab) with d_model = {h.shape[-1]}, got {tuple(w_vocab.shape)}")
    targets = torch.as_tensor(targets, device=dev)
    if targets.shape != h.shape[:-1]:
        raise ValueError(f"targets must have shape {tuple(h.shape[:-1])}, got {tuple(targets.shape)}")
    d, V = w_vocab.shape
    hf = _rows2d(h, d)
    t = targets.reshape(-1).to(torch.int64).contiguous()
    wop, layout, ldw = _w_operand(w_vocab)
    acc = _lib.accum_dtype(h.dtype)
    N = hf.shape[0]
    loss = torch.empty((), dtype=acc, device=dev)
    rows = torch.empty((N, ROW_FIELDS), dtype=acc, device=dev)
    code = _lib.dtype_code(h.dtype)
    # the backward reuses this workspace (and the transposed weights the forward leaves in it)
    wsb = _lib.lib().oace_workspace_size(code, N, d, V, layout, flags)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.lib().oace_linear_fwd(code, N, d, V, hf.data_ptr(), hf.stride(0), wop.data_ptr(), layout, ldw,
                                        t.data_ptr(), float(eps_vocab), float(gamma), loss.data_ptr(), rows.data_ptr(),
                                        flags, ws.data_ptr(), wsb, _lib.stream_ptr(dev))
    _lib.check(rc, "oace_linear_fwd")
    cache = (hf, w_vocab, t, rows, float(gamma), chunk_size, tuple(h.shape), flags, ws, w_vocab._version,
             hf._version)
    return loss, cache


def fused_linear_oace_backward(cache, g):
    """(dh, dw_vocab, None) from the forward cache and the loss cotangent g
    (src/kernels/pallas_oace.py:212-269)."""
    hf, w_vocab, t, rows, gamma, _chunk, shape, flags, ws, w_version, h_version = cache
    dev = hf.device
    d, V = w_vocab.shape
    wop, layout, ldw = _w_operand(w_vocab)
    acc = rows.dtype
    gt = torch.as_tensor(g, dtype=acc, device=dev).reshape(())
    dh = torch.empty((hf.shape[0], d), dtype=hf.dtype, device=dev)
    if layout == OACE_W_DV:
        dw_store = torch.empty((d, ldw), dtype=w_vocab.dtype, device=dev)
        dw = dw_store[:, :V]
    else:
        dw_store = torch.empty((V, ldw), dtype=w_vocab.dtype, device=dev)
        dw = dw_store[:, :d].t()
    # the forward's transposed weights are still valid unless w_vocab was modified in place since,
    # and its logits unless h or w_vocab was
    w_same = w_vocab._version == w_version
    bflags = flags | (FLAG_WT_READY if w_same else 0) | (FLAG_Z_READY if w_same and hf._version == h_version else 0)
    with torch.cuda.device(dev):
        rc = _lib.lib().oace_linear_bwd(_lib.dtype_code(hf.dtype), hf.shape[0], d, V, hf.data_ptr(), hf.stride(0),
                                        wop.data_ptr(), layout, ldw, t.data_ptr(), float(gamma), rows.data_ptr(),
                                        gt.data_ptr(), dh.data_ptr(), dw_store.data_ptr(), bflags, ws.data_ptr(),
                                        ws.numel(), _lib.stream_ptr(dev))
    _lib.check(rc, "oace_linear_bwd")
    return dh.reshape(shape), dw, None


class _FusedLinearOACE(torch.autograd.Function):
    """Custom VJP of fused_linear_oace (src/kernels/pallas_oace.py:272-293)."""

    @staticmethod
    def forward(ctx, h, w_vocab, targets, eps_vocab, gamma, chunk_size):
        loss, cache = fused_linear_oace_forward(h.detach(), w_vocab.detach(), targets, eps_vocab, gamma, chunk_size)
        ctx.cache = cache
        return loss

    @staticmethod
    def backward(ctx, g):
        dh, dw, _ = fused_linear_oace_backward(ctx.cache, g)
        ctx.cache = None
        return dh, dw, None, None, None, None


def fused_linear_oace(h, w_vocab, targets, eps_vocab: float = 100.0, gamma: float = 2.0,
                      chunk_size: int = 4096) -> torch.Tensor:
    """Fused Linear + OACE loss with zero (rows, vocab) allocation on the bf16/fp16 path
    (src/kernels/pallas_oace.py:272-293).  chunk_size is validated and does not change the
    result (the reference's chunking is a memory bound; the sums are additive)."""
    return _FusedLinearOACE.apply(h, w_vocab, targets, eps_vocab, gamma, chunk_size)


class _FusedOACESoftmaxLoss(torch.autograd.Function):
    """fused_oace_softmax_loss with its analytical VJP (src/model.py:180-240)."""

    @staticmethod
    def forward(ctx, logits, targets, eps, gamma):
        dev = _lib.require_device(logits)
        z = logits.detach().contiguous()
        V = z.shape[-1]
        z2 = z.reshape(-1, V)
        t = torch.as_tensor(targets, device=dev).reshape(-1).to(torch.int64).contiguous()
        if t.numel() != z2.shape[0]:
            raise ValueError(f"targets must have shape {tuple(logits.shape[:-1])}")
        acc = _lib.accum_dtype(z.dtype)
        loss = torch.empty((), dtype=acc, device=dev)
        rows = torch.empty((z2.shape[0], ROW_FIELDS), dtype=acc, device=dev)
        with torch.cuda.device(dev):
            rc = _lib.lib().oace_softmax_loss_fwd(_lib.dtype_code(z.dtype), z2.shape[0], V, z2.data_ptr(), t.data_ptr(),
                                                  float(eps), float(gamma), loss.data_ptr(), rows.data_ptr(),
                                                  _lib.stream_ptr(dev))
        _lib.check(rc, "oace_softmax_loss_fwd")
        ctx.save_for_backward(z, t, rows)
        ctx.gamma = float(gamma)
        return loss

    @staticmethod
    def backward(ctx, g):
        z, t, rows = ctx.saved_tensors
        dev = z.device
        gt = torch.as_tensor(g, dtype=rows.dtype, device=dev).reshape(())
        dz = torch.empty_like(z)
        V = z.shape[-1]
        with torch.cuda.device(dev):
            rc = _lib.lib().oace_softmax_loss_bwd(_lib.dtype_code(z.dtype), t.numel(), V, z.data_ptr(), t.data_ptr(),
                                                  ctx.gamma, rows.data_ptr(), gt.data_ptr(), dz.data_ptr(),
                                                  _lib.stream_ptr(dev))
        _lib.check(rc, "oace_softmax_loss_bwd")
        return dz, None, None, None


def fused_oace_softmax_loss(logits, targets, eps: float = 100.0, gamma: float = 2.0) -> torch.Tensor:
    """Mean OACE loss of the AVN-normalised A-Softmax over the last axis of logits
    (src/model.py:229-240).  Evaluated in fp32 (fp64 for fp64 logits); the reference evaluates
    in the logits dtype."""
    _check_scalars(gamma=gamma)
    if not (0.0 <= float(eps) < math.inf):
        raise ValueError("eps must be finite and nonnegative")
    if not isinstance(logits, torch.Tensor) or not logits.is_floating_point():
        raise TypeError("expected a floating point tensor of logits")
    if logits.dim() == 0 or logits.shape[-1] == 0:
        raise ValueError("logits must have a non-empty last axis")
    return _FusedOACESoftmaxLoss.apply(logits, targets, eps, gamma)
