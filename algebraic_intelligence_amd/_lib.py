"""ctypes binding of libafa_hip.so (C ABI declared in include/afa.h).

The library is required: there is no CPU implementation behind these entry points, and a
missing or stale build raises instead of falling back.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "_build", "libafa_hip.so")

AFA_F32, AFA_BF16, AFA_F16, AFA_F64 = 0, 1, 2, 3
FLAG_EXACT_TAIL, FLAG_GENERIC, FLAG_EXACT_REF, FLAG_SIMPLE_SCHEDULE = 0x1, 0x2, 0x4, 0x8
FLAG_ACCUMULATE, FLAG_PARTIAL = 0x100, 0x200

(OK, ERR_NULL, ERR_DTYPE, ERR_SHAPE, ERR_HEAD_DIM, ERR_SINK, ERR_VALID_LEN, ERR_EPS, ERR_ROTARY,
 ERR_ALIGN, ERR_WORKSPACE, ERR_UNSUPPORTED, ERR_GAMMA, ERR_SCRATCH_LIMIT) = range(14)
NOALLOC_SCRATCH_BYTES = 64 << 20
ERR_HIP = 100

# Every function include/afa.h declares, with its ctypes signature.
_i64, _vp, _dbl, _int, _uint, _sz = (ctypes.c_int64, ctypes.c_void_p, ctypes.c_double, ctypes.c_int,
                                     ctypes.c_uint, ctypes.c_size_t)
SIGNATURES = {
    "afa_status_string": (ctypes.c_char_p, [_int]),
    "afa_last_hip_error": (_int, []),
    "afa_version": (_int, []),
    "afa_fwd_workspace_size": (_sz, [_int, _i64, _i64, _i64, _i64, _int]),
    "afa_fwd": (_int, [_int, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                       _dbl, _int, _i64, _uint, _vp, _sz, _vp]),
    "afa_fwd_noalloc": (_int, [_int, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                               _dbl, _int, _i64, _uint, _vp]),
    "afa_ring_finish": (_int, [_int, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _dbl, _vp, _vp, _vp]),
    "afa_bwd_workspace_size": (_sz, [_int, _i64, _i64, _i64, _i64, _int]),
    "afa_bwd": (_int, [_int, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                       _vp, _vp, _i64, _dbl, _int, _i64, _uint, _vp, _sz, _vp]),
    "asoftmax_fwd": (_int, [_int, _i64, _i64, _vp, _vp, _dbl, _dbl, _vp]),
    "asoftmax_bwd": (_int, [_int, _i64, _i64, _vp, _vp, _vp, _dbl, _dbl, _vp]),
    "octic_fwd": (_int, [_int, _i64, _vp, _vp, _vp]),
    "octic_fwd_r": (_int, [_int, _i64, _vp, _vp, _vp, _vp]),
    "octic_bwd": (_int, [_int, _i64, _vp, _vp, _vp, _vp]),
    "ago_build_tables": (_int, [_int, _i64, _i64, _vp, _dbl, _vp, _vp, _vp]),
    "ago_rotate": (_int, [_int, _i64, _i64, _i64, _i64, _vp, _vp, _int, _vp, _vp, _i64, _vp]),
    "oace_workspace_size": (_sz, [_int, _i64, _i64, _i64, _int, _uint]),
    "oace_linear_fwd": (_int, [_int, _i64, _i64, _i64, _vp, _i64, _vp, _int, _i64, _vp, _dbl, _dbl, _vp, _vp,
                               _uint, _vp, _sz, _vp]),
    "oace_linear_bwd": (_int, [_int, _i64, _i64, _i64, _vp, _i64, _vp, _int, _i64, _vp, _dbl, _vp, _vp, _vp, _vp,
                               _uint, _vp, _sz, _vp]),
    "oace_softmax_loss_fwd": (_int, [_int, _i64, _i64, _vp, _vp, _dbl, _dbl, _vp, _vp, _vp]),
    "oace_softmax_loss_bwd": (_int, [_int, _i64, _i64, _vp, _vp, _dbl, _vp, _vp, _vp, _vp]),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load libafa_hip.so (built by algebraic_intelligence_amd.build / __graft_entry__.build)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build it with `python -m algebraic_intelligence_amd.build`"
                    )
                handle = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


_TORCH_DT = {torch.float32: AFA_F32, torch.bfloat16: AFA_BF16, torch.float16: AFA_F16,
             torch.float64: AFA_F64}


def dtype_code(t: torch.dtype) -> int:
    try:
        return _TORCH_DT[t]
    except KeyError:
        raise TypeError(f"expected a floating point array (float32, bfloat16, float16 or float64), got {t}")


def accum_dtype(t: torch.dtype) -> torch.dtype:
    return torch.float64 if t == torch.float64 else torch.float32


def require_device(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "the AFA kernels run on the GPU: pass tensors on a HIP device (torch 'cuda'), "
                f"got a tensor on {t.device}"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"all tensors must be on one device, got {dev} and {t.device}")
    return dev


def stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t):
    return None if t is None else t.data_ptr()


def check(rc: int, what: str) -> None:
    """Raise the reference's exception family for a non-zero afa_status."""
    if rc == OK:
        return
    msg = lib().afa_status_string(rc).decode()
    if rc == ERR_HIP:
        raise RuntimeError(f"{what}: {msg} (hipError {lib().afa_last_hip_error()})")
    if rc == ERR_DTYPE:
        raise TypeError(f"{what}: {msg}")
    if rc in (ERR_UNSUPPORTED, ERR_ALIGN):
        raise NotImplementedError(f"{what}: {msg}")
    raise ValueError(f"{what}: {msg}")


def table_2d(t: torch.Tensor, head_dim: int) -> torch.Tensor:
    """A (positions, head_dim/2) view of a Cayley table, broadcast axes of size 1 dropped.

    The reference aligns the tables to the sequence axis and the pair axis and fails when their
    shape does not fit the head dimension (src/attention.py:110-139); a table built for another
    head dimension must not be reinterpreted as more rows here."""
    if head_dim % 2 != 0:
        raise ValueError(f"rotary tables need an even head dimension, got {head_dim}")
    lead = [d for d in t.shape[:-1] if d != 1] if t.ndim >= 1 else []
    if t.ndim == 0 or len(lead) > 1 or t.shape[-1] != head_dim // 2:
        raise ValueError(
            f"rotary tables must have shape (positions, head_dim/2) = (L, {head_dim // 2}) up to axes of "
            f"size 1, got {tuple(t.shape)}")
    return t.reshape(lead[0] if lead else 1, head_dim // 2)
