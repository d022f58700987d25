"""ctypes wrapper of the C contract oracle (oracle/afa_contract.c).

TEST INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke(), bench.py cpu_baseline).

Arrays are numpy: float32 / float64 as themselves, bf16 and fp16 as uint16 bit patterns.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle_afa.so")
_lib = None

DT_F32, DT_BF16, DT_F16, DT_F64 = 0, 1, 2, 3
_NP = {DT_F32: np.float32, DT_BF16: np.uint16, DT_F16: np.uint16, DT_F64: np.float64}


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            from . import build_oracle
            build_oracle.build()
        L = ctypes.CDLL(_LIB_PATH)
        i64, vp, dbl, ci = ctypes.c_int64, ctypes.c_void_p, ctypes.c_double, ctypes.c_int
        L.oracle_afa_fwd.argtypes = [ci, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, dbl, ci,
                                     i64, i64, i64, ci]
        L.oracle_afa_fwd.restype = ci
        L.oracle_afa_bwd.argtypes = [ci, i64, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                     ci, i64, ci]
        L.oracle_afa_bwd.restype = ci
        L.oracle_rho8_f32.argtypes = [vp, vp, i64]
        L.oracle_afa_exact_ref.argtypes = [ci, i64, i64, i64, i64, vp, vp, vp, vp, vp, dbl, ci, ci]
        L.oracle_afa_exact_ref.restype = ci
        L.oracle_rho8_step.argtypes = [vp, vp, i64, ci]
        L.oracle_bf16_round.argtypes = [vp, vp, i64]
        L.oracle_f16_round.argtypes = [vp, vp, i64]
        L.oracle_max_threads.restype = ci
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=_NP[dt])


def bf16_bits(x):
    """float array -> bf16 bit patterns (uint16), round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_bf16_round(_ptr(x), _ptr(out), x.size)
    return out


def f16_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f16_round(_ptr(x), _ptr(out), x.size)
    return out


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_to_f32(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def to_f32(a, dt):
    if dt == DT_BF16:
        return bf16_to_f32(a)
    if dt == DT_F16:
        return f16_to_f32(a)
    return np.asarray(a, dtype=np.float64 if dt == DT_F64 else np.float32)


def rho8_f32(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().oracle_rho8_f32(_ptr(x), _ptr(y), x.size)
    return y


def afa_fwd(q, k, v, dtype, sink_omega=0.5, causal=False, valid_len=None, rotary=None,
            block_q=None, block_k=None, nthreads=0):
    """Contract forward on (B, H, L, D) arrays.  Returns (out, d) with d of shape (B, H, L, 1)."""
    q, k, v = _c(q, dtype), _c(k, dtype), _c(v, dtype)
    B, H, L, D = q.shape
    block_q = L if block_q is None else block_q
    block_k = L if block_k is None else block_k
    out = np.empty_like(q)
    dd = np.empty((B, H, L, 1), dtype=np.float64 if dtype == DT_F64 else np.float32)
    rc = rs = None
    if rotary is not None:
        tdt = np.float64 if dtype == DT_F64 else np.float32
        rc = np.ascontiguousarray(rotary[0], dtype=tdt)
        rs = np.ascontiguousarray(rotary[1], dtype=tdt)
    rc_ = np.ascontiguousarray(rc[:L]) if rc is not None else None
    rs_ = np.ascontiguousarray(rs[:L]) if rs is not None else None
    rc_code = lib().oracle_afa_fwd(dtype, B, H, L, D, _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(dd),
                                   _ptr(rc_), _ptr(rs_), float(sink_omega), int(bool(causal)),
                                   0 if valid_len is None else int(valid_len), block_q, block_k,
                                   nthreads)
    if rc_code:
        raise ValueError(f"oracle_afa_fwd rejected the arguments (code {rc_code})")
    return out, dd


def afa_exact_ref(q, k, v, dtype, sink_omega=0.5, causal=False, nthreads=0):
    """exact_afa_with_denominator (src/kernels/pallas_afa.py:300-327) for bf16 / fp16 bit patterns,
    every op rounded to the input dtype as the reference's JAX program types it.  Returns
    (out bits, d_total as float32 holding values of the input dtype) with d_total (B, H, L, 1)."""
    q, k, v = _c(q, dtype), _c(k, dtype), _c(v, dtype)
    B, H, L, D = q.shape
    out = np.empty_like(q)
    dd = np.empty((B, H, L, 1), dtype=np.float32)
    rc = lib().oracle_afa_exact_ref(dtype, B, H, L, D, _ptr(q), _ptr(k), _ptr(v), _ptr(out), _ptr(dd),
                                    float(sink_omega), int(bool(causal)), nthreads)
    if rc:
        raise ValueError(f"oracle_afa_exact_ref rejected the arguments (code {rc})")
    return out, dd


def rho8_step(x, dtype):
    """rho(s)^8 of the reference's _vmu_octic_kernel with every op rounded to bf16 / fp16
    (x: float32 values of that dtype)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().oracle_rho8_step(_ptr(x), _ptr(y), x.size, dtype)
    return y


def afa_bwd(q, k, v, out, d_total, g, dtype, causal=False, valid_len=None, nthreads=0):
    q, k, v, out, g = (_c(a, dtype) for a in (q, k, v, out, g))
    B, H, L, D = q.shape
    d_total = np.ascontiguousarray(d_total, dtype=np.float32)
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    rc_code = lib().oracle_afa_bwd(dtype, B, H, L, D, _ptr(q), _ptr(k), _ptr(v), _ptr(out),
                                   _ptr(d_total), _ptr(g), _ptr(dq), _ptr(dk), _ptr(dv),
                                   int(bool(causal)), 0 if valid_len is None else int(valid_len),
                                   nthreads)
    if rc_code:
        raise ValueError(f"oracle_afa_bwd rejected the arguments (code {rc_code})")
    return dq, dk, dv


def max_threads():
    return lib().oracle_max_threads()
