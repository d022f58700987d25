"""Rows past the end of a head are never read from memory.

The MFMA kernels stage key/value tiles (forward) and key/value or query/cotangent tiles
(backward) of 32 or 64 rows; when L is not a multiple of the tile, the last tile covers rows
past L.  Those rows belong to masked keys (or queries), but the kernels still multiply them on the
matrix cores (O += V^T P, dQ += K^T dS^T, ...), so their bytes must be finite: a NaN there turns
the whole output row into NaN even though its weight is zero.  The kernels read such rows as
zeros (buffer loads whose range ends with the head) or as a copy of row L - 1.

These tests put NaN right after every head (a padded head stride) or right after the last head
(a flat allocation one tail longer than the tensor), and NaN in every byte of the workspace that
the call does not write, at L % 32 != 0, and require outputs equal, bit for bit, to the same call
on inputs with no NaN anywhere, which the parity tests check against the contract.  Every call
goes through the C ABI.
"""
import numpy as np
import pytest
import torch

from tests.helpers import make_qkv, normwise, oracle_contract, to_f64

pytestmark = pytest.mark.gpu

import algebraic_intelligence_amd as A  # noqa: E402
from algebraic_intelligence_amd import _lib  # noqa: E402
from algebraic_intelligence_amd.afa import _strides  # noqa: E402

DEV = "cuda"
NAN16 = 0x7FC0  # a quiet NaN in bfloat16


def _nan_tailed_heads(x: torch.Tensor, pad: int) -> torch.Tensor:
    """x (B, H, L, D) as a view whose head stride leaves `pad` rows of NaN after every head."""
    B, H, L, D = x.shape
    big = torch.full((B, H, L + pad, D), float("nan"), dtype=x.dtype, device=x.device)
    big[:, :, :L] = x
    return big[:, :, :L]


def _nan_tailed_flat(x: torch.Tensor, pad_rows: int) -> torch.Tensor:
    """x as a contiguous tensor followed in memory by `pad_rows` rows of NaN."""
    B, H, L, D = x.shape
    n = x.numel()
    flat = torch.full((n + pad_rows * D,), float("nan"), dtype=x.dtype, device=x.device)
    flat[:n] = x.reshape(-1)
    return flat[:n].view(B, H, L, D)


def _nan_bytes(n: int) -> torch.Tensor:
    """A workspace whose every 16-bit word holds a bf16 NaN (every fp32 word a NaN as well)."""
    n = (n + 1) // 2 * 2
    return torch.full((n // 2,), NAN16, dtype=torch.int16, device=DEV).view(torch.uint8)


def _fwd_call(q, k, v, causal, rot, ws=None):
    B, H, L, D = q.shape
    dt = _lib.dtype_code(q.dtype)
    out = torch.empty((B, H, L, D), dtype=q.dtype, device=DEV)
    den = torch.empty((B, H, L, 1), dtype=torch.float32, device=DEV)
    c = s = None
    rot_len = 0
    if rot is not None:
        c, s, rot_len = rot.c.float().contiguous(), rot.s.float().contiguous(), rot.c.shape[0]
    ws_bytes = _lib.lib().afa_fwd_workspace_size(dt, B, H, L, D, int(rot is not None))
    if ws is None:
        ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    else:
        ws = ws(ws_bytes)
    rc = _lib.lib().afa_fwd(dt, B, H, L, D, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _strides(q, k, v, out),
                            _lib.ptr(out), _lib.ptr(den), _lib.ptr(c), _lib.ptr(s), rot_len, 0.5, int(causal), 0, 0,
                            _lib.ptr(ws), ws_bytes, _lib.stream_ptr(torch.device(DEV)))
    _lib.check(rc, "afa_fwd")
    torch.cuda.synchronize()
    return out, den


def _bwd_call(q, k, v, out, den, g, causal, rot, ws=None):
    B, H, L, D = q.shape
    dt = _lib.dtype_code(q.dtype)
    dq, dk, dv = (torch.empty((B, H, L, D), dtype=q.dtype, device=DEV) for _ in range(3))
    c = s = None
    rot_len = 0
    if rot is not None:
        c, s, rot_len = rot.c.float().contiguous(), rot.s.float().contiguous(), rot.c.shape[0]
    ws_bytes = _lib.lib().afa_bwd_workspace_size(dt, B, H, L, D, int(rot is not None))
    wsb = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=DEV) if ws is None else ws(ws_bytes)
    rc = _lib.lib().afa_bwd(dt, B, H, L, D, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(den),
                            _lib.ptr(g), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(c), _lib.ptr(s), rot_len,
                            0.5, int(causal), 0, 0, _lib.ptr(wsb), ws_bytes, _lib.stream_ptr(torch.device(DEV)))
    _lib.check(rc, "afa_bwd")
    torch.cuda.synchronize()
    return dq, dk, dv


# (B, H, L, D): the 128-query forward at head_dim 64 (small grid) and 128; the 256-query forward
# at head_dim 64 (enough workgroups for three per CU: 192 heads of 4 query blocks)
FWD_SHAPES = [(1, 2, 1000, 64), (1, 2, 1000, 128), (1, 2, 999, 128), (1, 192, 1000, 64)]


@pytest.mark.parametrize("rotary", [False, True], ids=["plain", "rotary"])
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
@pytest.mark.parametrize("shape", FWD_SHAPES)
def test_forward_never_reads_past_the_head(shape, causal, rotary):
    B, H, L, D = shape
    print(f"forward {shape} causal={causal} rotary={rotary}", flush=True)
    q, k, v = make_qkv(shape, torch.bfloat16, seed=L + D)
    rot = A.build_cayley_rotary_matrix(D, L) if rotary else None
    ref_out, ref_den = _fwd_call(q, k, v, causal, rot)
    # NaN after every head of k and v (and of q), and in every workspace byte the call leaves alone
    qn, kn, vn = (_nan_tailed_heads(x, 32) for x in (q, k, v))
    out, den = _fwd_call(qn, kn, vn, causal, rot, ws=_nan_bytes)
    assert torch.isfinite(out.float()).all() and torch.isfinite(den).all()
    assert torch.equal(out, ref_out) and torch.equal(den, ref_den)
    # NaN right after the last head of contiguous inputs
    qf, kf, vf = (_nan_tailed_flat(x, 64) for x in (q, k, v))
    out2, den2 = _fwd_call(qf, kf, vf, causal, rot, ws=_nan_bytes)
    assert torch.equal(out2, ref_out) and torch.equal(den2, ref_den)
    # the clean run itself against the contract on the last head (whose tail was NaN above)
    b, h = B - 1, H - 1
    c_out, c_den = oracle_contract(q[b:, h:], k[b:, h:], v[b:, h:], 0.5, causal,
                                   rotary=None if rot is None else (rot.c, rot.s))
    e = normwise(to_f64(ref_out[b:, h:]), c_out)
    print(f"  last head vs the C contract: {e:.2e}", flush=True)
    assert e <= 8e-3
    assert normwise(to_f64(ref_den[b:, h:]).reshape(c_den.shape), c_den) <= 1e-5


@pytest.mark.parametrize("rotary", [False, True], ids=["plain", "rotary"])
@pytest.mark.parametrize("D,L", [(64, 1000), (128, 999), (256, 1000)])
def test_backward_never_reads_past_the_head(D, L, rotary):
    """The MFMA backward's tile loads (dQ: k, v; dK/dV: q, g) with NaN after the last head of
    every contiguous input and in the workspace (where the rotated q and k live with tables)."""
    B, H = 1, 2
    print(f"backward D={D} L={L} rotary={rotary}", flush=True)
    q, k, v = make_qkv((B, H, L, D), torch.bfloat16, seed=D + 1)
    g = make_qkv((B, H, L, D), torch.bfloat16, seed=D + 2)[0]
    rot = A.build_cayley_rotary_matrix(D, L) if rotary else None
    out, den = _fwd_call(q, k, v, True, rot)
    ref = _bwd_call(q, k, v, out, den, g, True, rot)
    args = [_nan_tailed_flat(x, 128) for x in (q, k, v, out)]
    gn = _nan_tailed_flat(g, 128)
    got = _bwd_call(*args, den, gn, True, rot, ws=_nan_bytes)
    for name, x, y in zip(("dq", "dk", "dv"), got, ref):
        assert torch.isfinite(x.float()).all(), name
        assert torch.equal(x, y), name
