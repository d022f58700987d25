"""afa_fwd_noalloc, the allocation-free variant of afa_fwd: its workspace is the library's fixed
per-device scratch array.  Through the C ABI it must give afa_fwd's results bit for bit (the same
kernels on the same inputs) over consecutive calls, each smaller or on another path than the one
before (the array keeps the previous call's contents, which no call may depend on); refuse a call
that needs more than the array before any device work; and allocate no device memory."""
import numpy as np
import pytest
import torch

import algebraic_intelligence_amd as A
from algebraic_intelligence_amd import _lib
from tests.helpers import make_qkv

pytestmark = pytest.mark.gpu


def _run(entry, q, k, v, rot, causal, valid):
    lib = _lib.lib()
    B, H, L, D = q.shape
    code = _lib.dtype_code(q.dtype)
    out = torch.empty_like(q)
    den = torch.empty((B, H, L), dtype=_lib.accum_dtype(q.dtype), device=q.device)
    c, s, rlen = (None, None, 0) if rot is None else (rot.c.contiguous(), rot.s.contiguous(), L)
    args = (code, B, H, L, D, q.data_ptr(), k.data_ptr(), v.data_ptr(), None, out.data_ptr(), den.data_ptr(),
            _lib.ptr(c), _lib.ptr(s), rlen, 0.5, int(causal), valid, 0)
    stream = torch.cuda.current_stream().cuda_stream
    if entry == "afa_fwd":
        ws_bytes = lib.afa_fwd_workspace_size(code, B, H, L, D, int(rot is not None))
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
        rc = lib.afa_fwd(*args, ws.data_ptr(), ws_bytes, stream)
    else:
        rc = lib.afa_fwd_noalloc(*args, stream)
    _lib.check(rc, entry)
    return out, den


# consecutive calls: a large pipelined call with the K rotation (the whole rotated K in the
# array), a smaller one, the 256-query head_dim-64 kernel, head_dim 128 without tables (row-norm
# pass only), fp32 with split-K partials, fp64 (no workspace at all), and a small call again
CASES = [
    ((2, 12, 1024, 64), torch.bfloat16, True, True, 0),
    ((1, 3, 256, 64), torch.bfloat16, True, True, 200),
    ((4, 200, 256, 64), torch.bfloat16, True, True, 0),
    ((1, 4, 512, 128), torch.bfloat16, False, True, 0),
    ((1, 2, 512, 64), torch.float32, True, False, 300),
    ((1, 2, 128, 64), torch.float64, False, True, 0),
    ((1, 1, 64, 64), torch.float16, True, True, 0),
]


def _inputs(i, shape, dt, rot):
    q, k, v = make_qkv(shape, dt, seed=400 + i, scale=0.5)
    r = A.build_cayley_rotary_matrix(shape[-1], shape[2]) if rot else None
    return q, k, v, r


def test_noalloc_matches_afa_fwd_over_consecutive_calls():
    inputs = [_inputs(i, *c[:2], c[2]) for i, c in enumerate(CASES)]
    refs = [_run("afa_fwd", *inp, c[3], c[4]) for inp, c in zip(inputs, CASES)]
    torch.cuda.synchronize()
    for rnd in range(2):
        for (shape, dt, rot, causal, valid), inp, (o_ref, d_ref) in zip(CASES, inputs, refs):
            out, den = _run("afa_fwd_noalloc", *inp, causal, valid)
            torch.cuda.synchronize()
            print(f"round {rnd}: {shape} {dt} rot={rot} causal={causal} valid={valid}: "
                  f"equal {torch.equal(out, o_ref)} / {torch.equal(den, d_ref)}", flush=True)
            assert torch.equal(out, o_ref) and torch.equal(den, d_ref), shape


def test_noalloc_allocates_nothing():
    """Device free memory is the same before and after a run of calls on every path (the kernels
    were loaded by the first calls; the scratch array was placed when the library loaded)."""
    inputs = [_inputs(i, *c[:2], c[2]) for i, c in enumerate(CASES)]
    for inp, c in zip(inputs, CASES):
        _run("afa_fwd_noalloc", *inp, c[3], c[4])
    # the output buffers come from before the measurement
    bufs = [(torch.empty_like(inp[0]), torch.empty(inp[0].shape[:3], dtype=_lib.accum_dtype(inp[0].dtype),
                                                     device="cuda")) for inp in inputs]
    tables = [(None, None, 0) if inp[3] is None else (inp[3].c.contiguous(), inp[3].s.contiguous(), inp[0].shape[2])
              for inp in inputs]
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    stream = torch.cuda.current_stream().cuda_stream
    for _ in range(3):
        for inp, c, (out, den), (tc, ts, rlen) in zip(inputs, CASES, bufs, tables):
            q, k, v, _r = inp
            B, H, L, D = q.shape
            rc = _lib.lib().afa_fwd_noalloc(_lib.dtype_code(q.dtype), B, H, L, D, q.data_ptr(), k.data_ptr(),
                                           v.data_ptr(), None, out.data_ptr(), den.data_ptr(), _lib.ptr(tc),
                                           _lib.ptr(ts), rlen, 0.5, int(c[3]), c[4], 0, stream)
            assert rc == _lib.OK
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    print(f"device free memory before {free0} after {free1}", flush=True)
    assert free1 == free0


def test_noalloc_refuses_calls_beyond_the_scratch():
    """B=8 H=12 L=8192 D=64 bf16 with tables needs 100 MB of workspace (the rotated K): refused
    with AFA_ERR_SCRATCH_LIMIT before any device work (the pointers are never dereferenced)."""
    lib = _lib.lib()
    need = lib.afa_fwd_workspace_size(_lib.AFA_BF16, 8, 12, 8192, 64, 1)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    dummy = 0x1000
    rc = lib.afa_fwd_noalloc(_lib.AFA_BF16, 8, 12, 8192, 64, dummy, dummy, dummy, None, dummy, None, dummy, dummy,
                             8192, 0.5, 1, 0, 0, None)
    assert rc == _lib.ERR_SCRATCH_LIMIT
    assert "scratch" in lib.afa_status_string(rc).decode()
    # the C3 workload fits
    assert lib.afa_fwd_workspace_size(_lib.AFA_BF16, 8, 12, 4096, 64, 1) <= _lib.NOALLOC_SCRATCH_BYTES
