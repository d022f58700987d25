"""GPU parity of the sequence ring (distributed_ring_afa, src/kernels/pallas_afa.py:618-662).

The ring's hops run as afa_fwd calls with AFA_FLAG_ACCUMULATE and end in afa_ring_finish.  The
hops only re-associate the fp32 sums of the full forward, so the ring is checked against the
full fused forward on the same inputs (same per-tile arithmetic: at most a rounding step of the
output apart), against the C restatement of the forward's dtype contract, and against the
float64 ring of the oracle at the north-star tolerances (fp32 1e-5, bf16/fp16 2e-2 normwise).
"""
import numpy as np
import pytest
import torch

from oracle import afa_oracle as O
from tests.helpers import make_qkv, normwise, oracle_contract, to_f64

pytestmark = pytest.mark.gpu

import algebraic_intelligence_amd as A  # noqa: E402
from algebraic_intelligence_amd import _lib  # noqa: E402


def _ring_checks(shape, dtype, n, causal, sink=0.5, seed=0, tol_full=4e-3, tol_ref=2e-2, scale=1.0):
    q, k, v = make_qkv(shape, dtype, seed=seed, scale=scale)
    out = A.distributed_ring_afa(q, k, v, sink_omega=sink, causal=causal, num_devices=n)
    assert out.dtype == dtype and out.shape == q.shape
    full = A.pallas_afa_forward(q, k, v, sink_omega=sink, causal=causal)
    ref = O.ring_afa(to_f64(q), to_f64(k), to_f64(v), sink, causal, n)
    e_full, e_ref = normwise(to_f64(out), to_f64(full)), normwise(to_f64(out), ref)
    print(f"ring {tuple(shape)} {dtype} n={n} causal={causal}: vs full {e_full:.3e} vs fp64 {e_ref:.3e}",
          flush=True)
    assert e_full <= tol_full
    assert e_ref <= tol_ref
    return q, k, v, out


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n", [1, 2, 8])
def test_ring_bf16_d64(n, causal):
    q, k, v, out = _ring_checks((2, 4, 1024, 64), torch.bfloat16, n, causal, seed=40 + n)
    if n == 8:
        c_out, _ = oracle_contract(q, k, v, 0.5, causal)
        assert normwise(to_f64(out), c_out) <= 4e-3


@pytest.mark.parametrize("causal", [False, True])
def test_ring_fp16_d128(causal):
    # scale 0.5 keeps rho^8 within fp16's range as the PV operand (as in the forward's fp16 tests)
    _ring_checks((1, 3, 512, 128), torch.float16, 4, causal, seed=50, scale=0.5)


def test_ring_bf16_padded_head_dim():
    _ring_checks((1, 2, 256, 48), torch.bfloat16, 2, True, seed=51)


def test_ring_long_shards_split_keys():
    """Two shards of 4096 rows and one head: few query blocks per call, so the 128-query kernel
    splits each block's keys over several workgroups and the last part accumulates."""
    _ring_checks((1, 1, 8192, 64), torch.bfloat16, 2, False, seed=52)
    _ring_checks((1, 1, 8192, 128), torch.bfloat16, 2, True, seed=53)


@pytest.mark.parametrize("causal", [False, True])
def test_ring_fp32(causal):
    _ring_checks((1, 2, 256, 64), torch.float32, 4, causal, seed=54, tol_full=1e-5, tol_ref=1e-5)


def test_ring_fp64():
    _ring_checks((1, 2, 128, 32), torch.float64, 4, True, seed=55, tol_full=1e-12, tol_ref=1e-12)


def test_ring_zero_sink_and_determinism():
    q, k, v = make_qkv((1, 2, 512, 64), torch.bfloat16, seed=56)
    a = A.distributed_ring_afa(q, k, v, sink_omega=0.0, causal=True, num_devices=4)
    b = A.distributed_ring_afa(q, k, v, sink_omega=0.0, causal=True, num_devices=4)
    assert torch.equal(a, b)
    ref = O.ring_afa(to_f64(q), to_f64(k), to_f64(v), 0.0, True, 4)
    assert normwise(to_f64(a), ref) <= 2e-2


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 64), (torch.bfloat16, 128), (torch.float32, 64)])
def test_accumulate_flag_adds_unnormalised_sums(dtype, D):
    """afa_fwd with AFA_FLAG_ACCUMULATE adds sum_j rho^8 v_j and sum_j rho^8 to what the
    accumulators hold: starting from random contents, the increments equal out * d and d of a
    plain sink-0 forward on the same inputs."""
    q, k, v = make_qkv((2, 3, 384, D), dtype, seed=57)
    B, H, L, _ = q.shape
    out, den = A.afa._launch_fwd(q, k, v, 0.0, True, None, None, 0, True)
    g = torch.Generator(device="cuda").manual_seed(3)
    acc0 = torch.randn((B, H, L, D), generator=g, device="cuda", dtype=torch.float32)
    den0 = torch.randn((B, H, L), generator=g, device="cuda", dtype=torch.float32)
    acc, dacc = acc0.clone(), den0.clone()
    dt = _lib.dtype_code(dtype)
    ws_bytes = _lib.lib().afa_fwd_workspace_size(dt, B, H, L, D, 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    rc = _lib.lib().afa_fwd(dt, B, H, L, D, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                            A.afa._strides(q, k, v, acc), acc.data_ptr(), dacc.data_ptr(), None, None, 0,
                            0.0, 1, 0, _lib.FLAG_ACCUMULATE, ws.data_ptr(), ws_bytes,
                            _lib.stream_ptr(q.device))
    assert rc == _lib.OK
    torch.cuda.synchronize()
    d_inc = to_f64(dacc - den0)
    assert normwise(d_inc, to_f64(den[..., 0])) <= 1e-5
    o_inc = to_f64(acc - acc0)
    o_ref = to_f64(out) * to_f64(den)
    assert normwise(o_inc, o_ref) <= (1e-5 if dtype == torch.float32 else 8e-3)
