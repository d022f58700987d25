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


def test_ring_head_dim_off_the_vector_paths():
    """head_dim 20: the generic kernel's hops and the element-wise finish kernel."""
    _ring_checks((1, 2, 128, 20), torch.bfloat16, 2, True, seed=58)
    _ring_checks((1, 2, 128, 20), torch.float32, 4, False, seed=59, tol_full=1e-5, tol_ref=1e-5)


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


def test_ring_reference_check_configuration():
    """The reference's 16-chip ring check (scripts/run_phase6_tpu.py:358-435): B=1 H=8 L=4096 as 16
    shards of 256, D=64, fp32, non-causal, sink 0.5, inputs numpy default_rng(942) normals in the
    order q, k, v; every shard's max|ring - unsplit| / max|unsplit|.  The reference bounds it by 1e-6
    against its unsplit fp32 attention in the same arithmetic (its TPU run measured 4.15e-7,
    results/phase6/tpu/metrics.json:338); here the unsplit fp32 forward is pallas_afa_forward on the
    same kernel, and the float64 oracle is held to the fp32 north-star 1e-5."""
    q, k, v = make_qkv((1, 8, 4096, 64), torch.float32, seed=942)
    out = to_f64(A.distributed_ring_afa(q, k, v, sink_omega=0.5, causal=False, axis_name="ici_ring",
                                        num_devices=16))
    unsplit = to_f64(A.pallas_afa_forward(q, k, v, sink_omega=0.5))
    ref = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, False)

    def shard_err(r):
        return max(normwise(out[..., 256 * d:256 * (d + 1), :], r[..., 256 * d:256 * (d + 1), :]) for d in range(16))

    e_unsplit, e_ref = shard_err(unsplit), shard_err(ref)
    print(f"16-shard ring max rel err: vs unsplit fp32 {e_unsplit:.3e}, vs fp64 {e_ref:.3e}", flush=True)
    assert e_unsplit <= 1e-6
    assert e_ref <= 1e-5


@pytest.mark.parametrize("dtype,D,B,H,L", [(torch.bfloat16, 64, 2, 3, 384), (torch.bfloat16, 128, 2, 3, 384),
                                           (torch.float32, 64, 4, 8, 1024), (torch.float32, 64, 1, 1, 2048),
                                           (torch.bfloat16, 64, 8, 12, 2048), (torch.bfloat16, 256, 1, 2, 256)])
def test_shard_flags_store_and_add_unnormalised_sums(dtype, D, B, H, L):
    """afa_fwd with AFA_FLAG_PARTIAL stores sum_j rho^8 v_j and sum_j rho^8, with
    AFA_FLAG_ACCUMULATE adds them to what the arrays hold: starting from random contents, the
    stored values and the increments equal out * d and d of a plain sink-0 forward on the same
    inputs.  Shapes cover the 128-query pipelined kernel, the 256-query head_dim-64 kernel
    (B H L/256 >= 3 x CUs), the fp32 matrix-core kernel without and with its key split (B H L/128
    below the CU count), and the generic kernel (bf16 head_dim 256)."""
    q, k, v = make_qkv((B, H, L, D), dtype, seed=57)
    B, H, L, _ = q.shape
    out, den = A.afa._launch_fwd(q, k, v, 0.0, True, None, None, 0, True)
    g = torch.Generator(device="cuda").manual_seed(3)
    acc0 = torch.randn((B, H, L, D), generator=g, device="cuda", dtype=torch.float32)
    den0 = torch.randn((B, H, L), generator=g, device="cuda", dtype=torch.float32)
    dt = _lib.dtype_code(dtype)
    ws_bytes = _lib.lib().afa_fwd_workspace_size(dt, B, H, L, D, 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    o_ref = to_f64(out) * to_f64(den)
    tol = 1e-5 if dtype == torch.float32 else 8e-3
    for flag in (_lib.FLAG_PARTIAL, _lib.FLAG_ACCUMULATE):
        acc, dacc = acc0.clone(), den0.clone()
        rc = _lib.lib().afa_fwd(dt, B, H, L, D, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                A.afa._strides(q, k, v, acc), acc.data_ptr(), dacc.data_ptr(), None, None, 0,
                                0.0, 1, 0, flag, ws.data_ptr(), ws_bytes, _lib.stream_ptr(q.device))
        assert rc == _lib.OK
        torch.cuda.synchronize()
        base_o, base_d = (acc0, den0) if flag == _lib.FLAG_ACCUMULATE else (0.0, 0.0)
        assert normwise(to_f64(dacc - base_d), to_f64(den[..., 0])) <= 1e-5, flag
        assert normwise(to_f64(acc - base_o), o_ref) <= tol, flag


def test_sharded_pallas_afa_equals_pallas_afa():
    """sharded_pallas_afa (src/kernels/pallas_afa.py:665-692) on a (data 2, fsdp 3) mesh: the same
    output and gradients as pallas_afa on the whole arrays."""
    q, k, v = make_qkv((2, 6, 256, 64), torch.bfloat16, seed=60)
    qs, ks, vs = (t.clone().requires_grad_(True) for t in (q, k, v))
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = A.sharded_pallas_afa(qs, ks, vs, mesh={"data": 2, "fsdp": 3, "model": 1}, causal=True)
    ref = A.pallas_afa(qa, ka, va, causal=True)
    assert torch.equal(out, ref)
    g = torch.randn_like(out)
    out.backward(g)
    ref.backward(g)
    for a, b in ((qs, qa), (ks, ka), (vs, va)):
        assert torch.equal(a.grad, b.grad)


def test_ring_reference_test_configuration_fp64():
    """The reference's ring test (tests/test_pallas_afa.py:227-271): fp64, B=1 H=2 L=256 D=32 as 4
    shards, non-causal, sink 0.5; max error / max|exact| <= 1e-6 against exact_afa_reference
    (here: against this build's exact reference and the float64 oracle, <= 1e-12)."""
    q, k, v = make_qkv((1, 2, 256, 32), torch.float64, seed=107)
    out = to_f64(A.distributed_ring_afa(q, k, v, sink_omega=0.5, causal=False, num_devices=4))
    exact = to_f64(A.exact_afa_reference(q, k, v, sink_omega=0.5))
    assert normwise(out, exact) <= 1e-6
    assert normwise(out, O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, False)) <= 1e-12


@pytest.mark.parametrize("dtype,causal,n", [(torch.bfloat16, True, 4), (torch.bfloat16, False, 8),
                                            (torch.float32, True, 2), (torch.float64, False, 4)])
def test_ring_gradients(dtype, causal, n):
    """distributed_ring_afa is differentiable, as the reference's JAX function: its gradients equal
    pallas_afa's on the same inputs (same analytical backward, the ring's own output and total
    denominator), and the fp64 case matches the oracle's finite-difference-pinned backward."""
    q, k, v = make_qkv((1, 2, 256, 64), dtype, seed=61, scale=0.5 if dtype == torch.float16 else 1.0)
    g = make_qkv((1, 2, 256, 64), dtype, seed=62)[0]
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    A.distributed_ring_afa(qr, kr, vr, causal=causal, num_devices=n).backward(g)
    A.pallas_afa(qa, ka, va, causal=causal).backward(g)
    tol = {torch.bfloat16: 2e-2, torch.float32: 1e-5, torch.float64: 1e-12}[dtype]
    for a, b, name in ((qr, qa, "dq"), (kr, ka, "dk"), (vr, va, "dv")):
        e = normwise(to_f64(a.grad), to_f64(b.grad))
        print(f"ring grad {dtype} causal={causal} n={n} {name}: {e:.2e}", flush=True)
        assert e <= tol, name
    if dtype == torch.float64:
        dq, dk, dv = O.afa_backward(to_f64(q), to_f64(k), to_f64(v), to_f64(g), 0.5, causal)
        for a, ref in ((qr, dq), (kr, dk), (vr, dv)):
            assert normwise(to_f64(a.grad), ref) <= 1e-10
