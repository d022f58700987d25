"""GPU parity of the rest of the call surface: the golden fixtures through the forward, the
analytical backward (tiled_afa_backward / pallas_afa autograd), exact_afa_reference, the padding
front door, algebraic_softmax, octic_kernel and the Cayley rotary tables and rotation.

Oracles: the 40-digit mpmath fixtures of tests/golden/, the float64 numpy oracle and the C
contract restatement (oracle/).  Tolerances are normwise, max|y - ref| / max|ref|.
"""
import os

import numpy as np
import pytest
import torch

from oracle import afa_oracle as O
from oracle import contract as C
from tests.helpers import from_bits, make_qkv, normwise, to_bits, to_f64

pytestmark = pytest.mark.gpu

import algebraic_intelligence_amd as A  # noqa: E402

DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "afa_golden.npz")
FWD_CASES = ["fwd_plain", "fwd_causal_valid", "fwd_nosink_causal", "fwd_tail", "fwd_rotary",
             "fwd_d64_rotary", "fwd_d128"]
TOL = {torch.float64: 1e-12, torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 4e-3}


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _t(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(DEV)


# ------------------------------------------------------------------------------ forward fixtures
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name", FWD_CASES)
def test_forward_matches_golden(gold, name, dtype):
    sink, causal, valid = gold[f"{name}_cfg"]
    q, k, v = (_t(gold[f"{name}_{x}"], dtype) for x in "qkv")
    L = q.shape[2]
    rot = None
    if f"{name}_cos" in gold:
        rot = (torch.from_numpy(gold[f"{name}_cos"]).to(DEV), torch.from_numpy(gold[f"{name}_sin"]).to(DEV))
    out, den = A.pallas_afa_forward(q, k, v, float(sink), bool(causal), block_q=L, block_k=L,
                                    valid_seq_len=None if valid < 0 else int(valid),
                                    return_denominator=True, rotary_params=rot)
    err = normwise(to_f64(out), gold[f"{name}_out"])
    derr = normwise(to_f64(den), gold[f"{name}_den"])
    print(f"{name} {dtype}: out {err:.2e} den {derr:.2e}")
    assert out.dtype == dtype
    assert err <= TOL[dtype]
    assert derr <= (1e-12 if dtype == torch.float64 else 1e-5 if dtype == torch.float32 else 2e-2)


# ------------------------------------------------------------------------------ backward
@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-10), (torch.float32, 2e-5)])
def test_backward_matches_golden(gold, dtype, tol):
    q, k, v, g = (_t(gold[f"bwd_{x}"], dtype) for x in "qkvg")
    sink, causal, _ = gold["bwd_cfg"]
    L = q.shape[2]
    out, den = A.pallas_afa_forward(q, k, v, float(sink), bool(causal), block_q=L, block_k=L,
                                    return_denominator=True)
    grads = A.tiled_afa_backward(q, k, v, out, den, g, float(sink), bool(causal))
    for got, key in zip(grads, ("bwd_dq", "bwd_dk", "bwd_dv")):
        err = normwise(to_f64(got), gold[key])
        print(key, dtype, f"{err:.2e}")
        assert err <= tol


@pytest.mark.parametrize("causal,valid", [(False, None), (True, None), (True, 200), (False, 77)])
def test_backward_fp64_vs_oracle(causal, valid):
    q, k, v = make_qkv((2, 2, 256, 32), torch.float64, seed=31)
    g = make_qkv((2, 2, 256, 32), torch.float64, seed=32)[0]
    out, den = A.afa._launch_fwd(q, k, v, 0.5, causal, valid, None, 0, True)
    dq, dk, dv = A.tiled_afa_backward(q, k, v, out, den, g, 0.5, causal, valid_seq_len=valid)
    rq, rk, rv = O.afa_backward(to_f64(q), to_f64(k), to_f64(v), to_f64(g), 0.5, causal, valid)
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        assert normwise(to_f64(got), ref) <= 1e-10


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_backward_low_precision(dtype):
    """bf16 (C5's dtype, reduced length) and fp32 backward against the C contract restatement and
    the float64 oracle (the reference gates bf16 backward at 6e-3 against fp32,
    tests/test_pallas_afa.py:324-353)."""
    shape = (1, 2, 256, 128)
    q, k, v = make_qkv(shape, dtype, seed=41)
    g = make_qkv(shape, dtype, seed=42)[0]
    out, den = A.afa._launch_fwd(q, k, v, 0.5, True, None, None, 0, True)
    dq, dk, dv = A.tiled_afa_backward(q, k, v, out, den, g, 0.5, True)
    code = {torch.bfloat16: C.DT_BF16, torch.float32: C.DT_F32}[dtype]
    cq, ck, cv = C.afa_bwd(to_bits(q), to_bits(k), to_bits(v), to_bits(out), den.cpu().numpy(),
                           to_bits(g), code, True)
    rq, rk, rv = O.afa_backward(to_f64(q), to_f64(k), to_f64(v), to_f64(g), 0.5, True)
    for name, got, cref, ref in (("dq", dq, cq, rq), ("dk", dk, ck, rk), ("dv", dv, cv, rv)):
        e_c = normwise(to_f64(got), C.to_f32(cref, code))
        e_r = normwise(to_f64(got), ref)
        print(f"{dtype} {name}: vs contract {e_c:.2e} vs fp64 {e_r:.2e}")
        assert e_c <= (6e-3 if dtype == torch.bfloat16 else 1e-5)
        assert e_r <= (2e-2 if dtype == torch.bfloat16 else 1e-5)


def _bwd_flags(q, k, v, out, den, g, causal, valid, flags, rot=None):
    """afa_bwd through the C ABI with explicit flags (contiguous inputs; rot = fp32 (cos, sin)
    device tables or None)."""
    from algebraic_intelligence_amd import _lib
    B, H, L, D = q.shape
    dq, dk, dv = (torch.empty_like(t) for t in (q, k, v))
    code = _lib.dtype_code(q.dtype)
    ws_bytes = _lib.lib().afa_bwd_workspace_size(code, B, H, L, D, int(rot is not None))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    rc_p, rs_p, rlen = (None, None, 0) if rot is None else (rot[0].data_ptr(), rot[1].data_ptr(), rot[0].shape[0])
    rc = _lib.lib().afa_bwd(code, B, H, L, D, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                            den.data_ptr(), g.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                            rc_p, rs_p, rlen, 0.5, int(causal), 0 if valid is None else valid, flags,
                            ws.data_ptr(), ws_bytes, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "afa_bwd")
    return dq, dk, dv


@pytest.mark.parametrize("shape,causal,valid", [
    ((1, 2, 256, 64), True, None), ((2, 3, 200, 64), False, None), ((1, 2, 1000, 64), True, 777),
    ((1, 1, 4, 64), True, None), ((1, 2, 256, 128), True, None), ((2, 1, 392, 128), False, 300),
    ((1, 1, 128, 128), True, 61), ((1, 2, 256, 32), True, None), ((2, 3, 200, 48), False, None),
    ((1, 2, 300, 48), True, 257), ((1, 1, 8, 48), True, None), ((1, 2, 392, 96), True, None),
    ((2, 1, 200, 96), False, 150), ((1, 2, 257, 64), True, None), ((2, 1, 130, 128), False, 100),
    ((1, 1, 1, 64), True, None), ((1, 3, 3, 48), False, None), ((1, 2, 1001, 96), True, 999),
    ((1, 2, 260, 256), True, None), ((2, 1, 130, 256), False, 100),
])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_mfma_backward_vs_generic_and_contract(shape, causal, valid, dt):
    """The MFMA backward (bf16/fp16, head_dim 64/128, and 32/48/96 padded to 64/128) against the
    generic kernel (forced with AFA_FLAG_GENERIC), the C contract restatement and the float64
    oracle."""
    from algebraic_intelligence_amd import _lib
    scale = 1.0 if dt == torch.bfloat16 else 0.5
    q, k, v = make_qkv(shape, dt, seed=sum(shape) + 7, scale=scale)
    g = make_qkv(shape, dt, seed=sum(shape) + 8)[0]
    out, den = A.afa._launch_fwd(q, k, v, 0.5, causal, valid, None, 0, True)
    mq, mk, mv = _bwd_flags(q, k, v, out, den, g, causal, valid, 0)
    gq, gk, gv = _bwd_flags(q, k, v, out, den, g, causal, valid, _lib.FLAG_GENERIC)
    code = {torch.bfloat16: C.DT_BF16, torch.float16: C.DT_F16}[dt]
    cq, ck, cv = C.afa_bwd(to_bits(q), to_bits(k), to_bits(v), to_bits(out), den.cpu().numpy(),
                           to_bits(g), code, causal, valid)
    rq, rk, rv = O.afa_backward(to_f64(q), to_f64(k), to_f64(v), to_f64(g), 0.5, causal, valid)
    for name, m, gen, c, r in (("dq", mq, gq, cq, rq), ("dk", mk, gk, ck, rk), ("dv", mv, gv, cv, rv)):
        assert torch.isfinite(m.float()).all(), name
        e_g = normwise(to_f64(m), to_f64(gen))
        e_c = normwise(to_f64(m), C.to_f32(c, code))
        e_r = normwise(to_f64(m), r)
        print(f"{shape} causal={causal} valid={valid} {dt} {name}: vs generic {e_g:.2e} "
              f"vs contract {e_c:.2e} vs fp64 {e_r:.2e}")
        assert e_g <= 1e-2 and e_c <= 1e-2
        assert e_r <= 3e-2


@pytest.mark.parametrize("shape,causal,valid", [
    ((1, 2, 256, 64), True, None), ((2, 3, 200, 64), False, None), ((1, 2, 1000, 64), True, 777),
    ((1, 2, 256, 128), True, None), ((2, 1, 392, 128), False, 300), ((1, 2, 200, 48), True, None),
    ((1, 2, 300, 96), False, 257), ((1, 1, 128, 32), True, None), ((1, 2, 200, 256), True, None),
])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_mfma_backward_with_rotary_tables(shape, causal, valid, dt):
    """The MFMA backward with Cayley tables (q, k rotated once into scratch, dq and dk rotated
    back by R^T in the store epilogues) against the generic kernel with the same tables and the
    float64 oracle on the rotated inputs."""
    from algebraic_intelligence_amd import _lib
    B, H, L, D = shape
    scale = 1.0 if dt == torch.bfloat16 else 0.5
    q, k, v = make_qkv(shape, dt, seed=sum(shape) + 17, scale=scale)
    g = make_qkv(shape, dt, seed=sum(shape) + 18)[0]
    c, s = O.cayley_tables(D, L + 3, freqs=10000.0 ** (-2.0 * np.arange(D // 2) / D))
    c32, s32 = c.astype(np.float32), s.astype(np.float32)
    rot = (torch.from_numpy(c32).to(DEV), torch.from_numpy(s32).to(DEV))
    out, den = A.afa._launch_fwd(q, k, v, 0.5, causal, valid, rot, 0, True)
    mq, mk, mv = _bwd_flags(q, k, v, out, den, g, causal, valid, 0, rot)
    gq, gk, gv = _bwd_flags(q, k, v, out, den, g, causal, valid, _lib.FLAG_GENERIC, rot)
    cf, sf = c32[:L].astype(np.float64), s32[:L].astype(np.float64)
    qr, kr = O.rotate_pairs(to_f64(q), cf, sf), O.rotate_pairs(to_f64(k), cf, sf)
    rq, rk, rv = O.afa_backward(qr, kr, to_f64(v), to_f64(g), 0.5, causal, valid)
    rq, rk = O.rotate_pairs(rq, cf, -sf), O.rotate_pairs(rk, cf, -sf)
    for name, m, gen, r in (("dq", mq, gq, rq), ("dk", mk, gk, rk), ("dv", mv, gv, rv)):
        assert torch.isfinite(m.float()).all(), name
        e_g = normwise(to_f64(m), to_f64(gen))
        e_r = normwise(to_f64(m), r)
        print(f"rotary {shape} causal={causal} valid={valid} {dt} {name}: vs generic {e_g:.2e} vs fp64 {e_r:.2e}")
        assert e_g <= 1e-2
        assert e_r <= 3e-2


@pytest.mark.parametrize("shape,causal,valid,rot", [
    ((1, 2, 256, 64), True, None, False), ((2, 3, 200, 64), False, None, True), ((1, 2, 300, 32), True, 257, False),
    ((1, 1, 7, 32), True, None, True), ((1, 2, 256, 128), True, None, True), ((2, 1, 130, 128), False, 100, False),
    ((1, 2, 300, 96), True, None, True), ((2, 1, 140, 96), False, 99, False),
    ((1, 2, 260, 48), True, None, True), ((3, 1, 129, 48), False, 100, False),
])
def test_fp32_mfma_backward(shape, causal, valid, rot):
    """The fp32 backward on the fp32 matrix cores against the generic fp32 kernel (forced with
    AFA_FLAG_GENERIC) and the float64 oracle, with and without Cayley tables."""
    from algebraic_intelligence_amd import _lib
    B, H, L, D = shape
    q, k, v = make_qkv(shape, torch.float32, seed=sum(shape) + 27)
    g = make_qkv(shape, torch.float32, seed=sum(shape) + 28)[0]
    rt, cf, sf = None, None, None
    if rot:
        c, s_ = O.cayley_tables(D, L + 2, freqs=10000.0 ** (-2.0 * np.arange(D // 2) / D))
        c32, s32 = c.astype(np.float32), s_.astype(np.float32)
        rt = (torch.from_numpy(c32).to(DEV), torch.from_numpy(s32).to(DEV))
        cf, sf = c32[:L].astype(np.float64), s32[:L].astype(np.float64)
    out, den = A.afa._launch_fwd(q, k, v, 0.5, causal, valid, rt, 0, True)
    mq, mk, mv = _bwd_flags(q, k, v, out, den, g, causal, valid, 0, rt)
    gq, gk, gv = _bwd_flags(q, k, v, out, den, g, causal, valid, _lib.FLAG_GENERIC, rt)
    qr, kr = to_f64(q), to_f64(k)
    if rot:
        qr, kr = O.rotate_pairs(qr, cf, sf), O.rotate_pairs(kr, cf, sf)
    rq, rk, rv = O.afa_backward(qr, kr, to_f64(v), to_f64(g), 0.5, causal, valid)
    if rot:
        rq, rk = O.rotate_pairs(rq, cf, -sf), O.rotate_pairs(rk, cf, -sf)
    for name, m, gen, r in (("dq", mq, gq, rq), ("dk", mk, gk, rk), ("dv", mv, gv, rv)):
        assert torch.isfinite(m).all(), name
        e_g, e_r = normwise(to_f64(m), to_f64(gen)), normwise(to_f64(m), r)
        print(f"fp32 {shape} causal={causal} valid={valid} rot={rot} {name}: vs generic {e_g:.2e} vs fp64 {e_r:.2e}")
        assert e_g <= 1e-5 and e_r <= 1e-5


def test_backward_with_fused_rotation():
    """dq, dk are gradients with respect to the unrotated q, k: R^T applied to the gradients of
    the rotated inputs."""
    shape = (1, 2, 96, 16)
    q, k, v = make_qkv(shape, torch.float64, seed=51)
    g = make_qkv(shape, torch.float64, seed=52)[0]
    c, s = O.cayley_tables(16, 96, freqs=10000.0 ** (-2.0 * np.arange(8) / 16))
    rot = (torch.from_numpy(c).to(DEV), torch.from_numpy(s).to(DEV))
    out, den = A.afa._launch_fwd(q, k, v, 0.5, True, None, rot, 0, True)
    dq, dk, dv = A.tiled_afa_backward(q, k, v, out, den, g, 0.5, True, rotary_params=rot)
    qr, kr = O.rotate_pairs(to_f64(q), c, s), O.rotate_pairs(to_f64(k), c, s)
    rq, rk, rv = O.afa_backward(qr, kr, to_f64(v), to_f64(g), 0.5, True)
    assert normwise(to_f64(dq), O.rotate_pairs(rq, c, -s)) <= 1e-10
    assert normwise(to_f64(dk), O.rotate_pairs(rk, c, -s)) <= 1e-10
    assert normwise(to_f64(dv), rv) <= 1e-10


def test_pallas_afa_autograd():
    shape = (1, 2, 64, 16)
    q, k, v = (t.requires_grad_(True) for t in make_qkv(shape, torch.float64, seed=61))
    g = make_qkv(shape, torch.float64, seed=62)[0]
    out = A.pallas_afa(q, k, v, 0.5, True, block_q=32, block_k=32)
    (out * g).sum().backward()
    rq, rk, rv = O.afa_backward(to_f64(q), to_f64(k), to_f64(v), to_f64(g), 0.5, True)
    for got, ref in ((q.grad, rq), (k.grad, rk), (v.grad, rv)):
        assert normwise(to_f64(got), ref) <= 1e-10


@pytest.mark.parametrize("L", [180, 190])
def test_flash_attention_front_door_any_length(L):
    """Lengths that are not tile multiples (reference tests/test_pallas_afa.py:173-198)."""
    q, k, v = (t.requires_grad_(True) for t in make_qkv((1, 2, L, 64), torch.float32, seed=L))
    out = A.algebraic_flash_attention(q, k, v, causal=True, block_q=64, block_k=32)
    ref = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, True)
    assert out.shape == q.shape
    assert normwise(to_f64(out), ref) <= 1e-5
    g = torch.ones_like(out)
    out.backward(g)
    rq, rk, rv = O.afa_backward(to_f64(q), to_f64(k), to_f64(v), to_f64(g), 0.5, True)
    for got, r in ((q.grad, rq), (k.grad, rk), (v.grad, rv)):
        assert normwise(to_f64(got), r) <= 2e-5


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_exact_afa_reference(dtype):
    q, k, v = make_qkv((1, 2, 128, 64), dtype, seed=71)
    out, den = A.exact_afa_with_denominator(q, k, v, 0.5, True)
    ref, rden = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, True, return_denominator=True)
    tol = 1e-12 if dtype == torch.float64 else 1e-5
    assert normwise(to_f64(out), ref) <= tol
    assert normwise(to_f64(den), rden) <= tol
    assert normwise(to_f64(A.exact_afa_reference(q, k, v, 0.5, True)), ref) <= tol


@pytest.mark.parametrize("shape", [(1, 2, 96, 64), (2, 3, 200, 128), (1, 2, 333, 64)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("dtype,scale", [(torch.bfloat16, 1.0), (torch.float16, 0.3)])
def test_exact_afa_reference_half(dtype, scale, causal, shape):
    """exact_afa_reference / exact_afa_with_denominator in bf16 and fp16 (pallas_afa.py:267-327):
    every op of the reference program rounded to the input dtype.  Bit for bit equal to the C
    oracle's restatement (which fixes the summation orders the program leaves open), within the
    reference's bf16 parity gate of float64 (4e-2; fp16 1e-2, on inputs scaled so rho^8 stays below
    fp16's maximum, past which the reference's fp16 formula overflows), and the distance to the
    fp32-internal contract of pallas_afa_forward reported."""
    B, H, L, D = shape
    q, k, v = make_qkv(shape, dtype, seed=72 + D + causal, scale=scale)
    out, den = A.exact_afa_with_denominator(q, k, v, 0.5, causal)
    assert den.dtype == dtype and den.shape == (B, H, L, 1)
    code = C.DT_BF16 if dtype == torch.bfloat16 else C.DT_F16
    c_out, c_den = C.afa_exact_ref(to_bits(q), to_bits(k), to_bits(v), code, 0.5, causal)
    assert np.array_equal(to_bits(out), c_out)
    assert np.array_equal(den.float().cpu().numpy(), c_den)
    assert torch.equal(A.exact_afa_reference(q, k, v, 0.5, causal), out)
    ref, rden = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, causal, return_denominator=True)
    f3, _ = A.pallas_afa_forward(q, k, v, 0.5, causal, block_q=L, block_k=L, return_denominator=True)
    e64, e_d, e_f3 = normwise(to_f64(out), ref), normwise(to_f64(den), rden), normwise(to_f64(out), to_f64(f3))
    print(f"{dtype} {shape} causal={causal}: vs float64 {e64:.2e} (d_total {e_d:.2e}); "
          f"vs the fp32-internal forward {e_f3:.2e}")
    # how far the reference's own formula is from float64: a weight rounded op by op carries up
    # to about 39 units of the dtype's half-ulp (8 from the score's rounding through
    # d rho^8 / rho^8 = 8 ds / sqrt(1 + s^2), rho's ~3 roundings multiplied by 8 through the three
    # squarings, and 7 from the squarings themselves): 7.6% in bf16, 1.9% in fp16.  A causal row
    # with few keys has its d_total set by one or two weights (measured up to 4.1e-2 in bf16); the
    # output, a ratio of sums of the same rounded weights, stays within the reference's bf16
    # parity gate (4e-2; measured up to 2.8e-2)
    assert e64 <= (4e-2 if dtype == torch.bfloat16 else 1e-2)
    assert e_d <= (8e-2 if dtype == torch.bfloat16 else 2e-2)


# ------------------------------------------------------------------------------ A-Softmax / octic
@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-13), (torch.float32, 2e-5), (torch.bfloat16, 1.6e-2)])
@pytest.mark.parametrize("n", [1, 3, 7, 64])
def test_algebraic_softmax_matches_golden(gold, n, dtype, tol):
    sink, eps = gold[f"asm_{n}_cfg"]
    x = _t(gold[f"asm_{n}_x"][None, :], dtype)
    y = A.algebraic_softmax(x, float(sink), float(eps))
    assert y.dtype == dtype
    assert normwise(to_f64(y)[0], gold[f"asm_{n}_y"]) <= tol


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-12), (torch.float32, 2e-5)])
def test_algebraic_softmax_forward_and_vjp(dtype, tol):
    rng = np.random.default_rng(81)
    x = torch.from_numpy(rng.standard_normal((3, 37, 1000)) * 3).to(dtype).to(DEV).requires_grad_(True)
    g = torch.from_numpy(rng.standard_normal((3, 37, 1000))).to(dtype).to(DEV)
    for sink in (0.0, 0.5, 1.0):
        y = A.algebraic_softmax(x, sink)
        assert normwise(to_f64(y), O.asoftmax(to_f64(x), sink)) <= tol
        (dx,) = torch.autograd.grad(y, x, g)
        assert normwise(to_f64(dx), O.asoftmax_vjp(to_f64(x), to_f64(g), sink)) <= tol * 10


@pytest.mark.parametrize("shape", [(16, 2048), (8, 4096), (5, 520), (3, 8), (2, 6000)])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-5), (torch.bfloat16, 1.6e-2), (torch.float16, 4e-3)])
def test_algebraic_softmax_row_lengths(shape, dtype, tol):
    """Row lengths that take the register-resident row kernels (up to 4096 forward, 2048 VJP)
    and ones that fall back to the multi-pass kernels (not a multiple of the chunk width, longer
    rows)."""
    rng = np.random.default_rng(shape[1])
    x = torch.from_numpy(rng.standard_normal(shape) * 2).to(dtype).to(DEV).requires_grad_(True)
    g = torch.from_numpy(rng.standard_normal(shape)).to(dtype).to(DEV)
    y = A.algebraic_softmax(x, 0.5)
    assert normwise(to_f64(y), O.asoftmax(to_f64(x), 0.5)) <= tol
    (dx,) = torch.autograd.grad(y, x, g)
    assert normwise(to_f64(dx), O.asoftmax_vjp(to_f64(x), to_f64(g), 0.5)) <= tol * 10


def test_algebraic_softmax_jacobian_at_zero():
    eps = 1e-5
    x = torch.zeros(1, 2, dtype=torch.float64, device=DEV, requires_grad=True)
    J = torch.stack([torch.autograd.grad(A.algebraic_softmax(x, 0.0, eps)[0, i], x)[0][0] for i in range(2)])
    np.testing.assert_allclose(to_f64(J) * np.sqrt(eps), [[2, -2], [-2, 2]], rtol=1e-10)


@pytest.mark.parametrize("n", [1, 64, 4096])
def test_algebraic_softmax_simplex_extremes(n):
    rng = np.random.default_rng(n)
    x = torch.from_numpy(rng.choice([-1e15, 1e15], size=(4, n))).float().to(DEV)
    p = A.algebraic_softmax(x, 0.5)
    assert torch.isfinite(p).all() and (p >= 0).all() and (p.sum(-1) <= 1 + 1e-5).all()


@pytest.mark.parametrize("dtype,tol", [(torch.float64, 1e-14), (torch.float32, 3e-6)])
def test_octic_kernel_and_derivative(gold, dtype, tol):
    x = _t(gold["rho8_x"], dtype).requires_grad_(True)
    y = A.octic_kernel(x)
    np.testing.assert_allclose(to_f64(y), gold["rho8_y"], rtol=tol)
    (dx,) = torch.autograd.grad(y.sum(), x)
    np.testing.assert_allclose(to_f64(dx), O.rho8_derivative(to_f64(x)), rtol=tol * 4)


@pytest.mark.parametrize("dtype,tol,rtol", [(torch.float64, 1e-14, 1e-15), (torch.float32, 3e-6, 1e-6)])
def test_octic_pair_with_r(gold, dtype, tol, rtol):
    """_kernel returns (rho^8, r) from one evaluation (src/attention.py:18-26): rho^8 against the
    40-digit fixtures and bitwise equal to octic_kernel, r against 1/sqrt(1 + x^2), and the known
    answer rho(2)^8 = 51841 + 23184 sqrt(5), r(2) = 1/sqrt(5) (tests/test_attention.py:34)."""
    from algebraic_intelligence_amd.attention import _kernel
    x = _t(gold["rho8_x"], dtype)
    k, r = _kernel(x)
    assert k.dtype == dtype and r.dtype == dtype and k.shape == x.shape
    np.testing.assert_allclose(to_f64(k), gold["rho8_y"], rtol=tol)
    assert torch.equal(k, A.octic_kernel(x))
    xf = to_f64(x)
    np.testing.assert_allclose(to_f64(r), 1.0 / np.sqrt(1.0 + xf * xf), rtol=rtol)
    k2, r2 = _kernel(torch.tensor([2.0, -2.0], dtype=dtype, device=DEV))
    exact = 51841.0 + 23184.0 * np.sqrt(5.0)
    np.testing.assert_allclose(to_f64(k2), [exact, 1.0 / exact], rtol=tol)
    np.testing.assert_allclose(to_f64(r2), [1.0 / np.sqrt(5.0)] * 2, rtol=rtol)


def test_octic_pair_promotes_16_bit_input():
    """bf16 / fp16 input: the pair is evaluated and returned in fp32, as on the fp32 upcast."""
    from algebraic_intelligence_amd.attention import _kernel
    x = torch.linspace(-40, 40, 4001, device=DEV)
    for dt in (torch.bfloat16, torch.float16):
        xh = x.to(dt)
        k, r = _kernel(xh)
        kf, rf = _kernel(xh.float())
        assert k.dtype == torch.float32 and torch.equal(k, kf) and torch.equal(r, rf)


# ------------------------------------------------------------------------------ Cayley rotary
def _f32_recurrence(w, L, base=10000.0, default=False):
    """The table recurrence with every operation rounded in float32, in the kernel's order."""
    one, two = np.float32(1), np.float32(2)
    if default:
        pairs = len(w)
        b = np.float32(base)
        alpha = (b * (one / np.sqrt(b)) - one) / np.float32(max(pairs - 1, 1))
        lin = one + alpha * np.arange(pairs, dtype=np.float32)
        w = one / (lin * lin)
    w = np.asarray(w, dtype=np.float32)
    w2 = w * w
    cb, sb = (one - w2) / (one + w2), (two * w) / (one + w2)
    c, s = np.ones_like(w), np.zeros_like(w)
    C_, S_ = np.empty((L, len(w)), np.float32), np.empty((L, len(w)), np.float32)
    for m in range(L):
        C_[m], S_[m] = c, s
        cn, sn = cb * c - sb * s, sb * c + cb * s
        r = one / np.sqrt(cn * cn + sn * sn)
        c, s = cn * r, sn * r
    return C_, S_


@pytest.mark.parametrize("name", ["cayley_default", "cayley_c3"])
def test_cayley_tables_fp64_match_golden(gold, name):
    cos, sin, w = gold[f"{name}_cos"], gold[f"{name}_sin"], gold[f"{name}_freqs"]
    freqs = None if name == "cayley_default" else w
    rot = A.build_cayley_rotary_matrix(2 * cos.shape[1], cos.shape[0], freqs=freqs, dtype=torch.float64,
                                       device=DEV)
    np.testing.assert_allclose(to_f64(rot.c), cos, atol=1e-13)
    np.testing.assert_allclose(to_f64(rot.s), sin, atol=1e-13)


@pytest.mark.parametrize("default", [False, True])
def test_cayley_tables_fp32_bitwise_and_c3_accuracy(default):
    D, L = 64, 4096
    w = 10000.0 ** (-2.0 * np.arange(D // 2) / D)
    rot = A.build_cayley_rotary_matrix(D, L, freqs=None if default else w, device=DEV)
    c_ref, s_ref = _f32_recurrence(w, L, default=default)
    assert np.array_equal(rot.c.cpu().numpy(), c_ref)
    assert np.array_equal(rot.s.cpu().numpy(), s_ref)
    c64, s64 = O.cayley_tables(D, L, freqs=None if default else w)
    assert np.abs(to_f64(rot.c) - c64).max() < 5e-4
    assert np.abs(to_f64(rot.s) - s64).max() < 5e-4


@pytest.mark.parametrize("layout", ["bhld", "bld", "ld"])
@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-6), (torch.bfloat16, 8e-3)])
def test_apply_ago_rotations(layout, dtype, tol):
    """bf16: the tables and the result are each rounded once to bf16 (2^-9 relative)."""
    shape = {"bhld": (2, 3, 40, 16), "bld": (2, 40, 16), "ld": (40, 16)}[layout]
    rng = np.random.default_rng(91)
    q, k = (torch.from_numpy(rng.standard_normal(shape)).to(dtype).to(DEV) for _ in range(2))
    rot = A.build_cayley_rotary_matrix(16, 64, device=DEV)
    qr, kr = A.apply_ago_rotations(q, k, rot)
    c, s = to_f64(rot.c), to_f64(rot.s)  # the fp32 tables themselves are pinned above
    seq_axis = len(shape) - 2
    rq, rk = O.ago_apply(to_f64(q), to_f64(k), c, s, seq_axis)
    assert qr.dtype == dtype
    assert normwise(to_f64(qr), rq) <= tol and normwise(to_f64(kr), rk) <= tol


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-6), (torch.bfloat16, 8e-3)])
def test_model_rotation_helpers(dtype, tol):
    """The model's own rotation calls (src/model.py:263-264,355-357): _align_param, then
    _rotate_tensor on (B, H, T, D) q, against the float64 oracle and bitwise against
    rotate_tensor; an unaligned (T, D/2) table broadcasts the same way, and a one-row table
    rotates every position by that row.  bf16: the tables and the result are each rounded once
    (2^-9 relative per element)."""
    from algebraic_intelligence_amd.attention import _align_param, _rotate_tensor
    shape = (2, 3, 40, 16)
    rng = np.random.default_rng(93)
    q = torch.from_numpy(rng.standard_normal(shape)).to(dtype).to(DEV)
    rot = A.build_cayley_rotary_matrix(16, 64, device=DEV)
    c, s = _align_param(rot.c, shape, seq_axis=2), _align_param(rot.s, shape, seq_axis=2)
    y = _rotate_tensor(q, c, s)
    ref = O.rotate_pairs(to_f64(q), to_f64(rot.c), to_f64(rot.s))
    assert y.dtype == dtype and y.shape == q.shape
    assert normwise(to_f64(y), ref) <= tol
    assert torch.equal(y, A.rotate_tensor(q, rot.c, rot.s, 2))
    assert torch.equal(_rotate_tensor(q, rot.c[:40], rot.s[:40]), y)
    one_c, one_s = rot.c[5:6], rot.s[5:6]
    y1 = _rotate_tensor(q, one_c, one_s)
    ref1 = O.rotate_pairs(to_f64(q), np.repeat(to_f64(one_c), 40, 0), np.repeat(to_f64(one_s), 40, 0))
    assert normwise(to_f64(y1), ref1) <= tol


def test_rotation_vjp_is_transpose():
    x = torch.randn(2, 3, 40, 16, dtype=torch.float64, device=DEV, requires_grad=True)
    rot = A.build_cayley_rotary_matrix(16, 40, dtype=torch.float64, device=DEV)
    g = torch.randn_like(x)
    y = A.rotate_tensor(x, rot.c, rot.s, 2)
    (dx,) = torch.autograd.grad(y, x, g)
    ref = O.rotate_pairs(to_f64(g), to_f64(rot.c), -to_f64(rot.s))
    assert normwise(to_f64(dx), ref) <= 1e-14


def test_fused_rotation_equals_explicit_rotation_fp32():
    q, k, v = make_qkv((1, 2, 256, 64), torch.float32, seed=101)
    rot = A.build_cayley_rotary_matrix(64, 256, freqs=10000.0 ** (-2.0 * np.arange(32) / 64), device=DEV)
    fused = A.pallas_afa_forward(q, k, v, causal=True, rotary_params=rot)
    qr, kr = A.apply_ago_rotations(q, k, rot)
    explicit = A.pallas_afa_forward(qr, kr, v, causal=True)
    assert normwise(to_f64(fused), to_f64(explicit)) <= 1e-6


@pytest.mark.parametrize("shape,rot", [((1, 2, 65536, 64), True), ((1, 1, 32768, 128), False)])
def test_long_sequence_prefix_locality(shape, rot):
    """Causal attention at long lengths (the 256-query kernel at 65536 keys, the 128-query
    pipelined kernel at head_dim 128): the first 512 outputs and the first 512 rows of dq depend
    only on the first 512 keys, so they match the 512-long problem, which the C contract checks.
    dk and dv, which depend on every later query, must be finite; the default schedule is also
    checked against the fully fused kernel over the whole length."""
    from algebraic_intelligence_amd import _lib
    B, H, L, D = shape
    P = 512
    q, k, v = make_qkv(shape, torch.bfloat16, seed=L + D)
    g = make_qkv(shape, torch.bfloat16, seed=L + D + 1)[0]
    freqs = 10000.0 ** (-2.0 * np.arange(D // 2) / D)
    rot_l = A.build_cayley_rotary_matrix(D, L, freqs=freqs) if rot else None
    rot_p = A.build_cayley_rotary_matrix(D, P, freqs=freqs) if rot else None
    out, den = A.afa._launch_fwd(q, k, v, 0.5, True, None, rot_l, 0, True)
    out_s, _ = A.afa._launch_fwd(q, k, v, 0.5, True, None, rot_l, _lib.FLAG_SIMPLE_SCHEDULE, True)
    assert torch.isfinite(out.float()).all() and torch.isfinite(den).all()
    assert normwise(to_f64(out), to_f64(out_s)) <= 8e-3
    qp, kp, vp, gp = (t[:, :, :P].contiguous() for t in (q, k, v, g))
    out_p, den_p = A.afa._launch_fwd(qp, kp, vp, 0.5, True, None, rot_p, 0, True)
    assert normwise(to_f64(out[:, :, :P]), to_f64(out_p)) <= 8e-3
    assert normwise(to_f64(den[:, :, :P]), to_f64(den_p)) <= 1e-5
    tabs = None if rot_p is None else (rot_p.c.detach().cpu().numpy().astype(np.float32),
                                        rot_p.s.detach().cpu().numpy().astype(np.float32))
    c_out, _ = C.afa_fwd(to_bits(qp), to_bits(kp), to_bits(vp), C.DT_BF16, 0.5, True, None, tabs)
    assert normwise(to_f64(out_p), C.to_f32(c_out, C.DT_BF16)) <= 8e-3
    rt = None if rot_l is None else (rot_l.c.contiguous(), rot_l.s.contiguous())
    rtp = None if rot_p is None else (rot_p.c.contiguous(), rot_p.s.contiguous())
    dq, dk, dv = _bwd_flags(q, k, v, out, den, g, True, None, 0, rot=rt)
    for t in (dq, dk, dv):
        assert torch.isfinite(t.float()).all()
    pq, pk, pv = _bwd_flags(qp, kp, vp, out_p, den_p, gp, True, None, 0, rot=rtp)
    e = normwise(to_f64(dq[:, :, :P]), to_f64(pq))
    print(f"{shape} rot={rot}: out prefix vs 512-long {normwise(to_f64(out[:, :, :P]), to_f64(out_p)):.2e}, "
          f"dq prefix {e:.2e}")
    assert e <= 1e-2


@pytest.mark.parametrize("shape,rot", [((2, 16, 8192, 128), False), ((8, 12, 4096, 64), True)])
def test_backward_linearity_full_size(shape, rot):
    """At the full C5 and C3 (Cayley tables) sizes, the backward is linear in the output
    cotangent g: doubling g doubles dq, dk and dv bit for bit (every product and the bf16
    rounding of ds scale exactly by 2), and for g1, g2 whose sum bf16 holds exactly,
    d(g1 + g2) = d(g1) + d(g2) up to the rounding of ds."""
    B, H, L, D = shape
    q, k, v = make_qkv(shape, torch.bfloat16, seed=L + D + 5)
    rt = None
    rot_obj = None
    if rot:
        rot_obj = A.build_cayley_rotary_matrix(D, L, freqs=10000.0 ** (-2.0 * np.arange(D // 2) / D))
        rt = (rot_obj.c.contiguous(), rot_obj.s.contiguous())
    out, den = A.afa._launch_fwd(q, k, v, 0.5, True, None, rot_obj, 0, True)
    gen = torch.Generator(device=DEV).manual_seed(L)
    # multiples of 1/16 in [-4, 4]: sums of two stay exact in bf16
    g1 = (torch.randint(-64, 65, shape, generator=gen, device=DEV).float() / 16).to(torch.bfloat16)
    g2 = (torch.randint(-64, 65, shape, generator=gen, device=DEV).float() / 16).to(torch.bfloat16)
    g12 = (g1.float() + g2.float()).to(torch.bfloat16)
    assert torch.equal(g12.float(), g1.float() + g2.float())
    d1 = _bwd_flags(q, k, v, out, den, g1, True, None, 0, rot=rt)
    d2 = _bwd_flags(q, k, v, out, den, g2, True, None, 0, rot=rt)
    d12 = _bwd_flags(q, k, v, out, den, g12, True, None, 0, rot=rt)
    dd = _bwd_flags(q, k, v, out, den, (2 * g1.float()).to(torch.bfloat16), True, None, 0, rot=rt)
    for name, a1, a2, a12, a2x in zip(("dq", "dk", "dv"), d1, d2, d12, dd):
        assert torch.isfinite(a12.float()).all(), name
        assert torch.equal(a2x.float(), 2 * a1.float()), name
        e = normwise(to_f64(a12), to_f64(a1) + to_f64(a2))
        print(f"{shape} rot={rot} {name}: d(g1+g2) vs d(g1)+d(g2) {e:.2e}")
        assert e <= 1e-2, name
