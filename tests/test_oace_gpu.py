"""GPU parity of the OACE loss head (include/afa.h oace_*) against the 40-digit golden fixtures
and the float64 oracle (oracle/oace_oracle.py): fused_oace_softmax_loss (src/model.py:180-240)
and fused_linear_oace (src/kernels/pallas_oace.py:59-293), forward and backward, on the MFMA path
(bf16/fp16) and the generic path (every dtype), in both weight layouts.

Tolerances (normwise max error, the reference's metric): fp64 1e-10 against 40-digit values;
fp32 and the bf16/fp16 loss (inputs exact, fp32 arithmetic) 2e-5; bf16/fp16 gradients 2e-2
(dz and the outputs are rounded to the element type; the reference gates bf16 at 2e-2)."""
import os

import numpy as np
import pytest
import torch

import algebraic_intelligence_amd as A
from algebraic_intelligence_amd import _lib
from oracle import oace_oracle as O
from tests.helpers import normwise, to_f64

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "oace_golden.npz"))
LOW = (torch.bfloat16, torch.float16)


def _t(x, dtype):
    return torch.from_numpy(np.asarray(x, dtype=np.float64)).to(dtype).to(DEV)


def _case(N, d, V, dtype, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    h = _t(rng.standard_normal((N, d)) * scale, dtype)
    w = _t(rng.standard_normal((d, V)) * scale, dtype)
    t = torch.from_numpy(rng.integers(0, V, size=N)).to(DEV)
    return h, w, t


def _fwd(h, w, t, flags=0, eps=100.0, gamma=2.0):
    loss, cache = A.fused_linear_oace_forward(h, w, t, eps, gamma, flags=flags)
    return loss, cache


def _grads(cache, g=1.0):
    dh, dw, _ = A.fused_linear_oace_backward(cache, torch.tensor(g, dtype=torch.float64, device=DEV))
    return dh, dw


def _tied(w):
    """The same (d, V) weight as the transposed view of a contiguous (V, d) embedding."""
    return w.t().contiguous().t()


# ------------------------------------------------------------------------------ golden
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", ["lin_small", "lin_d32"])
@pytest.mark.parametrize("tied", [False, True])
def test_linear_matches_golden(name, dtype, tied):
    h, w = _t(GOLD[f"{name}_h"], dtype), _t(GOLD[f"{name}_w"], dtype)
    if tied:
        w = _tied(w)
    t = torch.from_numpy(GOLD[f"{name}_t"]).to(DEV)
    eps, gamma = (float(x) for x in GOLD[f"{name}_cfg"])
    loss, cache = _fwd(h, w, t, eps=eps, gamma=gamma)
    rows = cache[3]
    ref = float(GOLD[f"{name}_loss"])
    tol_f = 1e-10 if dtype == torch.float64 else 2e-5
    tol_g = 1e-10 if dtype == torch.float64 else (2e-5 if dtype == torch.float32 else 2e-2)
    assert abs(float(loss) - ref) <= tol_f * abs(ref)
    assert normwise(to_f64(rows[:, 6]), GOLD[f"{name}_row_loss"]) <= tol_f
    assert normwise(to_f64(rows[:, 0]), GOLD[f"{name}_tau"]) <= tol_f
    dh, dw = _grads(cache)
    e_h = normwise(to_f64(dh), GOLD[f"{name}_dh"])
    e_w = normwise(to_f64(dw), GOLD[f"{name}_dw"])
    print(f"{name} {dtype} tied={tied}: loss {abs(float(loss) - ref) / abs(ref):.2e} dh {e_h:.2e} dw {e_w:.2e}")
    assert e_h <= tol_g and e_w <= tol_g


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
def test_softmax_loss_matches_golden(dtype):
    z = _t(GOLD["sm_z"], dtype).requires_grad_(True)
    t = torch.from_numpy(GOLD["sm_t"]).to(DEV)
    eps, gamma = (float(x) for x in GOLD["sm_cfg"])
    loss = A.fused_oace_softmax_loss(z, t, eps, gamma)
    loss.backward()
    ref = float(GOLD["sm_loss"])
    tol = 1e-10 if dtype == torch.float64 else 2e-5
    assert abs(float(loss) - ref) <= tol * abs(ref)
    assert normwise(to_f64(z.grad), GOLD["sm_dz"]) <= (tol if dtype != torch.bfloat16 else 1e-2)


# ------------------------------------------------------------------------------ oracle
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(5, 203), (4, 50257), (33, 1000)])
def test_softmax_loss_vs_oracle(shape, dtype):
    N, V = shape
    rng = np.random.default_rng(N + V)
    z = _t(rng.standard_normal((N, V)) * 30.0, dtype).requires_grad_(True)
    t = torch.from_numpy(rng.integers(0, V, size=N)).to(DEV)
    loss = A.fused_oace_softmax_loss(z, t)
    g = 0.7
    (loss * g).backward()
    ref, cache = O.oace_softmax_loss(to_f64(z), t.cpu().numpy())
    rz = O.oace_softmax_loss_vjp(cache, g)
    tol = 1e-12 if dtype == torch.float64 else 2e-5
    assert abs(float(loss) - ref) <= tol * abs(ref)
    assert normwise(to_f64(z.grad), rz) <= (tol if dtype != torch.bfloat16 else 1e-2)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
@pytest.mark.parametrize("shape", [(16, 32, 256), (10, 20, 203), (7, 48, 1031)])
@pytest.mark.parametrize("tied", [False, True])
def test_linear_generic_vs_oracle(shape, dtype, tied):
    N, d, V = shape
    h, w, t = _case(N, d, V, dtype, seed=N * d + V, scale=1.5)
    if tied:
        w = _tied(w)
    loss, cache = _fwd(h, w, t)
    dh, dw = _grads(cache, 1.3)
    hf, wf, tn = to_f64(h), to_f64(w), t.cpu().numpy()
    ref, rows = O.fused_linear_oace_forward(hf, wf, tn)
    rh, rw = O.fused_linear_oace_backward(hf, wf, tn, rows, g=1.3)
    tol = 1e-11 if dtype == torch.float64 else 2e-5
    assert abs(float(loss) - ref) <= tol * abs(ref)
    assert normwise(to_f64(cache[3][:, 5]), rows["radial"][:, 0]) <= (tol if dtype == torch.float64 else 1e-4)
    assert normwise(to_f64(dh), rh) <= (tol if dtype == torch.float64 else 1e-4)
    assert normwise(to_f64(dw), rw) <= (tol if dtype == torch.float64 else 1e-4)


@pytest.mark.parametrize("dtype", LOW)
@pytest.mark.parametrize("shape", [(8, 64, 300), (130, 96, 1000), (512, 768, 50257), (3, 32, 7)])
@pytest.mark.parametrize("tied", [False, True])
def test_linear_mfma_vs_oracle_and_generic(shape, dtype, tied):
    """The MFMA path (one GEMM sweep keeping the fp32 logits, the octic sums and dz from them,
    the MFMA GEMMs of oace_bwd_gemm.hip for dh and dW) against the float64 oracle on the same
    exact inputs and against the generic kernels (AFA_FLAG_GENERIC); (512, 768, 50257) is the
    reference benchmark's configuration (scripts/benchmark_kernels.py:118)."""
    N, d, V = shape
    h, w, t = _case(N, d, V, dtype, seed=N + d + V, scale=1.0 if dtype == torch.bfloat16 else 0.5)
    if tied:
        w = _tied(w)
    loss, cache = _fwd(h, w, t)
    dh, dw = _grads(cache, 1.0)
    gl, gcache = _fwd(h, w, t, flags=_lib.FLAG_GENERIC)
    gh, gw = _grads(gcache, 1.0)
    hf, wf, tn = to_f64(h), to_f64(w), t.cpu().numpy()
    ref, rows = O.fused_linear_oace_forward(hf, wf, tn)
    rh, rw = O.fused_linear_oace_backward(hf, wf, tn, rows, g=1.0)
    e_loss = abs(float(loss) - ref) / abs(ref)
    e_rows = normwise(to_f64(cache[3][:, 6]), rows["loss"][:, 0])
    e_h, e_w = normwise(to_f64(dh), rh), normwise(to_f64(dw), rw)
    e_gh, e_gw = normwise(to_f64(dh), to_f64(gh)), normwise(to_f64(dw), to_f64(gw))
    print(f"{shape} {dtype} tied={tied}: loss {e_loss:.2e} rows {e_rows:.2e} dh {e_h:.2e} dw {e_w:.2e} "
          f"vs generic loss {abs(float(loss) - float(gl)) / abs(float(gl)):.2e} dh {e_gh:.2e} dw {e_gw:.2e}")
    assert e_loss <= 2e-5 and e_rows <= 2e-5
    assert abs(float(loss) - float(gl)) <= 2e-5 * abs(float(gl))
    assert e_h <= 2e-2 and e_w <= 2e-2
    assert e_gh <= 2e-2 and e_gw <= 2e-2


@pytest.mark.parametrize("dtype", LOW)
@pytest.mark.parametrize("shape", [(130, 96, 1000), (512, 768, 50257), (3, 32, 7)])
@pytest.mark.parametrize("tied", [False, True])
def test_kept_logits_match_recomputed(shape, dtype, tied):
    """The forward that keeps the fp32 logits (octic sums from them) against the two-sweep forward
    (OACE_FLAG_RECOMPUTE_Z): the same sums in another order.  On one forward's row records, the
    backward's dz from the kept logits (OACE_FLAG_Z_READY) against the dz GEMM sweep: the same
    fp32 logits and arithmetic, so dh and dW are bitwise equal.  The gradients from the two
    forwards' records agree to one rounding of the element type."""
    N, d, V = shape
    h, w, t = _case(N, d, V, dtype, seed=N + 2 * d + V, scale=1.0 if dtype == torch.bfloat16 else 0.5)
    if tied:
        w = _tied(w)
    loss, cache = _fwd(h, w, t)
    rloss, rcache = _fwd(h, w, t, flags=A.oace.FLAG_RECOMPUTE_Z)
    assert abs(float(loss) - float(rloss)) <= 1e-6 * abs(float(rloss))
    assert normwise(to_f64(cache[3][:, :7]), to_f64(rcache[3][:, :7])) <= 1e-6
    dh, dw = _grads(cache, 1.0)
    stale_h = cache[:-1] + (-1,)  # as if h had changed: the backward recomputes z by the GEMM sweep
    gh, gw = _grads(stale_h, 1.0)
    assert torch.equal(dh, gh) and torch.equal(dw, gw)
    rh, rw = _grads(rcache, 1.0)
    # the two records differ in the order of their fp32 sums, so an output that sits at a rounding
    # boundary of the element type can round the other way: at most one unit in the last place of
    # the largest element (the element type's eps), and in few elements
    ulp = torch.finfo(dtype).eps
    for x, y in ((dh, rh), (dw, rw)):
        assert normwise(to_f64(x), to_f64(y)) <= ulp
        assert (x != y).double().mean().item() <= 1e-2


def test_backward_after_inputs_change_in_place():
    """The forward's kept logits are reused only while h and w_vocab are unchanged; after an
    in-place update of h the backward recomputes them with the current h."""
    h, w, t = _case(16, 64, 700, torch.bfloat16, seed=23)
    loss, cache = _fwd(h, w, t)
    h.mul_(0.5)
    dh, dw = _grads(cache, 1.0)
    hf, wf, tn = to_f64(h), to_f64(w), t.cpu().numpy()
    rows = {k: to_f64(cache[3][:, i:i + 1]) for i, k in enumerate(O.ROW_FIELDS)}
    rh, rw = O.fused_linear_oace_backward(hf, wf, tn, rows, g=1.0)
    assert normwise(to_f64(dh), rh) <= 2e-2 and normwise(to_f64(dw), rw) <= 2e-2


def test_linear_autograd_and_chunk_size():
    """fused_linear_oace through torch autograd; chunk_size does not change the result."""
    h, w, t = _case(6, 32, 500, torch.float32, seed=5)
    h.requires_grad_(True)
    w.requires_grad_(True)
    loss = A.fused_linear_oace(h, w, t, chunk_size=64)
    loss.backward()
    ref, rows = O.fused_linear_oace_forward(to_f64(h), to_f64(w), t.cpu().numpy())
    rh, rw = O.fused_linear_oace_backward(to_f64(h), to_f64(w), t.cpu().numpy(), rows)
    assert abs(float(loss) - ref) <= 2e-5 * abs(ref)
    assert normwise(to_f64(h.grad), rh) <= 1e-4 and normwise(to_f64(w.grad), rw) <= 1e-4
    assert float(A.fused_linear_oace(h.detach(), w.detach(), t, chunk_size=7)) == float(loss)
    with pytest.raises(ValueError):
        A.fused_linear_oace(h, w, t, chunk_size=0)


@pytest.mark.parametrize("dtype,flags", [(torch.float32, 0), (torch.bfloat16, 0), (torch.bfloat16, 2)])
def test_target_outside_vocabulary_gives_infinite_loss(dtype, flags):
    """As in the reference, a target that no vocabulary chunk contains leaves rho_t = 0."""
    h, w, t = _case(4, 32, 100, dtype, seed=9)
    t[1] = 100
    loss, cache = _fwd(h, w, t, flags=flags)
    assert torch.isinf(cache[3][1, 6]) and torch.isfinite(cache[3][[0, 2, 3], 6]).all()
    assert torch.isinf(loss)


def test_backward_after_weights_change_in_place():
    """The backward reuses the transposed weights the forward left in its workspace only while
    w_vocab is unchanged; an in-place update in between must not leave a stale copy in use."""
    h, w, t = _case(16, 64, 700, torch.bfloat16, seed=21)
    loss, cache = _fwd(h, w, t)
    w.mul_(0.5)
    dh, dw = _grads(cache, 1.0)
    # the forward's row records belong to the old weights; the backward recomputes the logits with
    # the current ones, exactly as the oracle backward does with those records
    hf, wf, tn = to_f64(h), to_f64(w), t.cpu().numpy()
    rows = {k: to_f64(cache[3][:, i:i + 1]) for i, k in enumerate(O.ROW_FIELDS)}
    rh, rw = O.fused_linear_oace_backward(hf, wf, tn, rows, g=1.0)
    assert normwise(to_f64(dh), rh) <= 2e-2 and normwise(to_f64(dw), rw) <= 2e-2


# ------------------------------------------------------------------------------ dW row strides
@pytest.mark.parametrize("tied,V,pad,off", [(False, 1000, 3, 0), (False, 517, 0, 0), (False, 517, 1, 1),
                                            (False, 50257, 0, 1), (False, 2049, 8, 1), (True, 700, 1, 1),
                                            (True, 700, 0, 0)])
def test_dw_rows_of_any_stride_and_start(tied, V, pad, off):
    """dW stored into rows of any stride (the weight's, odd ones included) starting at any 2-byte
    boundary: equal to the result in a buffer of the Python layer's own, and no element outside
    each row's dW columns changes.  Rows that are not dword aligned take the overlapping-tile stores whose seam dwords
    are written whole; this is where an element of a neighbouring tile, of the next row or of
    the padding would be overwritten if they were wrong."""
    N, d = 70, 64
    h, w, t = _case(N, d, V, torch.bfloat16, seed=V + 7 * pad + off)
    # the weight with the padded row stride; dW gets that stride too (include/afa.h).  The
    # reference is the Python layer's backward on the same weight (the same kernels: an odd
    # stride of a tied embedding is not matrix-core eligible), into a buffer of its own.
    rows_n, cols = (V, d) if tied else (d, V)
    wide = torch.zeros((rows_n, cols + pad), dtype=torch.bfloat16, device=DEV)
    wide[:, :cols] = w.t() if tied else w
    wv = wide[:, :cols].t() if tied else wide[:, :cols]
    _, cache = _fwd(h, wv, t)
    dh_ref, dw_ref = _grads(cache)
    hf, wop, tt, rows, gamma, _c, _s, flags, ws, _wv, _hv = cache
    ldw = cols + pad
    sentinel = 0x7F7B  # a bf16 NaN pattern no gradient takes
    store = torch.full((rows_n * ldw + off + 64,), sentinel, dtype=torch.int16, device=DEV)
    g = torch.ones((), dtype=rows.dtype, device=DEV)
    dh = torch.empty((N, d), dtype=torch.bfloat16, device=DEV)
    lay = A.oace.OACE_W_VD if tied else A.oace.OACE_W_DV
    rc = _lib.lib().oace_linear_bwd(_lib.dtype_code(torch.bfloat16), N, d, V, hf.data_ptr(), hf.stride(0),
                                    wop.data_ptr(), lay, ldw, tt.data_ptr(), float(gamma), rows.data_ptr(),
                                    g.data_ptr(), dh.data_ptr(), store.data_ptr() + 2 * off, flags, ws.data_ptr(),
                                    ws.numel(), _lib.stream_ptr(torch.device(DEV)))
    _lib.check(rc, "oace_linear_bwd")
    torch.cuda.synchronize()
    mat = store[off:off + rows_n * ldw].view(rows_n, ldw)
    got = mat[:, :cols].view(torch.bfloat16)
    ref = dw_ref.t() if tied else dw_ref
    assert normwise(to_f64(got), to_f64(ref)) <= 1e-6
    assert normwise(to_f64(dh), to_f64(dh_ref)) <= 1e-6
    assert bool((mat[:, cols:] == sentinel).all()), "padding columns changed"
    assert bool((store[:off] == sentinel).all()) and bool((store[off + rows_n * ldw:] == sentinel).all())
