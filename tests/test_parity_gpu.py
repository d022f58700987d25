"""GPU parity at the full BASELINE.json workloads and of the numeric corner cases.

* C4 (B=32 H=4 L=1024 D=64, causal, default Cayley tables, q,k,v ~ 0.5 N(0,1), seeds 0..7)
  in fp32 and bf16: every head against the C restatement of the dtype contract, two heads per
  seed against float64 (scripts/run_phase6_tpu.py:54-144, scripts/phase6_experiments.py:66-132).
* C5 (B=2 H=16 L=8192 D=128, bf16, causal) forward and backward at full length against the
  contract on two heads, the first 2048 rows against float64, and 36 rows spread over the whole
  length against float64 (out, d, dq of those query rows; dk, dv of those key rows).
* tiled_afa_forward against float64 with valid_seq_len and return_denominator
  (src/kernels/pallas_afa.py:330-406).
* The denominator of the bf16 path is the fp32 row sum of the unrounded weights
  (pallas_afa.py:127-139): on bf16 inputs it matches float64 to 1e-5, which a sum of the
  bf16-rounded weights (relative error up to 2^-9 each) would not.
* Rows whose every score is very negative, where the branch-free rho^8 cancels: per row against
  float64, for scores in [-31, -30] (inside the fast-rho bound |s| <= 32, where the branch-free
  form runs), in [-2000, -1000] and near -1e6 (outside it: the two-branch form runs).
Every call goes through the C ABI (afa_fwd / afa_bwd).
"""
import numpy as np
import pytest
import torch

from oracle import afa_oracle as O
from oracle import contract as C
from tests.helpers import make_qkv, normwise, oracle_contract, to_bits, to_f64

pytestmark = pytest.mark.gpu

import algebraic_intelligence_amd as A  # noqa: E402
from algebraic_intelligence_amd import _lib  # noqa: E402

DEV = "cuda"


def _fwd(q, k, v, causal=True, valid=None, rotary=None, flags=0):
    return A.afa._launch_fwd(q, k, v, 0.5, causal, valid, rotary, flags, True)


def _ulp_tol(dt):
    """One output rounding flip in the top binade: 2^-7 of max|ref| in bf16, 2^-10 in fp16; fp32
    outputs of two fp32 accumulation orders agree far below the 1e-5 bound."""
    return 8e-3 if dt == torch.bfloat16 else 4e-3 if dt == torch.float16 else 1e-5


def _tables64(rot):
    """The device's fp32 Cayley tables promoted to float64 (the same rotation input for the
    float64 oracle; the tables' own accuracy is checked against the closed form elsewhere)."""
    return rot.c.double().cpu().numpy(), rot.s.double().cpu().numpy()


# ----------------------------------------------------------------------------------- C4
@pytest.mark.parametrize("seed", range(8))
@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_c4_full_size(dt, seed):
    """B=32 H=4 L=1024 D=64, causal, default Cayley rotary tables,
    q, k, v ~ 0.5 N(0, 1); fp32 within 1e-5 and bf16 within 2e-2 of float64, and every head
    within one output ulp of the contract."""
    B, H, L, D = 32, 4, 1024, 64
    q, k, v = make_qkv((B, H, L, D), dt, seed=seed, scale=0.5)
    rot = A.build_cayley_rotary_matrix(D, L)
    out, den = _fwd(q, k, v, rotary=rot)
    c_out, c_den = oracle_contract(q, k, v, 0.5, True, rotary=rot)
    e_c = normwise(to_f64(out), c_out)
    e_d = normwise(to_f64(den), c_den)
    heads = [(0, 0), (B - 1, H - 1)]
    e_r = 0.0
    for b, h in heads:
        ref, dref = O.afa_forward(to_f64(q[b, h]), to_f64(k[b, h]), to_f64(v[b, h]), 0.5, True,
                                  rotary=_tables64(rot), return_denominator=True)
        e_r = max(e_r, normwise(to_f64(out[b, h]), ref))
        # bf16: the contract rounds the rotated q and k to bf16 before the dot (the reference's
        # _rotate_tensor works in the input dtype), float64 does not; the contract check above
        # pins the denominator to 1e-5
        assert normwise(to_f64(den[b, h]), dref) <= (1e-5 if dt == torch.float32 else 2e-2)
    print(f"C4 {dt} seed {seed}: vs contract {e_c:.2e} (128 heads), denominator {e_d:.2e}, "
          f"vs fp64 {e_r:.2e} (2 heads)")
    assert np.isfinite(to_f64(out)).all()
    assert e_c <= _ulp_tol(dt)
    # both dtypes add the same fp32 weights of up to 1024 keys in another order than the contract:
    # measured up to 1.9e-6 (fp32) and 1.3e-6 (bf16) over the eight seeds
    assert e_d <= 1e-5
    assert e_r <= (1e-5 if dt == torch.float32 else 2e-2)


# ----------------------------------------------------------------------------------- C5
@pytest.fixture(scope="module")
def c5():
    """B=2 H=16 L=8192 D=128 bf16 causal, q, k, v, g ~ N(0, 1): the
    forward (out, d) and the analytical backward at full size."""
    shape = (2, 16, 8192, 128)
    q, k, v = make_qkv(shape, torch.bfloat16, seed=55)
    out, den = _fwd(q, k, v)
    g = make_qkv(shape, torch.bfloat16, seed=56)[0]
    dq, dk, dv = A.tiled_afa_backward(q, k, v, out, den, g, 0.5, True)
    torch.cuda.synchronize()
    return q, k, v, g, out, den, dq, dk, dv


C5_HEADS = [(0, 0), (1, 15)]


def test_c5_forward_full_length(c5):
    q, k, v, g, out, den = c5[:6]
    for b, h in C5_HEADS:
        sl = (slice(b, b + 1), slice(h, h + 1))
        c_out, c_den = oracle_contract(q[sl], k[sl], v[sl], 0.5, True)
        e_c, e_d = normwise(to_f64(out[sl]), c_out), normwise(to_f64(den[sl]), c_den)
        # causal: the first 2048 rows are the 2048-long problem, small enough for float64
        n = 2048
        ref = O.afa_forward(to_f64(q[b, h, :n]), to_f64(k[b, h, :n]), to_f64(v[b, h, :n]), 0.5, True)
        e_r = normwise(to_f64(out[b, h, :n]), ref)
        print(f"C5 forward head ({b},{h}): vs contract {e_c:.2e}, denominator {e_d:.2e}, "
              f"first {n} rows vs fp64 {e_r:.2e}")
        # the denominator sums up to 8192 fp32 weights in another order than the contract
        # (lane partials, a tree and a cross-lane add against a sequential sum): measured 6.3e-6
        # and 6.9e-6
        assert e_c <= _ulp_tol(torch.bfloat16) and e_d <= 3e-5 and e_r <= 2e-2


def test_c5_backward_full_length(c5):
    """dq, dk, dv of two full heads against the C restatement of the backward contract on the
    same (q, k, v, out, d, g); 1e-2 as the other bf16 backward checks."""
    q, k, v, g, out, den, dq, dk, dv = c5
    for b, h in C5_HEADS:
        sl = (slice(b, b + 1), slice(h, h + 1))
        cq, ck, cv = C.afa_bwd(to_bits(q[sl]), to_bits(k[sl]), to_bits(v[sl]), to_bits(out[sl]),
                               den[sl].detach().cpu().numpy().astype(np.float32).reshape(1, 1, -1),
                               to_bits(g[sl]), C.DT_BF16, True)
        for name, got, ref in (("dq", dq, cq), ("dk", dk, ck), ("dv", dv, cv)):
            e = normwise(to_f64(got[sl]), C.to_f32(ref, C.DT_BF16))
            print(f"C5 backward head ({b},{h}) {name}: vs contract {e:.2e}")
            assert np.isfinite(to_f64(got[sl])).all()
            assert e <= 1e-2, name


# rows spread over the whole length: the first and last, the 2048 boundary, and 28 more drawn
# once with a fixed seed
C5_ROWS = sorted({0, 1, 2047, 2048, 4095, 4096, 8190, 8191} |
                 set(np.random.default_rng(5).integers(0, 8192, 28).tolist()))


def test_c5_long_rows_fp64(c5):
    """Full-length rows of C5 against float64 (tests/helpers.py: afa_rows_forward64 and
    afa_rows_backward64, pinned against the oracle on the CPU): out and d of the sampled query
    rows, each over all its keys up to 8192; dq of the same rows and dk, dv of the same key rows,
    the key rows summed over all queries after them, from the GPU's own out and d as the
    backward takes them."""
    from tests.helpers import afa_rows_backward64, afa_rows_forward64

    q, k, v, g, out, den, dq, dk, dv = c5
    rows = C5_ROWS
    for b, h in C5_HEADS:
        qh, kh, vh, gh = (to_f64(t[b, h]) for t in (q, k, v, g))
        o_r, d_r = afa_rows_forward64(qh, kh, vh, rows)
        e_o = normwise(to_f64(out[b, h])[rows], o_r)
        e_d = float(np.max(np.abs(den[b, h, rows, 0].double().cpu().numpy() - d_r) / d_r))
        oh = to_f64(out[b, h])
        dh = den[b, h, :, 0].double().cpu().numpy()
        rq, rk, rv = afa_rows_backward64(qh, kh, vh, gh, oh, dh, rows, rows)
        e_q = normwise(to_f64(dq[b, h])[rows], rq)
        e_k = normwise(to_f64(dk[b, h])[rows], rk)
        e_v = normwise(to_f64(dv[b, h])[rows], rv)
        print(f"C5 head ({b},{h}), {len(rows)} full-length rows vs fp64: out {e_o:.2e}, d {e_d:.2e} (max rel), "
              f"dq {e_q:.2e}, dk {e_k:.2e}, dv {e_v:.2e}")
        # measured: out 2.9e-3 and 3.7e-3, d 4.9e-7 and 5.7e-7, dq / dk / dv 2.6e-3 to 3.2e-3 (the bf16
        # rounding of the outputs and of the P, W and dS operands); bounds about four times that
        assert e_o <= 1.5e-2 and e_d <= 3e-6
        assert max(e_q, e_k, e_v) <= 1.5e-2


# ----------------------------------------------------------------------------------- key split
@pytest.mark.parametrize("shape,causal,valid,dt,rotary", [
    ((1, 8, 2048, 64), True, None, torch.bfloat16, False),
    ((1, 8, 2048, 64), False, 1500, torch.bfloat16, False),
    ((2, 4, 2048, 128), True, None, torch.bfloat16, True),
    ((1, 4, 2048, 96), True, 1900, torch.float16, False),
    ((1, 2, 1536, 32), False, None, torch.bfloat16, True),
])
def test_key_split_matches_contract(shape, causal, valid, dt, rotary):
    """Grids with few 128-query blocks split the long key ranges over several workgroups, whose
    fp32 partials the last one to finish adds up.  Such a call reserves workspace beyond the
    guard's key bounds (B H ceil(L/64) floats, and the rotated k with rotary tables); its output
    and denominator match the C restatement of the contract as unsplit calls do, also where
    valid_len leaves some parts without keys."""
    B, H, L, D = shape
    q, k, v = make_qkv(shape, dt, seed=61 + D, scale=0.5)
    rot = A.build_cayley_rotary_matrix(D, L) if rotary else None
    ws = _lib.lib().afa_fwd_workspace_size(_lib.dtype_code(dt), B, H, L, D, int(rotary))
    base = -(-B * H * ((L + 63) // 64) * 4 // 256) * 256
    if rotary:
        base += -(-B * H * L * D * 2 // 256) * 256
    assert ws > base, "no key split planned for this shape"
    out, den = _fwd(q, k, v, causal=causal, valid=valid, rotary=rot)
    c_out, c_den = oracle_contract(q, k, v, 0.5, causal, valid, rotary=rot)
    e, e_d = normwise(to_f64(out), c_out), normwise(to_f64(den), c_den)
    print(f"{shape} causal={causal} valid={valid} {dt} rotary={rotary}: workspace {ws} B, vs contract {e:.2e}, "
          f"denominator {e_d:.2e}")
    assert np.isfinite(to_f64(out)).all()
    # the split adds each part's fp32 row sums in part order: measured 1.1e-6 to 1.6e-6
    assert e <= _ulp_tol(dt) and e_d <= 1e-5
    # the parts are added in part order whichever finishes last: calls are bit for bit repeatable
    out2, den2 = _fwd(q, k, v, causal=causal, valid=valid, rotary=rot)
    assert torch.equal(out, out2) and torch.equal(den, den2)


# ----------------------------------------------------------------------------------- tiled entry point
@pytest.mark.parametrize("dt,causal,valid", [(torch.float32, False, 200), (torch.bfloat16, True, 300),
                                             (torch.bfloat16, False, None), (torch.float16, True, 129)])
def test_tiled_afa_forward_vs_fp64(dt, causal, valid):
    """tiled_afa_forward with valid_seq_len and return_denominator against float64 (the masked
    keys carry no weight; d = sum of weights + sink, shaped (B, H, L, 1))."""
    # fp16: P is cast to fp16 for the PV product, where rho^8 overflows past |s| ~ 1.8; at scale
    # 0.5 the largest score of these heads stays below 1.6 (the reference's cast overflows alike)
    q, k, v = make_qkv((2, 3, 384, 64), dt, seed=77, scale=0.5 if dt == torch.float16 else 0.7)
    out, den = A.tiled_afa_forward(q, k, v, 0.5, causal, 128, 64, valid_seq_len=valid, return_denominator=True)
    ref, dref = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, causal, valid, return_denominator=True)
    assert out.shape == q.shape and den.shape == (2, 3, 384, 1) and den.dtype == torch.float32
    e, e_d = normwise(to_f64(out), ref), normwise(to_f64(den), dref)
    print(f"tiled_afa_forward {dt} causal={causal} valid={valid}: vs fp64 {e:.2e}, denominator {e_d:.2e}")
    assert e <= (1e-5 if dt == torch.float32 else 2e-2)
    assert e_d <= 1e-5


@pytest.mark.parametrize("shape", [(1, 4, 512, 64), (4, 200, 256, 64), (1, 4, 512, 128)])
def test_bf16_denominator_is_fp32_sum_of_unrounded_weights(shape):
    """bf16 inputs are exact in float64, so d = sum_j rho(s_ij)^8 + sink in float64 differs from
    the kernel's only by the fp32 scores and the fp32 sum (~1e-6 here).  Summing the weights after
    rounding them to bf16 (the PV operand) would be off by up to 2^-9 per weight; a check at 1e-5
    tells the two apart.  (4, 200, 256, 64) runs the 256-query head_dim-64 kernel, the others the
    pipelined one."""
    q, k, v = make_qkv(shape, torch.bfloat16, seed=91, scale=0.6)
    out, den = _fwd(q, k, v, causal=True)
    n = min(shape[1], 4)
    _, dref = O.afa_forward(to_f64(q[:, :n]), to_f64(k[:, :n]), to_f64(v[:, :n]), 0.5, True, return_denominator=True)
    e = normwise(to_f64(den[:, :n]), dref)
    # the same weights rounded to bf16 before the sum, for scale
    s = np.einsum("bhid,bhjd->bhij", to_f64(q[:, :n]), to_f64(k[:, :n])) / np.sqrt(shape[-1])
    w = np.where(np.tril(np.ones(s.shape[-2:], bool)), O.rho8(s), 0.0)
    wr = torch.from_numpy(w).to(torch.bfloat16).double().numpy()
    e_rounded = normwise(wr.sum(-1, keepdims=True) + 0.5, dref)
    print(f"{shape}: denominator vs fp64 {e:.2e} (sum of bf16-rounded weights: {e_rounded:.2e})")
    assert e <= 1e-5
    assert e_rounded > 1e-5


# ----------------------------------------------------------------------------------- negative rows
def _negative_rows(B, H, L, D, dt, c, seed, n_neg, hollow=False):
    """q, k, v where the first n_neg queries of every head score about -c sqrt(D) against every
    key: k_j = u + 0.02 n_j and q_i = -c u (1 + 0.002 m_i) with |u|^2 = D, so
    s_ij = q_i . k_j / sqrt(D) ~ -c |u|^2 / sqrt(D).  The other queries are N(0, 1).  hollow:
    u is zero on the first two elements of every 8 (the first 4 bytes of every 16-byte chunk)."""
    rng = np.random.default_rng(seed)
    u = rng.standard_normal(D)
    if hollow:
        u[np.arange(D) % 8 < 2] = 0.0
    u *= np.sqrt(D) / np.linalg.norm(u)
    k = u + 0.02 * rng.standard_normal((B, H, L, D))
    q = rng.standard_normal((B, H, L, D))
    q[:, :, :n_neg] = -c * u * (1.0 + 0.002 * rng.standard_normal((B, H, n_neg, 1)))
    v = rng.standard_normal((B, H, L, D))
    return [torch.from_numpy(x).to(dt).to(DEV) for x in (q, k, v)]


def _row_errors(out, ref):
    """Per row: max_d |out - ref| / max_d |ref|."""
    out, ref = to_f64(out), np.asarray(ref)
    return np.abs(out - ref).max(-1) / np.abs(ref).max(-1)


@pytest.mark.parametrize("c,label", [(3.8, "fast"), (190.0, "exact")])
@pytest.mark.parametrize("shape,flags", [((1, 2, 256, 64), 0), ((2, 384, 256, 64), 0), ((1, 2, 256, 128), 0),
                                         ((1, 2, 256, 64), _lib.FLAG_SIMPLE_SCHEDULE),
                                         ((1, 2, 256, 64), _lib.FLAG_EXACT_TAIL)])
def test_all_negative_rows_per_row(c, label, shape, flags):
    """Rows whose every score is negative and large: c = 3.8 puts them in [-31, -30] (inside the
    fast-rho bound |s| <= 32: the branch-free form runs, its per-weight error at most
    16 s^2 eta = 3.4e-3), c = 190 near -1500 (outside the bound: the two-branch form runs).  Each
    such row must match float64 to 1e-2 relative to the row itself (its weights are 1e-14 and
    smaller, far below what a tensor-wide norm sees).  Shapes: the pipelined head_dim-64 kernel,
    the 256-query one (768 workgroups), head_dim 128, the fully fused kernel, and the two-branch
    form forced everywhere."""
    B, H, L, D = shape
    n_neg = 40
    scale_c = c * 8.0 / np.sqrt(D)  # the same scores at head_dim 128
    q, k, v = _negative_rows(B, H, L, D, torch.bfloat16, scale_c, seed=31 + D, n_neg=n_neg)
    out, den = _fwd(q, k, v, causal=True, flags=flags)
    heads = [(0, 0), (B - 1, H - 1)]
    for b, h in heads:
        qh, kh, vh = to_f64(q[b, h]), to_f64(k[b, h]), to_f64(v[b, h])
        s = qh[:n_neg] @ kh.T / np.sqrt(D)
        lo, hi = s[np.tril(np.ones((n_neg, L), bool))].min(), s[np.tril(np.ones((n_neg, L), bool))].max()
        ref = O.afa_forward(qh, kh, vh, 0.5, True)
        err = _row_errors(out[b, h, :n_neg], ref[:n_neg])
        print(f"{shape} flags={flags} c={c} ({label}): scores of the negative rows in [{lo:.1f}, {hi:.1f}], "
              f"max|out| {np.abs(ref[:n_neg]).max():.1e}, worst per-row error {err.max():.2e}")
        if label == "fast":
            assert hi < 0 and lo > -32.0
        else:
            assert hi < -1000.0
        assert err.max() <= 1e-2
        # the other rows as usual
        assert normwise(to_f64(out[b, h, n_neg:]), ref[n_neg:]) <= 2e-2


def _identity_tables(L, D):
    """Rotary tables of the identity rotation (c = 1, s = 0): the rotary code paths (k rotated
    once per call, q at load, the backward's rotation pre-pass) run and the scores stay those of
    the unrotated rows."""
    return torch.ones(L, D // 2, device=DEV), torch.zeros(L, D // 2, device=DEV)


@pytest.mark.parametrize("rotary", [False, True], ids=["plain", "rotary"])
@pytest.mark.parametrize("shape,flags", [((1, 2, 256, 64), 0), ((2, 384, 256, 64), 0), ((1, 2, 256, 128), 0),
                                         ((1, 2, 256, 96), 0), ((1, 2, 256, 64), _lib.FLAG_SIMPLE_SCHEDULE)])
def test_guard_sees_every_feature(shape, flags, rotary):
    """Rows near s = -1500 whose q and k are zero on the first 4 bytes of every 16-byte chunk.
    The guard's row norms must cover every element: a norm that read one 4-byte word per chunk
    would be 0 here (a miscompile of __builtin_bit_cast on a vector element did exactly that),
    the guard would pass the branch-free rho^8, and its weights would be off by factors
    (|s| eta ~ rho(s) at |s| ~ 1500).  Per row against float64 to 1e-2, as above."""
    B, H, L, D = shape
    n_neg = 40
    q, k, v = _negative_rows(B, H, L, D, torch.bfloat16, 190.0 * 8.0 / np.sqrt(D), seed=41 + D, n_neg=n_neg,
                             hollow=True)
    out, den = _fwd(q, k, v, causal=True, rotary=_identity_tables(L, D) if rotary else None, flags=flags)
    for b, h in [(0, 0), (B - 1, H - 1)]:
        qh, kh, vh = to_f64(q[b, h]), to_f64(k[b, h]), to_f64(v[b, h])
        assert np.all(qh[:n_neg, np.arange(D) % 8 < 2] == 0.0)
        s = qh[:n_neg] @ kh.T / np.sqrt(D)
        ref = O.afa_forward(qh, kh, vh, 0.5, True)
        err = _row_errors(out[b, h, :n_neg], ref[:n_neg])
        print(f"{shape} flags={flags} rotary={rotary}: hollow rows, scores up to {s.max():.1f}, "
              f"worst per-row error {err.max():.2e}")
        assert s.max() < -1000.0
        assert err.max() <= 1e-2
        assert normwise(to_f64(out[b, h, n_neg:]), ref[n_neg:]) <= 2e-2


@pytest.mark.parametrize("rotary", [False, True], ids=["plain", "rotary"])
@pytest.mark.parametrize("D", [64, 128])
def test_guard_sees_every_feature_backward(D, rotary):
    """The backward's guards (dq: the wave's q rows against the key-block norms; dk/dv: the
    wave's k rows against the query-block norms) on hollow rows where every score is near -1500,
    so that dq, dk and dv all come from weights the branch-free form would get wrong: every row
    of each against the C restatement of the contract, relative to the row.  dv_j sums
    w_ij g_i / d_i and is well conditioned: 1e-2.  dq_i and dk_j sum ds_ij k_j and ds_ij q_i of
    both signs over near-parallel rows after ds is rounded to bf16, so single rounding flips of
    ds show: the contract itself is up to 0.1 (dq) and 0.2 (dk) off float64 per row on these
    inputs, and the bound against it is 3e-2.  Weights of the branch-free form would be off by
    factors."""
    B, H, L = 1, 2, 256
    q, k, v = _negative_rows(B, H, L, D, torch.bfloat16, 190.0 * 8.0 / np.sqrt(D), seed=43 + D, n_neg=L,
                             hollow=True)
    rot = _identity_tables(L, D) if rotary else None
    out, den = _fwd(q, k, v, causal=True, rotary=rot)
    g = make_qkv((B, H, L, D), torch.bfloat16, seed=44)[0]
    dq, dk, dv = A.tiled_afa_backward(q, k, v, out, den, g, 0.5, True, rotary_params=rot)
    cq, ck, cv = C.afa_bwd(to_bits(q), to_bits(k), to_bits(v), to_bits(out),
                           den.detach().cpu().numpy().astype(np.float32).reshape(B, H, L), to_bits(g), C.DT_BF16, True)
    s = to_f64(q[0, 0]) @ to_f64(k[0, 0]).T / np.sqrt(D)
    assert s[np.tril(np.ones((L, L), bool))].max() < -1000.0
    for name, got, ref in (("dq", dq, cq), ("dk", dk, ck), ("dv", dv, cv)):
        ref = C.to_f32(ref, C.DT_BF16).astype(np.float64)
        err = _row_errors(got.reshape(-1, D), ref.reshape(-1, D))
        print(f"backward D={D} rotary={rotary}, hollow rows near s = -1500: worst per-row {name} error {err.max():.2e}")
        assert np.isfinite(to_f64(got)).all()
        assert err.max() <= (1e-2 if name == "dv" else 3e-2), name


@pytest.mark.parametrize("shape", [(1, 2, 256, 64), (2, 384, 256, 64), (1, 2, 256, 128)])
def test_extreme_negative_scores(shape):
    """Scores near -1e6: rho(s)^8 ~ (2|s|)^-8 ~ 1e-50, so those rows are 0 in fp32.  The
    branch-free form would return weights of order (|s| * 2^-23)^8, up to O(1) at |s| ~ 1e7, and
    the row would come out near the mean of v; the guard routes such scores to the two-branch form."""
    B, H, L, D = shape
    n_neg = 40
    q, k, v = _negative_rows(B, H, L, D, torch.bfloat16, 1.5e5 * 8.0 / np.sqrt(D), seed=7, n_neg=n_neg)
    out, den = _fwd(q, k, v, causal=True)
    qh, kh = to_f64(q[0, 0]), to_f64(k[0, 0])
    s = qh[:n_neg] @ kh.T / np.sqrt(D)
    print(f"{shape}: scores of the negative rows down to {s.min():.2e}; max|out| of those rows "
          f"{np.abs(to_f64(out[:, :, :n_neg])).max():.2e}")
    assert s.max() < -5e5
    assert np.abs(to_f64(out[:, :, :n_neg])).max() <= 1e-30
    assert np.all(to_f64(den[:, :, :n_neg]) == 0.5)
    ref = O.afa_forward(to_f64(q[0, 0]), to_f64(k[0, 0]), to_f64(v[0, 0]), 0.5, True)
    assert normwise(to_f64(out[0, 0, n_neg:]), ref[n_neg:]) <= 2e-2


def test_negative_rows_backward_per_row():
    """The MFMA backward follows the same guard: rows near s = -1500 (two-branch form) give dq rows
    within 1e-2 of the C restatement of the contract relative to each row.  (Against float64 such
    rows are off by more: dq_i sums ds_ij k_j of both signs with near-parallel k_j, and the
    contract rounds ds to bf16 before that sum.  Had the branch-free rho run there, its weights
    would be off by factors, |s| eta ~ rho(s) at |s| ~ 1500.)"""
    B, H, L, D = 1, 2, 256, 64
    n_neg = 40
    q, k, v = _negative_rows(B, H, L, D, torch.bfloat16, 190.0, seed=33, n_neg=n_neg)
    out, den = _fwd(q, k, v, causal=True)
    g = make_qkv((B, H, L, D), torch.bfloat16, seed=34)[0]
    dq, dk, dv = A.tiled_afa_backward(q, k, v, out, den, g, 0.5, True)
    cq, ck, cv = C.afa_bwd(to_bits(q), to_bits(k), to_bits(v), to_bits(out),
                           den.detach().cpu().numpy().astype(np.float32).reshape(B, H, L), to_bits(g), C.DT_BF16, True)
    cq, ck, cv = (C.to_f32(x, C.DT_BF16).astype(np.float64) for x in (cq, ck, cv))
    err = _row_errors(dq[0, :, :n_neg].reshape(-1, D), cq[0, :, :n_neg].reshape(-1, D))
    print(f"backward, rows near s = -1500: worst per-row dq error against the contract {err.max():.2e}")
    assert err.max() <= 1e-2
    rq, rk, rv = O.afa_backward(to_f64(q), to_f64(k), to_f64(v), to_f64(g), 0.5, True)
    for name, got, cref, ref in (("dq", dq, cq, rq), ("dk", dk, ck, rk), ("dv", dv, cv, rv)):
        assert normwise(to_f64(got), cref) <= 1e-2, name
        assert normwise(to_f64(got), ref) <= 3e-2, name
