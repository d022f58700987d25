"""GPU parity of the fused AFA forward against the oracles (float64 numpy and the C contract).

Configurations follow BASELINE.json (C1..C5); tolerances are the north-star ones (fp32 1e-5,
bf16 2e-2 normwise against float64 on identical inputs) plus tighter bounds against the C
restatement of the kernel's dtype contract.  Every call goes through the C ABI (afa_fwd).
"""
import numpy as np
import pytest
import torch

from oracle import afa_oracle as O
from tests.helpers import make_qkv, normwise, oracle_contract, to_f64

pytestmark = pytest.mark.gpu

import algebraic_intelligence_amd as A  # noqa: E402
from algebraic_intelligence_amd import _lib  # noqa: E402


def _fwd(q, k, v, sink=0.5, causal=False, valid=None, rotary=None, flags=0):
    """Direct afa_fwd call returning (out, denominator)."""
    return A.afa._launch_fwd(q, k, v, sink, causal, valid, rotary, flags, True)


def _c3_freqs(D):
    """Config-3 Cayley parameters t_i = 10000^(-2i/D), computed in fp64 on the host."""
    return 10000.0 ** (-2.0 * np.arange(D // 2) / D)


# ----------------------------------------------------------------------------------- fp32 / fp64
def test_c1_fp32_noncausal_vs_fp64():
    q, k, v = make_qkv((1, 4, 256, 64), torch.float32, seed=0)
    out, den = _fwd(q, k, v)
    ref, dref = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, False, return_denominator=True)
    err = normwise(to_f64(out), ref)
    print("C1 fp32 err", err)
    assert err <= 1e-5
    assert normwise(to_f64(den), dref) <= 1e-5


@pytest.mark.parametrize("causal", [False, True])
def test_fp64_vs_oracle(causal):
    q, k, v = make_qkv((1, 2, 256, 64), torch.float64, seed=102)
    out, den = _fwd(q, k, v, causal=causal)
    ref, dref = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, causal, return_denominator=True)
    assert out.dtype == torch.float64 and den.dtype == torch.float64
    assert normwise(to_f64(out), ref) <= 1e-12
    assert normwise(to_f64(den), dref) <= 1e-12


# ----------------------------------------------------------------------------------- bf16 MFMA
@pytest.mark.parametrize("causal", [False, True])
def test_bf16_small_vs_contract_and_fp64(causal):
    q, k, v = make_qkv((1, 4, 256, 64), torch.bfloat16, seed=1)
    out, den = _fwd(q, k, v, causal=causal)
    c_out, c_den = oracle_contract(q, k, v, 0.5, causal)
    ref = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, causal)
    e_c, e_r = normwise(to_f64(out), c_out), normwise(to_f64(out), ref)
    print(f"bf16 small causal={causal}: vs contract {e_c:.3e} vs fp64 {e_r:.3e}")
    assert e_c <= 4e-3
    assert e_r <= 2e-2
    assert normwise(to_f64(den), c_den) <= 1e-5


def test_c2_bf16_causal():
    """C2: B=4 H=8 L=2048 D=64 bf16 causal, q,k,v ~ N(0,1)/sqrt(D)."""
    q, k, v = make_qkv((4, 8, 2048, 64), torch.bfloat16, seed=2, scale=1 / 8)
    out, den = _fwd(q, k, v, causal=True)
    c_out, c_den = oracle_contract(q, k, v, 0.5, True)
    e_c = normwise(to_f64(out), c_out)
    ref = O.afa_forward(to_f64(q[:1, :2]), to_f64(k[:1, :2]), to_f64(v[:1, :2]), 0.5, True)
    e_r = normwise(to_f64(out[:1, :2]), ref)
    print(f"C2: vs contract {e_c:.3e}, vs fp64 (2 heads) {e_r:.3e}")
    assert e_c <= 4e-3 and e_r <= 2e-2
    assert normwise(to_f64(den), c_den) <= 1e-5


def test_c2_outlier_keys():
    """C2 outlier variant: a seeded 1% of k rows per (b, h) multiplied by 20 (in fp32, rounded once)."""
    B, H, L, D = 4, 8, 2048, 64
    rng = np.random.default_rng(22)
    q, k, v = (rng.standard_normal((B, H, L, D)) / 8 for _ in range(3))
    k = k.astype(np.float32)
    for b in range(B):
        for h in range(H):
            rows = rng.choice(L, size=L // 100, replace=False)
            k[b, h, rows] *= np.float32(20.0)
    q, k, v = (torch.from_numpy(np.asarray(x)).to(torch.bfloat16).cuda() for x in (q, k, v))
    out, den = _fwd(q, k, v, causal=True)
    c_out, _ = oracle_contract(q, k, v, 0.5, True)
    ref = O.afa_forward(to_f64(q[:1, :2]), to_f64(k[:1, :2]), to_f64(v[:1, :2]), 0.5, True)
    e_c, e_r = normwise(to_f64(out), c_out), normwise(to_f64(out[:1, :2]), ref)
    print(f"C2 outlier: vs contract {e_c:.3e}, vs fp64 {e_r:.3e}")
    assert np.isfinite(to_f64(out)).all()
    assert e_c <= 4e-3 and e_r <= 2e-2


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_c3_fused_ago_full_size(dt):
    """C3 (north star): B=8 H=12 L=4096 D=64 causal, AGO with t_i = 10000^(-2i/D) fused; bf16,
    and fp16 on inputs scaled by 0.5 (fp16 weights of rho^8 overflow past |s| of about 4)."""
    B, H, L, D = 8, 12, 4096, 64
    q, k, v = make_qkv((B, H, L, D), dt, seed=3, scale=1.0 if dt == torch.bfloat16 else 0.5)
    rot = A.build_cayley_rotary_matrix(D, L, freqs=_c3_freqs(D))
    out, den = _fwd(q, k, v, causal=True, rotary=rot)
    c_out, c_den = oracle_contract(q, k, v, 0.5, True, rotary=rot)
    e_c = normwise(to_f64(out), c_out)
    # fp64 end-to-end on two heads: fp64 tables, fp64 rotation of the same bf16 inputs
    ct, st = O.cayley_tables(D, L, freqs=_c3_freqs(D))
    ref = O.afa_forward(to_f64(q[:1, :2]), to_f64(k[:1, :2]), to_f64(v[:1, :2]), 0.5, True, rotary=(ct, st))
    e_r = normwise(to_f64(out[:1, :2]), ref)
    e_d = normwise(to_f64(den), c_den)
    print(f"C3 {dt}: vs contract {e_c:.3e}, denominator {e_d:.3e}, vs fp64 (2 heads) {e_r:.3e}")
    assert e_c <= _ulp_tol(dt) and e_r <= 2e-2
    # the kernel and the contract add the same fp32 weights of up to 4096 keys in different
    # orders (lane partials and a tree against a sequential sum): measured 3e-6 to 4e-6
    assert e_d <= 2e-5


# ----------------------------------------------------------------------------------- invariants
def test_causal_prefix_invariance_is_bitwise():
    """Perturbing keys/values at positions >= 150 leaves outputs < 150 bit-identical
    (tests/test_pallas_afa.py:151-158)."""
    for dt in (torch.float32, torch.bfloat16):
        q, k, v = make_qkv((1, 1, 256, 64), dt, seed=104)
        y = A.pallas_afa_forward(q, k, v, causal=True)
        k2, v2 = k.clone(), v.clone()
        k2[:, :, 150:] += 10.0
        v2[:, :, 150:] += 10.0
        y2 = A.pallas_afa_forward(q, k2, v2, causal=True)
        assert torch.equal(y[:, :, :150], y2[:, :, :150])


@pytest.mark.parametrize("L,bq,bk", [(180, 128, 128), (190, 64, 128)])
def test_arbitrary_length_front_door(L, bq, bk):
    """algebraic_flash_attention on lengths that are not tile multiples
    (tests/test_pallas_afa.py:173-198)."""
    for dt, tol in ((torch.float32, 1e-5), (torch.bfloat16, 2e-2)):
        q, k, v = make_qkv((1, 2, L, 64), dt, seed=105)
        y = A.algebraic_flash_attention(q, k, v, block_q=bq, block_k=bk)
        ref = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, False)
        assert y.shape == q.shape
        assert normwise(to_f64(y), ref) <= tol


def test_valid_seq_len_masks_keys():
    q, k, v = make_qkv((2, 2, 256, 64), torch.bfloat16, seed=7)
    for causal in (False, True):
        y = A.pallas_afa_forward(q, k, v, causal=causal, valid_seq_len=200)
        c_out, _ = oracle_contract(q, k, v, 0.5, causal, valid_len=200)
        ref = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, causal, valid_len=200)
        assert normwise(to_f64(y), c_out) <= 4e-3
        assert normwise(to_f64(y), ref) <= 2e-2


def test_strided_model_layout_matches_contiguous():
    """q, k, v as (B, T, H, D).transpose(1, 2) views (the model's layout, src/model.py:257-260)."""
    B, T, H, D = 2, 512, 4, 64
    rng = np.random.default_rng(9)
    base = [torch.from_numpy(rng.standard_normal((B, T, H, D))).to(torch.bfloat16).cuda() for _ in range(3)]
    views = [x.transpose(1, 2) for x in base]
    y_view = A.pallas_afa_forward(*views, causal=True)
    y_cont = A.pallas_afa_forward(*[x.contiguous() for x in views], causal=True)
    assert torch.equal(y_view, y_cont)


def test_mfma_matches_generic_kernel():
    """The MFMA kernel and the generic kernel are independent implementations of one contract."""
    q, k, v = make_qkv((2, 3, 512, 64), torch.bfloat16, seed=11)
    for causal in (False, True):
        a, da = _fwd(q, k, v, causal=causal)
        b, db = _fwd(q, k, v, causal=causal, flags=_lib.FLAG_GENERIC)
        assert normwise(to_f64(a), to_f64(b)) <= 4e-3
        assert normwise(to_f64(da), to_f64(db)) <= 1e-5


def test_exact_tail_flag_agrees():
    q, k, v = make_qkv((1, 4, 512, 64), torch.bfloat16, seed=12)
    a, _ = _fwd(q, k, v, causal=True)
    b, _ = _fwd(q, k, v, causal=True, flags=_lib.FLAG_EXACT_TAIL)
    ref = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, True)
    assert normwise(to_f64(a), ref) <= 2e-2 and normwise(to_f64(b), ref) <= 2e-2
    assert normwise(to_f64(a), to_f64(b)) <= 4e-3


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_head_dim_128(dt):
    """C5-shaped forward (D=128) at reduced size.  fp16 inputs are scaled so that rho^8 stays
    below the fp16 overflow threshold when P is cast to v.dtype (the reference casts the same way)."""
    q, k, v = make_qkv((1, 4, 512, 128), dt, seed=13, scale=1.0 if dt == torch.bfloat16 else 0.3)
    out, den = _fwd(q, k, v, causal=True)
    c_out, c_den = oracle_contract(q, k, v, 0.5, True)
    ref = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, True)
    print(f"D=128 {dt}: vs contract {normwise(to_f64(out), c_out):.3e} vs fp64 {normwise(to_f64(out), ref):.3e}")
    assert normwise(to_f64(out), c_out) <= 4e-3
    assert normwise(to_f64(out), ref) <= 2e-2
    assert normwise(to_f64(den), c_den) <= 1e-5


@pytest.mark.parametrize("shape,causal,valid,rot", [
    ((1, 2, 300, 256), True, None, True), ((2, 1, 200, 256), False, 150, False), ((1, 1, 1, 256), True, None, False),
    ((1, 3, 513, 256), True, None, False),
])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_head_dim_256(shape, causal, valid, rot, dt):
    """head_dim 256 (the reference accepts multiples of 128 above 128) on the fully fused MFMA
    kernel, 1/sqrt(256) = 2^-4 folded into q: against the generic kernel, the C contract and
    float64.  fp16 inputs are scaled to keep the fp16 weights below overflow."""
    B, H, L, D = shape
    q, k, v = make_qkv(shape, dt, seed=sum(shape), scale=1.0 if dt == torch.bfloat16 else 0.3)
    rotary = A.build_cayley_rotary_matrix(D, L, freqs=_c3_freqs(D)) if rot else None
    out, den = _fwd(q, k, v, causal=causal, valid=valid, rotary=rotary)
    gout, gden = _fwd(q, k, v, causal=causal, valid=valid, rotary=rotary, flags=_lib.FLAG_GENERIC)
    c_out, c_den = oracle_contract(q, k, v, 0.5, causal, valid_len=valid, rotary=rotary)
    tol = _ulp_tol(dt)
    e_g, e_c = normwise(to_f64(out), to_f64(gout)), normwise(to_f64(out), c_out)
    print(f"D=256 {shape} causal={causal} valid={valid} rot={rot} {dt}: vs generic {e_g:.2e} vs contract {e_c:.2e}")
    assert e_g <= tol and e_c <= tol
    assert normwise(to_f64(den), c_den) <= 1e-5
    if not rot:
        ref = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, causal, valid_len=valid)
        assert normwise(to_f64(out), ref) <= 2e-2


@pytest.mark.parametrize("D", [8, 16, 32, 48, 96, 256])
def test_generic_head_dims(D):
    q, k, v = make_qkv((1, 2, 96, D), torch.float32, seed=14)
    y = A.pallas_afa_forward(q, k, v, causal=True, block_q=32, block_k=32)
    ref = O.afa_forward(to_f64(q), to_f64(k), to_f64(v), 0.5, True)
    assert normwise(to_f64(y), ref) <= 1e-5


def _ulp_tol(dt):
    """Bound for max|y - ref| / max|ref| between two outputs that are each rounded to dt after fp32
    accumulation in different orders: one rounding flip of an element in the top binade costs up
    to one ulp, 2^-7 of max|ref| in bf16 (7 explicit mantissa bits) and 2^-10 in fp16."""
    return 8e-3 if dt == torch.bfloat16 else 4e-3


def _cu_count():
    return torch.cuda.get_device_properties(0).multi_processor_count


@pytest.mark.parametrize("shape,causal,valid,rot", [
    ((1, 1, 1, 64), True, None, False), ((1, 1, 32, 64), False, None, False), ((2, 3, 96, 64), True, None, True),
    ((1, 2, 300, 64), True, None, False), ((1, 2, 300, 64), False, 257, True), ((3, 5, 513, 64), True, 400, False),
    ((1, 1, 1024, 64), False, None, False), ((2, 4, 1000, 64), True, None, True),
])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("wide", [False, True])
def test_pipelined_d64_edge_shapes(shape, causal, valid, rot, dt, wide):
    """The head_dim-64 kernels against the simple MFMA kernel and the C contract on lengths that
    are not tile multiples, tiny lengths, valid_len tails and odd batch x head counts (so the
    workgroup remap sees counts not divisible by 8).  Small grids take the 32-query kernel
    (afa_fwd_pipe.hip); `wide` repeats the heads until the 256-query workgroups number at least
    three per CU, which takes afa_fwd_d64.hip, and checks every copy of a head is bitwise equal."""
    B, H, L, D = shape
    scale = 1.0 if dt == torch.bfloat16 else 0.4
    q, k, v = make_qkv(shape, dt, seed=sum(shape), scale=scale)
    rotary = A.build_cayley_rotary_matrix(D, L, freqs=_c3_freqs(D)) if rot else None
    c_out, c_den = oracle_contract(q, k, v, 0.5, causal, valid_len=valid, rotary=rotary)
    reps = 1
    if wide:
        reps = -(-3 * _cu_count() // (B * H * -(-L // 256)))
        q, k, v = (x.repeat(1, reps, 1, 1).contiguous() for x in (q, k, v))
    a, da = _fwd(q, k, v, causal=causal, valid=valid, rotary=rotary)
    b, db = _fwd(q, k, v, causal=causal, valid=valid, rotary=rotary, flags=_lib.FLAG_SIMPLE_SCHEDULE)
    assert np.isfinite(to_f64(a)).all()
    tol = _ulp_tol(dt)
    assert normwise(to_f64(a), to_f64(b)) <= tol
    if wide:
        assert torch.equal(a, a[:, :H].repeat(1, reps, 1, 1))
        assert torch.equal(da, da[:, :H].repeat(1, reps, 1, 1))
        a, da = a[:, :H], da[:, :H]
    e_c = normwise(to_f64(a), c_out)
    print(f"d64 {shape} causal={causal} valid={valid} rot={rot} {dt} wide={wide} (x{reps}): vs contract {e_c:.2e}")
    assert e_c <= tol
    assert normwise(to_f64(da), c_den) <= 1e-5


@pytest.mark.parametrize("D", [32, 48, 96])
@pytest.mark.parametrize("shape,causal,valid,rot", [
    ((1, 1, 1), True, None, False), ((2, 3, 96), True, None, True), ((1, 2, 300), False, 257, True),
    ((3, 5, 513), True, 400, False), ((2, 4, 1000), True, None, True),
])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_padded_head_dims(D, shape, causal, valid, rot, dt):
    """head_dim 32, 48 and 96 on the matrix-core kernel (rows zero-padded to 64 / 128 in LDS,
    1/sqrt(D) split into a power of two on q and an fp32 factor on the score) against the
    generic kernel, the C contract and the float64 oracle."""
    B, H, L = shape
    scale = 1.0 if dt == torch.bfloat16 else 0.4
    q, k, v = make_qkv((B, H, L, D), dt, seed=D + L + 5, scale=scale)
    rotary = A.build_cayley_rotary_matrix(D, L, freqs=_c3_freqs(D)) if rot else None
    a, da = _fwd(q, k, v, causal=causal, valid=valid, rotary=rotary)
    b, db = _fwd(q, k, v, causal=causal, valid=valid, rotary=rotary, flags=_lib.FLAG_GENERIC)
    c_out, c_den = oracle_contract(q, k, v, 0.5, causal, valid_len=valid, rotary=rotary)
    qr, kr = to_f64(q), to_f64(k)
    if rot:
        c64, s64 = rotary.c.double().cpu().numpy(), rotary.s.double().cpu().numpy()
        qr, kr = O.rotate_pairs(qr, c64, s64), O.rotate_pairs(kr, c64, s64)
    ref, dref = O.afa_forward(qr, kr, to_f64(v), 0.5, causal, valid, return_denominator=True)
    assert np.isfinite(to_f64(a)).all()
    e_g, e_c, e_r = normwise(to_f64(a), to_f64(b)), normwise(to_f64(a), c_out), normwise(to_f64(a), ref)
    print(f"D={D} {shape} causal={causal} valid={valid} rot={rot} {dt}: vs generic {e_g:.2e} "
          f"vs contract {e_c:.2e} vs fp64 {e_r:.2e}")
    tol = _ulp_tol(dt)
    assert e_g <= tol and e_c <= tol
    assert e_r <= 2e-2
    assert normwise(to_f64(da), c_den) <= 1e-5
    assert normwise(to_f64(da), dref) <= 1e-2


def test_device_is_the_build_target():
    """The library holds gfx950 code only (its kernels place up to 141 KB of LDS per workgroup,
    within a CDNA4 CU's 160 KB): the device must be a gfx950 and report at least 64 KB of LDS
    per workgroup."""
    p = torch.cuda.get_device_properties(0)
    arch = getattr(p, "gcnArchName", "")
    print("device", p.name, arch, "CUs", p.multi_processor_count,
          "sharedMemPerBlock", getattr(p, "shared_memory_per_block", None))
    assert arch.split(":")[0] == "gfx950"
    assert p.multi_processor_count >= 1
    lds = getattr(p, "shared_memory_per_block", None)
    if lds is not None:
        assert lds >= 64 * 1024


@pytest.mark.parametrize("shape,causal,valid,rot", [
    ((1, 2, 256, 64), True, None, False), ((2, 3, 200, 64), False, None, True),
    ((1, 2, 1000, 64), True, 777, True), ((1, 1, 1, 64), True, None, False),
    ((1, 2, 130, 32), True, None, True), ((2, 1, 392, 128), False, 300, False),
    ((1, 2, 256, 128), True, None, True), ((3, 5, 129, 64), True, None, False),
    ((1, 2, 300, 96), True, None, True), ((2, 1, 200, 96), False, 150, False),
    ((1, 2, 260, 48), True, None, True), ((3, 1, 129, 48), False, 100, False),
])
@pytest.mark.parametrize("wide", [False, True])
def test_fp32_mfma_vs_generic_and_fp64(shape, causal, valid, rot, wide):
    """The fp32 matrix-core kernel (afa_fwd_f32.hip) against the generic fp32 kernel
    (AFA_FLAG_GENERIC) and the float64 oracle: the same fp32 contract in another summation order.
    Small grids split the key tiles over several workgroups and add the partials (split-K);
    `wide` repeats the heads until the grid has a 128-query workgroup per CU, which runs unsplit,
    and checks every copy of a head is bitwise equal."""
    B, H, L, D = shape
    q, k, v = make_qkv(shape, torch.float32, seed=sum(shape) + 3)
    rotary = None
    qr, kr = to_f64(q), to_f64(k)
    if rot:
        rotary = A.build_cayley_rotary_matrix(D, L, freqs=torch.from_numpy(_c3_freqs(D)).cuda())
        c, s = rotary.c.double().cpu().numpy(), rotary.s.double().cpu().numpy()
        qr, kr = O.rotate_pairs(qr, c, s), O.rotate_pairs(kr, c, s)
    ref, dref = O.afa_forward(qr, kr, to_f64(v), 0.5, causal, valid, return_denominator=True)
    reps = -(-_cu_count() // (B * H * -(-L // 128))) if wide else 1
    if wide:
        q, k, v = (x.repeat(1, reps, 1, 1).contiguous() for x in (q, k, v))
    a, da = _fwd(q, k, v, causal=causal, valid=valid, rotary=rotary)
    b, db = _fwd(q, k, v, causal=causal, valid=valid, rotary=rotary, flags=_lib.FLAG_GENERIC)
    e_g = normwise(to_f64(a), to_f64(b))
    if wide:
        assert torch.equal(a, a[:, :H].repeat(1, reps, 1, 1))
        assert torch.equal(da, da[:, :H].repeat(1, reps, 1, 1))
        a, da = a[:, :H], da[:, :H]
    e_r = normwise(to_f64(a), ref)
    print(f"fp32 {shape} causal={causal} valid={valid} rot={rot} wide={wide} (x{reps}): vs generic {e_g:.2e} "
          f"vs fp64 {e_r:.2e}")
    assert e_g <= 1e-5 and e_r <= 1e-5
    assert normwise(to_f64(da), dref) <= 1e-5


def test_fp32_strided_model_layout():
    """(B, T, H, D).transpose(1, 2) fp32 views run the matrix-core kernel with the strides."""
    B, T, H, D = 2, 300, 4, 64
    rng = np.random.default_rng(19)
    base = [torch.from_numpy(rng.standard_normal((B, T, H, D))).float().cuda() for _ in range(3)]
    views = [x.transpose(1, 2) for x in base]
    y_view = A.pallas_afa_forward(*views, causal=True, block_q=100, block_k=100)
    y_cont = A.pallas_afa_forward(*[x.contiguous() for x in views], causal=True, block_q=100, block_k=100)
    assert torch.equal(y_view, y_cont)


@pytest.mark.parametrize("shape,causal,valid,rot", [
    ((1, 1, 1, 128), True, None, False), ((1, 1, 32, 128), False, None, True), ((2, 3, 96, 128), True, None, False),
    ((1, 2, 300, 128), True, None, True), ((1, 2, 300, 128), False, 257, False), ((3, 5, 513, 128), True, 400, True),
    ((1, 1, 1024, 128), False, None, False), ((2, 4, 1000, 128), True, None, True),
])
@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_pipelined_d128_edge_shapes(shape, causal, valid, rot, dt):
    """The head_dim-128 kernel (afa_fwd_pipe.hip; with Cayley tables after the K rotation
    pre-pass, q rotated at load) against the simple MFMA kernel (which rotates at tile load) and
    the C contract on ragged and tiny lengths, valid_len tails and odd head counts."""
    D, L = shape[3], shape[2]
    scale = 1.0 if dt == torch.bfloat16 else 0.3
    q, k, v = make_qkv(shape, dt, seed=sum(shape) + 1, scale=scale)
    rotary = A.build_cayley_rotary_matrix(D, L, freqs=_c3_freqs(D)) if rot else None
    a, da = _fwd(q, k, v, causal=causal, valid=valid, rotary=rotary)
    b, db = _fwd(q, k, v, causal=causal, valid=valid, rotary=rotary, flags=_lib.FLAG_SIMPLE_SCHEDULE)
    c_out, c_den = oracle_contract(q, k, v, 0.5, causal, valid_len=valid, rotary=rotary)
    assert np.isfinite(to_f64(a)).all()
    e_s, e_c = normwise(to_f64(a), to_f64(b)), normwise(to_f64(a), c_out)
    print(f"d128 {shape} causal={causal} valid={valid} rot={rot} {dt}: vs simple {e_s:.2e} vs contract {e_c:.2e}")
    tol = _ulp_tol(dt)
    assert e_s <= tol and e_c <= tol
    assert normwise(to_f64(da), c_den) <= 1e-5
