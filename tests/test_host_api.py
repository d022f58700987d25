"""The Python call surface (algebraic_intelligence_amd) without a GPU: the reference's argument
checks and exception types (src/kernels/pallas_afa.py:167-186, src/attention.py:60-63,155-204,
src/primitives.py:17-21,56-59), and no silent CPU fallback for valid calls."""
import math

import pytest
import torch

import algebraic_intelligence_amd as A


def _qkv(shape=(1, 2, 128, 64), dtype=torch.float32):
    return [torch.zeros(shape, dtype=dtype) for _ in range(3)]


@pytest.mark.parametrize("fn", [A.pallas_afa_forward, A.tiled_afa_forward, A.pallas_afa])
def test_forward_argument_checks(fn):
    q, k, v = _qkv()
    with pytest.raises(ValueError):
        fn(q[0], k[0], v[0])
    with pytest.raises(ValueError):
        fn(q, k[:, :, :64], v)
    for bad in (-1.0, math.nan, math.inf):
        with pytest.raises(ValueError, match="sink_omega"):
            fn(q, k, v, sink_omega=bad)
    with pytest.raises(ValueError):
        fn(q, k, v, block_q=0)
    with pytest.raises(ValueError):
        fn(q, k, v, block_q=96)
    with pytest.raises(ValueError, match="valid_seq_len"):
        fn(q, k, v, valid_seq_len=0)
    with pytest.raises(ValueError, match="valid_seq_len"):
        fn(q, k, v, valid_seq_len=129)


def test_head_dim_rule():
    q, k, v = _qkv((1, 1, 128, 192))
    with pytest.raises(ValueError, match="divisible by 128"):
        A.pallas_afa_forward(q, k, v)
    with pytest.raises(ValueError, match="divisible by 128"):
        A.algebraic_flash_attention(q, k, v)


@pytest.mark.parametrize("fn", [A.pallas_afa_forward, A.tiled_afa_forward, A.algebraic_flash_attention])
def test_valid_calls_on_host_tensors_fail_loudly(fn):
    """There is no CPU implementation behind the API: a valid call on host tensors raises."""
    q, k, v = _qkv()
    with pytest.raises(RuntimeError, match="GPU"):
        fn(q, k, v, causal=True)


def test_ring_argument_checks():
    """distributed_ring_afa (src/kernels/pallas_afa.py:618-662): shapes, sink and the shard count
    are checked first; a valid call on host tensors raises (no CPU implementation)."""
    q, k, v = _qkv()
    with pytest.raises(ValueError):
        A.distributed_ring_afa(q[0], k[0], v[0])
    with pytest.raises(ValueError):
        A.distributed_ring_afa(q, k[:, :, :64], v)
    with pytest.raises(ValueError, match="sink_omega"):
        A.distributed_ring_afa(q, k, v, sink_omega=-1.0)
    for n in (0, -2, 3, 256):
        with pytest.raises(ValueError, match="num_devices"):
            A.distributed_ring_afa(q, k, v, num_devices=n)
    with pytest.raises(RuntimeError, match="GPU"):
        A.distributed_ring_afa(q, k, v, causal=True, num_devices=4)


def test_sharded_argument_checks():
    """sharded_pallas_afa (src/kernels/pallas_afa.py:665-692): batch must split over 'data' and
    heads over 'fsdp'; the mesh is None, a mapping of axis sizes or an object with .shape; the
    pallas_afa checks follow, and a valid call on host tensors raises."""
    q, k, v = _qkv((4, 6, 128, 64))
    with pytest.raises(ValueError, match="data"):
        A.sharded_pallas_afa(q, k, v, mesh={"data": 3, "fsdp": 1, "model": 1})
    with pytest.raises(ValueError, match="fsdp"):
        A.sharded_pallas_afa(q, k, v, mesh={"data": 2, "fsdp": 4, "model": 1})
    with pytest.raises(TypeError):
        A.sharded_pallas_afa(q, k, v, mesh=[2, 3])
    with pytest.raises(ValueError):
        A.sharded_pallas_afa(q, k, v, mesh=None, block_q=96)

    class _Mesh:
        shape = {"data": 2, "fsdp": 3, "model": 1}
    with pytest.raises(RuntimeError, match="GPU"):
        A.sharded_pallas_afa(q, k, v, mesh=_Mesh(), causal=True)


def test_algebraic_softmax_checks():
    x = torch.zeros(4, 8)
    for bad in (-0.1, math.nan, math.inf):
        with pytest.raises(ValueError, match="sink_omega"):
            A.algebraic_softmax(x, sink_omega=bad)
    for bad in (0.0, -1e-5, math.inf, math.nan):
        with pytest.raises(ValueError, match="eps"):
            A.algebraic_softmax(x, eps=bad)
    with pytest.raises(ValueError):
        A.algebraic_softmax(torch.zeros(4, 0))
    with pytest.raises(TypeError):
        A.algebraic_softmax(torch.zeros(4, 8, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="GPU"):
        A.algebraic_softmax(x)


def test_cayley_rotary_checks():
    for dim in (0, -2, 7):
        with pytest.raises(ValueError, match="dim"):
            A.build_cayley_rotary_matrix(dim, 16)
    with pytest.raises(ValueError, match="max_seq_len"):
        A.build_cayley_rotary_matrix(8, 0)
    with pytest.raises(ValueError, match="freqs"):
        A.build_cayley_rotary_matrix(8, 16, freqs=[0.1, 0.2, 0.3])


def test_apply_ago_rotations_checks():
    q = torch.zeros(1, 2, 16, 8)
    with pytest.raises(ValueError, match="shapes must match"):
        A.apply_ago_rotations(q, torch.zeros(1, 2, 16, 6))
    with pytest.raises(ValueError, match="even"):
        A.apply_ago_rotations(torch.zeros(1, 2, 16, 7), torch.zeros(1, 2, 16, 7))
    with pytest.raises(TypeError):
        A.apply_ago_rotations(q, q, rotary_params=3.0)


def test_align_param_and_rotate_tensor_checks():
    """_align_param (src/attention.py:123-139) is a view of the table's first seq_len rows shaped
    to broadcast on the sequence axis, which it infers as the reference does; _rotate_tensor
    (:142-152) refuses tables that do not broadcast against the feature pairs and, on host
    tensors, fails loudly like every other entry point."""
    from algebraic_intelligence_amd.attention import _align_param, _rotate_tensor
    c = torch.arange(32 * 4, dtype=torch.float32).reshape(32, 4)
    a = _align_param(c, (2, 3, 16, 8), seq_axis=2)
    assert a.shape == (1, 1, 16, 4) and torch.equal(a[0, 0], c[:16]) and a.data_ptr() == c.data_ptr()
    assert _align_param(c, (2, 16, 3, 8)).shape == (1, 16, 1, 4)  # (B, T, H, D): T > H, T <= rows
    assert _align_param(c, (2, 3, 16, 8)).shape == (1, 1, 16, 4)
    assert _align_param(c, (2, 16, 8)).shape == (1, 16, 4)
    assert _align_param(c, (16, 8)).shape == (16, 4)
    x = torch.zeros(2, 3, 16, 8)
    with pytest.raises(ValueError, match="even"):
        _rotate_tensor(torch.zeros(2, 3, 16, 7), a, a)
    with pytest.raises(ValueError, match="broadcast"):
        _rotate_tensor(x, c[:16, :3], c[:16, :3])
    with pytest.raises(ValueError, match="one axis"):
        _rotate_tensor(x, torch.zeros(1, 3, 16, 4), torch.zeros(1, 3, 16, 4))
    with pytest.raises(RuntimeError, match="GPU"):
        _rotate_tensor(x, a, a)


def test_octic_pair_checks():
    """_kernel (src/attention.py:18-26) takes floating point input only and runs on the GPU."""
    from algebraic_intelligence_amd.attention import _kernel, _octic
    assert _octic is A.octic_kernel
    with pytest.raises(TypeError):
        _kernel(torch.zeros(4, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="GPU"):
        _kernel(torch.zeros(4))


def test_reference_module_names_import():
    """Every name the reference's tests and scripts import from src/kernels/pallas_afa.py
    (tests/test_pallas_afa.py:24-35, src/kernels/__init__.py:3-14) exists in afa.py; the Pallas
    tile body afa_kernel raises when called (its loop runs inside the library)."""
    from algebraic_intelligence_amd import afa as M
    for n in ("_vmu_octic_kernel", "afa_kernel", "algebraic_flash_attention", "distributed_ring_afa",
              "exact_afa_reference", "exact_afa_with_denominator", "pallas_afa", "pallas_afa_forward",
              "sharded_pallas_afa", "tiled_afa_backward", "tiled_afa_forward"):
        assert hasattr(M, n), n
    with pytest.raises(NotImplementedError, match="pallas_afa_forward"):
        M.afa_kernel(None, None, None, None, None, None, None, scale=0.125, sink_omega=0.5)


def test_flop_count_matches_definition():
    # 4 B H D N_pairs; non-causal is the reference's 4 b h l^2 d (scripts/run_phase6_tpu.py:236)
    assert A.afa_flops(8, 12, 4096, 64, True) == 4 * 8 * 12 * 64 * 4096 * 4097 // 2
    assert A.afa_flops(1, 4, 256, 64, False) == 4 * 4 * 256 * 256 * 64


def test_rotary_tables_must_fit_the_head_dim():
    """Cayley tables are (positions, head_dim / 2), up to broadcast axes of size 1; tables built for
    another head dimension are refused instead of being reinterpreted as more rows (the reference's
    alignment of the tables fails on the same mismatch, src/attention.py:110-139)."""
    from algebraic_intelligence_amd._lib import table_2d
    assert table_2d(torch.zeros(128, 32), 64).shape == (128, 32)
    assert table_2d(torch.zeros(1, 1, 128, 32), 64).shape == (128, 32)
    assert table_2d(torch.zeros(1, 128, 1, 32), 64).shape == (128, 32)
    assert table_2d(torch.zeros(32), 64).shape == (1, 32)
    for bad in (torch.zeros(128, 64), torch.zeros(128, 16), torch.zeros(2, 128, 32), torch.zeros(()),
                torch.zeros(64 * 32)):
        with pytest.raises(ValueError, match="head_dim/2"):
            table_2d(bad, 64)
    with pytest.raises(ValueError, match="even head dimension"):
        table_2d(torch.zeros(8, 3), 7)
    # both entry points check before any device work: a (L, 64) table with D = 64
    q, k, v = _qkv((1, 1, 128, 64))
    with pytest.raises(ValueError, match="head_dim/2"):
        A.pallas_afa_forward(q, k, v, rotary_params=(torch.zeros(128, 64), torch.zeros(128, 64)))
    with pytest.raises(ValueError, match="head_dim/2"):
        A.apply_ago_rotations(q, k, (torch.zeros(128, 64), torch.zeros(128, 64)), seq_axis=2)
