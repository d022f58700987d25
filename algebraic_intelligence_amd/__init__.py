"""algebraic_intelligence_amd — Algebraic FlashAttention (AFA) for AMD MI355X (gfx950).

A drop-in for the AFA hot path of tasmaikeni13/algebraic-intelligence: the fused forward
(pallas_afa_forward / tiled_afa_forward), its analytical backward (pallas_afa custom VJP),
the padding front door (algebraic_flash_attention), the sequence ring (distributed_ring_afa, its
hops run in turn on one GPU) and the batch x heads placement (sharded_pallas_afa), the A-Softmax (algebraic_softmax), the
octic weight (octic_kernel), the Cayley rotary (AGO) tables and rotation, and the OACE loss head
(fused_linear_oace, fused_oace_softmax_loss) — all running in hand-written HIP kernels behind the
C ABI of include/afa.h.
"""
from .afa import (
    afa_flops,
    algebraic_flash_attention,
    distributed_ring_afa,
    exact_afa_reference,
    exact_afa_with_denominator,
    pallas_afa,
    pallas_afa_forward,
    sharded_pallas_afa,
    tiled_afa_backward,
    tiled_afa_forward,
)
from .attention import (
    CayleyRotary,
    algebraic_softmax,
    apply_ago_rotations,
    build_cayley_rotary_matrix,
    octic_kernel,
    rotate_tensor,
)
from .oace import (
    fused_linear_oace,
    fused_linear_oace_backward,
    fused_linear_oace_forward,
    fused_oace_softmax_loss,
)

__all__ = [
    "afa_flops", "algebraic_flash_attention", "distributed_ring_afa", "exact_afa_reference", "exact_afa_with_denominator",
    "pallas_afa", "pallas_afa_forward", "sharded_pallas_afa", "tiled_afa_backward", "tiled_afa_forward",
    "CayleyRotary", "algebraic_softmax", "apply_ago_rotations", "build_cayley_rotary_matrix",
    "octic_kernel", "rotate_tensor", "fused_linear_oace", "fused_linear_oace_forward",
    "fused_linear_oace_backward", "fused_oace_softmax_loss",
]
