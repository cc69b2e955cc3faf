"""kore_amd -- MI355X (gfx950) native GEMM family for the KORE operator task suite.

Operators (all on HIP device tensors, launched on torch's current stream):
dense bf16/fp16/fp32 GEMM with fused bias + activation epilogues, the linear-layer GEMM
backward, batched GEMM, OCP-e4m3
fp8 a8w8 block-scaled GEMM, fp8/int8 a8w8 GEMM with row/column scales, and the fused top-k MoE SiLU grouped GEMM.  The kernels
live in ``libkore_amd.so`` (built by ``python kore_amd/build.py``); see
``include/kore_amd.h`` for its C ABI.
"""

from .ops import (  # noqa: F401
    ACT_CODE,
    GEMM_FUSION_OPS,
    batched_gemm,
    fused_moe,
    gemm,
    gemm_a8w8,
    gemm_a8w8_blockscale,
    gemm_backward,
    gemm_fused,
    grouped_gemm,
    grouped_gemm_fp8,
    moe_align,
    moe_align_block_offsets,
    moe_expert_offsets,
    moe_gated_silu,
    moe_permute,
    moe_unpermute,
)
from . import ops as _ops

for _name in _ops.GEMM_FUSION_OPS:
    globals()[_name] = getattr(_ops, _name)

__all__ = ["gemm", "gemm_fused", "batched_gemm", "gemm_backward", "gemm_a8w8_blockscale", "gemm_a8w8", "fused_moe", "moe_gated_silu", "moe_align",
           "grouped_gemm", "grouped_gemm_fp8", "moe_permute", "moe_unpermute", "moe_align_block_offsets", "moe_expert_offsets",
           *_ops.GEMM_FUSION_OPS]
