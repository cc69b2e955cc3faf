"""kore_amd drop-in candidate for the KORE task ``fused_moe_silu_bf16``.

The entry keeps the task oracle's signature; the body is the hand-written gfx950
HIP kernel in libkore_amd.so (kore_amd must be importable, e.g. on PYTHONPATH).
"""
import kore_amd


def fused_moe(hidden_states, w1, w2, topk_weight, topk_ids):
    return kore_amd.moe_gated_silu(hidden_states, w1, w2, topk_weight, topk_ids)
