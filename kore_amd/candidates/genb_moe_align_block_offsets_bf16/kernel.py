"""kore_amd drop-in candidate for the KORE task ``genb_moe_align_block_offsets_bf16``.

The entry keeps the task oracle's signature; the body is the hand-written gfx950
HIP kernel in libkore_amd.so (kore_amd must be importable, e.g. on PYTHONPATH).
"""
import kore_amd


def moe_align_block_offsets(expert_ids, E, block):
    return kore_amd.moe_align_block_offsets(expert_ids, E, block)
