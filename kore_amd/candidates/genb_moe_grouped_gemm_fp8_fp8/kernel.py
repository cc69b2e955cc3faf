"""kore_amd drop-in candidate for the KORE task ``genb_moe_grouped_gemm_fp8_fp8``.

The entry keeps the task oracle's signature; the body is the hand-written gfx950
HIP kernel in libkore_amd.so (kore_amd must be importable, e.g. on PYTHONPATH).
"""
import kore_amd


def moe_grouped_gemm_fp8(xq, wq, xs, ws, expert_ids):
    return kore_amd.grouped_gemm_fp8(xq, wq, xs, ws, expert_ids)
