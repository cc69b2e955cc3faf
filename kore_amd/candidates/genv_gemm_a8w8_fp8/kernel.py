"""kore_amd drop-in candidate for the KORE task ``genv_gemm_a8w8_fp8``.

The entry keeps the task oracle's signature; the body is the hand-written gfx950
HIP kernel in libkore_amd.so (kore_amd must be importable, e.g. on PYTHONPATH).
"""
import kore_amd


def gemm_a8w8(xq, wq, x_scale, w_scale):
    return kore_amd.gemm_a8w8(xq, wq, x_scale, w_scale)
