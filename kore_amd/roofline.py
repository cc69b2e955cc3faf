"""Roofline model for the GEMM family on MI355X.

FLOP and byte counts follow the reference's scorer (``kore/analysis/rooflines.py:153-282``):
GEMM ``F = 2MNK``, ``Q = (MK + KN + MN)*e``; fp8 / int8 GEMM ``Q = (MK + KN)*1 + MN*2``;
batched/grouped GEMM multiply both by B; fused MoE ``F = M*topk*6*D*I``,
``Q = (E*3*D*I + 2*M*D)*e``.  ``T_min = max(F/peak_flops, Q/peak_bw)``.

Two operators are priced here by what they must move, not by the scorer's formula:
the top-1 expert GEMM ``moe_grouped_gemm`` (the scorer's B=1 grouped form counts one
``K x N`` weight, but every expert that receives a token has its weight read once:
``Q = (M*K + E_used*N*K + M*N)*e``) and the row permute ``moe_permute``
(``F = 0``, ``Q = 2*M*D*e + 4*M``: rows in, rows out, one int32 index per row).

Peaks are MI355X's published dense figures (no sparsity): bf16/fp16 2.5 PFLOP/s,
fp8 5.0 PFLOP/s, int8 5.0 POP/s, fp32 157.3 TFLOP/s, HBM3E 8.0 TB/s.  ``KORE_PEAK_BF16`` / ``KORE_PEAK_FP8`` /
``KORE_PEAK_HBM_BW`` override them as in the reference (``rooflines.py:84-97``).
"""

from __future__ import annotations

import os
from dataclasses import dataclass

MI355X_PEAKS = {
    "hbm_bytes_per_s": 8.0e12,
    "bf16_flops_per_s": 2.5e15,
    "fp16_flops_per_s": 2.5e15,
    "fp8_flops_per_s": 5.0e15,
    "int8_flops_per_s": 5.0e15,
    "fp32_flops_per_s": 1.573e14,
}


def resolve_peaks() -> dict[str, float]:
    p = dict(MI355X_PEAKS)
    for env, keys in (("KORE_PEAK_BF16", ("bf16_flops_per_s", "fp16_flops_per_s")),
                      ("KORE_PEAK_FP8", ("fp8_flops_per_s",)),
                      ("KORE_PEAK_HBM_BW", ("hbm_bytes_per_s",))):
        v = os.environ.get(env)
        if v:
            for k in keys:
                p[k] = float(v)
    return p


def dtype_bytes(dtype: str) -> int:
    d = dtype.lower()
    if "fp8" in d or "int8" in d:
        return 1
    if "fp32" in d or "float32" in d:
        return 4
    return 2


def flops_bytes(operation: str, dims: dict[str, int], dtype: str) -> tuple[float, float]:
    """Algorithmic (FLOPs, HBM bytes) of one call, per the reference's formulas."""
    op = operation.lower()
    e = dtype_bytes(dtype)
    fp8 = "fp8" in dtype.lower() or "int8" in dtype.lower()  # 8-bit operands, bf16 output
    if op == "moe_grouped_gemm":
        M, N, K = dims["M"], dims["N"], dims["K"]
        Eu = dims.get("E_used", dims["E"])
        return 2.0 * M * N * K, float((M * K + Eu * N * K + M * N) * e)
    if op == "gemm_backward":
        # two GEMMs (dX = dY.W, dW = dY^T.X): the reference's dense formula counts one
        M, N, K = dims["M"], dims["N"], dims["K"]
        return 4.0 * M * N * K, float((2 * M * K + 2 * N * K + M * N) * e)
    if op in ("moe_permute", "moe_unpermute"):
        M, D = dims["M"], dims["D"]
        return 0.0, float(2 * M * D * e + 4 * M)
    if "batched_gemm" in op or "grouped_gemm" in op or op == "bmm":
        B = dims.get("B", dims.get("batch", 1))
        M, N, K = dims["M"], dims["N"], dims["K"]
        by = B * ((M * K + K * N) + M * N * 2) if fp8 else B * (M * K + K * N + M * N) * e
        return 2.0 * B * M * N * K, float(by)
    if "moe" in op:
        M, E, topk, D, I = dims["M"], dims["E"], dims["topk"], dims["D"], dims["I"]
        return float(M * topk * 6 * D * I), float((E * 3 * D * I + 2 * M * D) * e)
    if "gemm" in op or "matmul" in op:
        M, N, K = dims["M"], dims["N"], dims["K"]
        by = (M * K + K * N) + M * N * 2 if fp8 else (M * K + K * N + M * N) * e
        return 2.0 * M * N * K, float(by)
    raise ValueError(f"no roofline model for {operation!r}")


@dataclass
class Roofline:
    flops: float
    bytes: float
    t_compute_s: float
    t_mem_s: float
    t_min_s: float
    bound: str          # "mfma" | "hbm"
    peak_flops: float
    peak_bw: float


def roofline(operation: str, dims: dict[str, int], dtype: str) -> Roofline:
    peaks = resolve_peaks()
    f, q = flops_bytes(operation, dims, dtype)
    d = dtype.lower()
    pf = peaks["fp8_flops_per_s"] if "fp8" in d else peaks["int8_flops_per_s"] if "int8" in d else \
        peaks["fp32_flops_per_s"] if ("fp32" in d or "float32" in d) else peaks["bf16_flops_per_s"]
    pb = peaks["hbm_bytes_per_s"]
    tc, tm = f / pf, q / pb
    return Roofline(f, q, tc, tm, max(tc, tm), "mfma" if tc >= tm else "hbm", pf, pb)
