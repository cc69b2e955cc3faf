"""Comparators of the reference's drivers and its four-prong verifier (CPU).

Test infrastructure only (see ``oracle/__init__.py``).

Two layers, both restated from the reference:

* the task-driver verdict (``SNR:`` / ``allclose:`` / ``max_diff:``):
  ``snr_db`` (``kore/tasks/gemm_bf16/driver.py:44-50``) and the non-finite-aware
  ``compare_outputs`` (``kore/tasks/_genops.py:906-945``) with per-task atol/rtol;
* the four-prong verifier's per-pair rule (``kore/verify/equivalence.py:108-253``):
  worst per-element ``|c-r|/(|r|+atol) <= rtol`` AND ``SNR >= floor`` AND exact
  agreement of non-finite positions, with dtype-aware tolerances and tighter
  (determinism) / looser (metamorphic) variants.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

# Per-task driver tolerances and SNR gates (task.yaml snr_threshold / driver atol):
# gemm_bf16/driver.py:122, _genops.py:941, _quant_common ATOL/RTOL,
# fused_moe_silu_bf16/driver.py:123, moe_batched_gemm_bf16/reference.py.
TASK_TOL = {
    "gemm": dict(atol=1e-2, rtol=1e-2, snr=30.0),
    "gemm_fusion": dict(atol=1e-2, rtol=1e-2, snr=30.0),
    "gemm_fusion_fp32": dict(atol=1e-2, rtol=1e-2, snr=40.0),  # _genops.py:44 fp32 gate
    "batched_gemm": dict(atol=1e-2, rtol=1e-2, snr=30.0),
    # gemm_backward_bf16/reference.py:26 TOL and task.yaml snr_threshold
    "gemm_backward_dx": dict(atol=5e-2, rtol=2e-2, snr=25.0),
    "gemm_backward_dw": dict(atol=2e-1, rtol=2e-2, snr=25.0),
    "blockscale": dict(atol=5e-1, rtol=5e-2, snr=25.0),
    "blockscale_genv": dict(atol=1e-2, rtol=1e-2, snr=25.0),
    # a8w8 row/column scales: gemm_fp8_a8w8/driver.py:122, _quant_common ATOL/RTOL;
    # the generated vendor task compares at the _genops tolerance
    "a8w8": dict(atol=5e-1, rtol=5e-2, snr=25.0),
    "a8w8_genv": dict(atol=1e-2, rtol=1e-2, snr=25.0),
    "fused_moe": dict(atol=3e-2, rtol=3e-2, snr=25.0),
    "moe_batched": dict(atol=2e-2, rtol=2e-2, snr=25.0),
    # top-1 grouped expert GEMM: moe_grouped_gemm_bf16/reference.py:27-28, task.yaml snr
    "grouped": dict(atol=2e-2, rtol=2e-2, snr=25.0),
    "grouped_fp8": dict(atol=3e-2, rtol=3e-2, snr=25.0),  # moe_grouped_gemm_fp8/reference.py:30-31
    # max-abs/rel <= 1e-2 in allclose form for bf16/fp16 out
    "north_star": dict(atol=1e-2, rtol=1e-2, snr=25.0),
}


def snr_db(out: torch.Tensor, ref: torch.Tensor) -> float:
    """``20*log10(||r|| / ||o-r||)``; 999 when exact, -999 when the reference is 0.

    Follows ``kore/tasks/gemm_bf16/driver.py:44-50``.
    """
    o, r = out.float().cpu(), ref.float().cpu()
    noise = (o - r).norm().item()
    signal = r.norm().item()
    if noise == 0:
        return 999.0
    return 20.0 * math.log10(signal / noise) if signal > 0 else -999.0


def compare_outputs(out: torch.Tensor, ref: torch.Tensor, atol: float = 1e-2,
                    rtol: float = 1e-2):
    """Non-finite-aware driver comparison -> ``(snr_db, max_abs_diff, allclose)``.

    Follows ``kore/tasks/_genops.py:906-945``: non-finite positions must match
    exactly and infinities must agree in sign; SNR, max-diff and ``allclose`` are
    taken over the finite subset.
    """
    of, rf = out.float().cpu(), ref.float().cpu()
    if of.shape != rf.shape:
        return -999.0, float("inf"), False
    rfin, ofin = torch.isfinite(rf), torch.isfinite(of)
    if not torch.equal(rfin, ofin):
        return -999.0, float("inf"), False
    rinf = torch.isinf(rf)
    if bool(rinf.any()) and not torch.equal(torch.sign(rf[rinf]), torch.sign(of[rinf])):
        return -999.0, float("inf"), False
    if bool(rfin.all()):
        of_c, rf_c = of, rf
    else:
        of_c, rf_c = of[rfin], rf[rfin]
    if rf_c.numel() == 0:
        return 999.0, 0.0, True
    snr = snr_db(of_c, rf_c)
    maxd = (of_c - rf_c).abs().max().item()
    ok = bool(torch.allclose(of_c, rf_c, atol=atol, rtol=rtol))
    return snr, maxd, ok


@dataclass(frozen=True)
class Tolerance:
    """Four-prong tolerance (``kore/verify/equivalence.py:108-132``)."""

    rtol: float = 3e-3
    atol: float = 1e-4
    snr_db_min: float = 50.0
    determinism_rtol: float = 1e-5
    determinism_snr_db_min: float = 80.0
    metamorphic_rtol: float = 6e-3
    metamorphic_snr_db_min: float = 46.0


def tolerance_for(dtype: str) -> Tolerance:
    """Low-precision dtypes get the relaxed bounds (``equivalence.py:135-151``)."""
    d = (dtype or "").lower()
    if any(t in d for t in ("fp16", "bf16", "float16", "bfloat16", "fp8", "fp4")):
        return Tolerance(rtol=3e-2, atol=1e-2, snr_db_min=30.0,
                         determinism_rtol=1e-3, determinism_snr_db_min=40.0,
                         metamorphic_rtol=5e-2, metamorphic_snr_db_min=28.0)
    return Tolerance()


@dataclass
class PairResult:
    ok: bool
    worst_rel_err: float
    snr_db: float
    reason: str = ""


def _f64(a) -> np.ndarray:
    if isinstance(a, torch.Tensor):
        return a.detach().to(dtype=torch.float64, device="cpu").numpy()
    return np.asarray(a, dtype=np.float64)


def compare_pair(actual, expected, tol: Tolerance, rtol: float | None = None,
                 snr_db_min: float | None = None) -> PairResult:
    """One (candidate, reference) pair under the four-prong rule.

    Follows ``kore/verify/equivalence.py:197-253``: strict non-finite agreement,
    worst per-element ``|a-e|/(|e|+atol)`` against ``rtol`` and aggregate SNR
    against the floor.  An exact match has infinite SNR.
    """
    r = tol.rtol if rtol is None else rtol
    s = tol.snr_db_min if snr_db_min is None else snr_db_min
    a, e = _f64(actual), _f64(expected)
    if a.shape != e.shape:
        return PairResult(False, math.inf, -math.inf, f"shape {a.shape} vs {e.shape}")
    af, ef = a.ravel(), e.ravel()
    if ef.size == 0:
        return PairResult(True, 0.0, math.inf, "empty")
    fin = np.isfinite(af) & np.isfinite(ef)
    nonfin = ~fin
    nonfinite_ok = True
    if nonfin.any():
        an, en = af[nonfin], ef[nonfin]
        nonfinite_ok = bool(((an == en) | (np.isnan(an) & np.isnan(en))).all())
    if fin.any():
        diff = np.abs(af[fin] - ef[fin])
        worst = float((diff / (np.abs(ef[fin]) + tol.atol)).max())
        noise = float(np.linalg.norm(diff))
        signal = float(np.linalg.norm(ef[fin]))
        if noise == 0.0:
            snr = math.inf
        elif signal == 0.0:
            snr = -math.inf
        else:
            snr = 20.0 * math.log10(signal / noise)
    else:
        worst, snr = 0.0, math.inf
    if not nonfinite_ok:
        worst = math.inf
    ok = nonfinite_ok and worst <= r and snr >= s
    reason = ""
    if not ok:
        if not nonfinite_ok:
            reason = "non-finite mismatch"
        elif worst > r:
            reason = f"rel-err {worst:.3e} > {r:.1e}"
        else:
            reason = f"SNR {snr:.1f} dB < {s:.1f} dB"
    return PairResult(ok, worst, snr, reason)
