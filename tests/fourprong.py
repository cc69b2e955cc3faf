"""Four-prong verification helpers for the GPU parity tests (test infrastructure).

Restates the reference's verification protocol for one operator:
  random       >= 5 reseeded trials vs the oracle, driver verdict (SNR gate +
               allclose, ``kore/tasks/_genops.py:948-989``) and the four-prong pair
               rule (``kore/verify/equivalence.py:197-253``);
  adversarial  the generic float fills of ``kore/tasks/_genops.py:855-879``
               (zeros, ones, neg_ones, large=1e3, neg_large, small=1e-3, sign_alt)
               with the non-finite-structure rule;
  metamorphic  GEMM identities defined here (the reference has none for GEMM,
               ``kore/verify/metamorphic.py:183-205``): row split, column permutation,
               power-of-two scaling;
  determinism  two runs on the same inputs must agree bit for bit.
"""

from __future__ import annotations

import math

import torch

from oracle.compare import TASK_TOL, compare_outputs, compare_pair, tolerance_for


def verdict(out: torch.Tensor, ref: torch.Tensor, task: str, dtype: str, label: str = "") -> dict:
    """Driver verdict + four-prong pair result; raises AssertionError with detail on failure."""
    tol = TASK_TOL[task]
    snr, maxd, ok = compare_outputs(out, ref, atol=tol["atol"], rtol=tol["rtol"])
    pair = compare_pair(out, ref, tolerance_for(dtype))
    info = dict(snr=snr, max_diff=maxd, allclose=ok, pair_ok=pair.ok, rel=pair.worst_rel_err,
                pair_snr=pair.snr_db, reason=pair.reason)
    assert ok, f"{label}: allclose failed {info}"
    assert snr >= tol["snr"], f"{label}: SNR {snr:.2f} dB < {tol['snr']} {info}"
    return info


def pair_only(out, ref, dtype: str, label: str, kind: str = "random") -> None:
    tol = tolerance_for(dtype)
    if kind == "metamorphic":
        res = compare_pair(out, ref, tol, rtol=tol.metamorphic_rtol, snr_db_min=tol.metamorphic_snr_db_min)
    elif kind == "determinism":
        res = compare_pair(out, ref, tol, rtol=tol.determinism_rtol, snr_db_min=tol.determinism_snr_db_min)
    else:
        res = compare_pair(out, ref, tol)
    assert res.ok, f"{label}: {kind} prong failed: {res.reason} (rel {res.worst_rel_err:.3e}, SNR {res.snr_db:.1f})"


ADV_FILLS = {
    "zeros": lambda t: torch.zeros_like(t),
    "ones": lambda t: torch.ones_like(t),
    "neg_ones": lambda t: -torch.ones_like(t),
    "large": lambda t: torch.full_like(t, 1.0e3),
    "neg_large": lambda t: torch.full_like(t, -1.0e3),
    "small": lambda t: torch.full_like(t, 1.0e-3),
    "sign_alt": lambda t: ((torch.arange(t.numel(), device=t.device) % 2) * 2 - 1).to(t.dtype).reshape(t.shape),
}


def adversarial(inputs):
    """Yield ``(name, inputs)`` with every floating tensor replaced by the fill."""
    for name, fill in ADV_FILLS.items():
        yield name, tuple(fill(t) if torch.is_tensor(t) and torch.is_floating_point(t) else t for t in inputs)


def bit_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    if a.shape != b.shape or a.dtype != b.dtype:
        return False
    if a.dtype in (torch.bfloat16, torch.float16):
        return torch.equal(a.view(torch.int16), b.view(torch.int16))
    if a.dtype == torch.float32:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a, b)


def finite_snr(snr: float) -> str:
    return "inf" if not math.isfinite(snr) or snr >= 999 else f"{snr:.1f}"
