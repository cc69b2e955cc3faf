"""Golden fixtures (``tests/golden/golden.pt``, written by ``tests/golden/make_golden.py``).

CPU: the seeded generators still draw the stored inputs, and the oracle still
produces the stored outputs bit for bit.  GPU: every HIP operator, called through
the package, matches the stored outputs within its task tolerance (SNR + allclose)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from kore_amd import workloads as W
from oracle.gemm import batched_gemm_ref, gemm_backward_ref, gemm_fusion_ref, matmul_ref
from oracle.moe import moe_align_ref, moe_ref, trace32_bias
from oracle.quant import matmul_a8w8_ref, matmul_blockscale_ref
from tests.fourprong import verdict

GOLDEN = torch.load(Path(__file__).parent / "golden" / "golden.pt", weights_only=True)
FP8 = torch.float8_e4m3fn


def _eq(x, y):
    return x.dtype == y.dtype and x.shape == y.shape and torch.equal(x.view(torch.uint8) if x.dtype == FP8 else x,
                                                                      y.view(torch.uint8) if y.dtype == FP8 else y)


def test_golden_inputs_are_the_seeded_draws():
    a, b = W.dense_inputs(64, 96, 128, seed=11)
    assert _eq(a.contiguous(), GOLDEN["gemm_bf16"]["a"]) and _eq(b.t().contiguous(), GOLDEN["gemm_bf16"]["bt"])
    a, b, bias = W.fused_inputs(64, 128, 256, seed=12)
    assert _eq(bias, GOLDEN["gemm_bias_act_fp16"]["bias"]) and _eq(a, GOLDEN["gemm_bias_act_fp16"]["a"])
    xq, wq, xs, ws = W.fp8_inputs(40, 256, 384, seed=14)
    assert _eq(xq.view(torch.uint8), GOLDEN["fp8_blockscale"]["xq"]) and _eq(ws, GOLDEN["fp8_blockscale"]["ws"])
    hidden, w1, w2, tw, ti = W.moe_inputs(24, 4, 2, 128, 128, seed=15, wscale=0.05, router_bias=trace32_bias(4))
    assert _eq(ti, GOLDEN["fused_moe"]["ti"]) and _eq(w2, GOLDEN["fused_moe"]["w2"])
    xq, wq, xs, ws = W.a8w8_inputs(24, 256, 384, "int8", "pertoken", seed=17)
    assert _eq(xq, GOLDEN["a8w8_int8"]["xq"]) and _eq(ws, GOLDEN["a8w8_int8"]["ws"])
    x, w, dy = W.backward_inputs(48, 40, 72, seed=18)
    g = GOLDEN["gemm_backward_bf16"]
    assert _eq(x, g["x"]) and _eq(w, g["w"]) and _eq(dy, g["dy"])


def _ulp_eq(x, y):
    """Oracle outputs against the fixture: equal, except that a host whose BLAS sums in
    another order may round an element to the neighbouring value (one unit in the last
    place of the output dtype)."""
    if x.dtype != y.dtype or x.shape != y.shape:
        return False
    if x.dtype not in (torch.bfloat16, torch.float16):
        return torch.equal(x, y)
    ulp = 2.0 ** (-7 if x.dtype == torch.bfloat16 else -10)
    yf = y.float()
    return bool(((x.float() - yf).abs() <= ulp * yf.abs().clamp(min=2.0 ** -14)).all())


def test_oracle_reproduces_golden_outputs():
    g = GOLDEN["gemm_bf16"]
    assert _ulp_eq(matmul_ref(g["a"], g["bt"].t()), g["out"])
    g = GOLDEN["gemm_bias_act_fp16"]
    for act in ("gelu", "relu", "silu"):
        assert _ulp_eq(gemm_fusion_ref(g["a"], g["bt"].t(), g["bias"], act), g[f"out_{act}"])
    g = GOLDEN["batched_bf16"]
    assert _ulp_eq(batched_gemm_ref(g["a"], g["bt"].transpose(1, 2)), g["out"])
    g = GOLDEN["fp8_blockscale"]
    assert _ulp_eq(matmul_blockscale_ref(g["xq"].view(FP8), g["wq"].view(FP8), g["xs"], g["ws"]), g["out"])
    g = GOLDEN["fused_moe"]
    assert _ulp_eq(moe_ref(g["hidden"], g["w1"], g["w2"], g["tw"], g["ti"]), g["out"])
    g = GOLDEN["a8w8_fp8"]
    assert _ulp_eq(matmul_a8w8_ref(g["xq"].view(FP8), g["wq"].view(FP8), g["xs"], g["ws"]), g["out"])
    g = GOLDEN["a8w8_int8"]
    assert _ulp_eq(matmul_a8w8_ref(g["xq"], g["wq"], g["xs"], g["ws"]), g["out"])
    g = GOLDEN["gemm_backward_bf16"]
    dx, dw = gemm_backward_ref(g["x"], g["w"], g["dy"])
    # fp32 gradients: another CPU's BLAS may sum in another order, so within fp32 rounding
    assert torch.allclose(dx, g["dx"], rtol=1e-5, atol=1e-5) and torch.allclose(dw, g["dw"], rtol=1e-5, atol=1e-5)
    g = GOLDEN["moe_align"]
    off, srt, blk = moe_align_ref(g["ti"], int(g["E"]), int(g["block"]))
    assert np.array_equal(off, g["offsets"].numpy()) and np.array_equal(srt, g["sorted"].numpy())
    assert np.array_equal(blk, g["block_expert"].numpy())


@pytest.mark.gpu
def test_hip_matches_golden(gpu):
    import kore_amd

    d = lambda t: t.to(gpu)  # noqa: E731
    g = GOLDEN["gemm_bf16"]
    verdict(kore_amd.gemm(d(g["a"]), d(g["bt"]).t()), g["out"], "gemm", "bf16", "golden gemm_bf16")
    g = GOLDEN["gemm_bias_act_fp16"]
    for act in ("gelu", "relu", "silu"):
        out = kore_amd.gemm_fused(d(g["a"]), d(g["bt"]).t(), d(g["bias"]), act)
        verdict(out, g[f"out_{act}"], "gemm_fusion", "fp16", f"golden gemm_bias_{act}")
    g = GOLDEN["batched_bf16"]
    verdict(kore_amd.batched_gemm(d(g["a"]), d(g["bt"]).transpose(1, 2)), g["out"], "batched_gemm", "bf16",
            "golden batched")
    g = GOLDEN["fp8_blockscale"]
    out = kore_amd.gemm_a8w8_blockscale(d(g["xq"]).view(FP8), d(g["wq"]).view(FP8), d(g["xs"]), d(g["ws"]))
    verdict(out, g["out"], "blockscale", "fp8", "golden fp8_blockscale")
    g = GOLDEN["a8w8_fp8"]
    out = kore_amd.gemm_a8w8(d(g["xq"]).view(FP8), d(g["wq"]).view(FP8), d(g["xs"]), d(g["ws"]))
    verdict(out, g["out"], "a8w8", "fp8", "golden a8w8_fp8")
    g = GOLDEN["a8w8_int8"]
    out = kore_amd.gemm_a8w8(d(g["xq"]), d(g["wq"]), d(g["xs"]), d(g["ws"]))
    verdict(out, g["out"], "a8w8", "int8", "golden a8w8_int8")
    g = GOLDEN["fused_moe"]
    out = kore_amd.fused_moe(d(g["hidden"]), d(g["w1"]), d(g["w2"]), d(g["tw"]), d(g["ti"]))
    verdict(out, g["out"], "fused_moe", "bf16", "golden fused_moe")
    g = GOLDEN["gemm_backward_bf16"]
    dx, dw = kore_amd.gemm_backward(d(g["x"]), d(g["w"]), d(g["dy"]))
    verdict(dx, g["dx"], "gemm_backward_dx", "bf16", "golden gemm_backward dx")
    verdict(dw, g["dw"], "gemm_backward_dw", "bf16", "golden gemm_backward dw")
    g = GOLDEN["moe_align"]
    off, srt, blk = kore_amd.moe_align(d(g["ti"]), int(g["E"]), int(g["block"]))
    n = int(g["offsets"][-1])
    assert torch.equal(off.cpu(), g["offsets"]) and torch.equal(srt.cpu()[:n], g["sorted"])
    assert torch.equal(blk.cpu()[: n // int(g["block"])], g["block_expert"])
