"""Write the golden fixtures: small seeded inputs and the CPU oracle's outputs.

``python tests/golden/make_golden.py`` (from the repository root) rewrites
``tests/golden/golden.pt``.  Every fixture is a dict of plain tensors, loadable with
``torch.load(..., weights_only=True)``.  The oracle that fills in the expected
outputs is pinned independently (closed forms, fp64 brute force, second paths and
the reference's own known-answer tests in ``tests/test_oracle_*.py``); the fixtures
freeze its outputs so a later change to the oracle, the input generators or the
kernels is caught against fixed numbers.
"""

from __future__ import annotations

import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from kore_amd import workloads as W  # noqa: E402
from oracle.gemm import batched_gemm_ref, gemm_backward_ref, gemm_fusion_ref, matmul_ref  # noqa: E402
from oracle.moe import moe_align_ref, moe_ref, trace32_bias  # noqa: E402
from oracle.quant import matmul_a8w8_ref, matmul_blockscale_ref  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.pt")


def build() -> dict:
    g = {}
    a, b = W.dense_inputs(64, 96, 128, seed=11)
    g["gemm_bf16"] = {"a": a.contiguous(), "bt": b.t().contiguous(), "out": matmul_ref(a, b)}
    a, b, bias = W.fused_inputs(64, 128, 256, seed=12)
    g["gemm_bias_act_fp16"] = {"a": a.contiguous(), "bt": b.t().contiguous(), "bias": bias}
    for act in ("gelu", "relu", "silu"):
        g["gemm_bias_act_fp16"][f"out_{act}"] = gemm_fusion_ref(a, b, bias, act)
    a, b = W.batched_inputs(3, 32, 64, 128, seed=13)
    g["batched_bf16"] = {"a": a.contiguous(), "bt": b.transpose(1, 2).contiguous(), "out": batched_gemm_ref(a, b)}
    x, w, dy = W.backward_inputs(48, 40, 72, seed=18)
    dx, dw = gemm_backward_ref(x, w, dy)
    g["gemm_backward_bf16"] = {"x": x, "w": w, "dy": dy, "dx": dx, "dw": dw}
    xq, wq, xs, ws = W.fp8_inputs(40, 256, 384, seed=14)
    g["fp8_blockscale"] = {"xq": xq.view(torch.uint8), "wq": wq.view(torch.uint8), "xs": xs, "ws": ws,
                           "out": matmul_blockscale_ref(xq, wq, xs, ws)}
    for kind, seed in (("fp8", 16), ("int8", 17)):
        xq, wq, xs, ws = W.a8w8_inputs(24, 256, 384, kind, "pertoken", seed=seed)
        u8 = (lambda t: t.view(torch.uint8)) if kind == "fp8" else (lambda t: t)
        g[f"a8w8_{kind}"] = {"xq": u8(xq), "wq": u8(wq), "xs": xs, "ws": ws, "out": matmul_a8w8_ref(xq, wq, xs, ws)}
    hidden, w1, w2, tw, ti = W.moe_inputs(24, 4, 2, 128, 128, seed=15, wscale=0.05, router_bias=trace32_bias(4))
    g["fused_moe"] = {"hidden": hidden, "w1": w1, "w2": w2, "tw": tw, "ti": ti,
                      "out": moe_ref(hidden, w1, w2, tw, ti)}
    off, srt, blk = moe_align_ref(ti, 4, 32)
    g["moe_align"] = {"ti": ti, "E": torch.tensor(4), "block": torch.tensor(32),
                      "offsets": torch.as_tensor(off), "sorted": torch.as_tensor(srt), "block_expert": torch.as_tensor(blk)}
    return g


if __name__ == "__main__":
    torch.save(build(), OUT)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")
