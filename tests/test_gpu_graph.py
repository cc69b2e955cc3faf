"""GPU: operators captured in a HIP graph replay to the eager result.

``bench.py`` times small kernels by graph replay, so every operator it times must
replay correctly: each case is captured once, replayed three times with eager work
and a synchronisation between replays, and every replay is compared bit for bit with
the eager output.
"""

from __future__ import annotations

import pytest
import torch

import kore_amd
from kore_amd import workloads as W

pytestmark = pytest.mark.gpu


def _cases(dev):
    a, b = W.dense_inputs(320, 256, 192, seed=1, device=dev)
    yield "gemm", lambda: kore_amd.gemm(a, b)
    a2, b2, bias = W.fused_inputs(256, 512, 256, seed=2, device=dev)
    yield "gemm_bias_gelu", lambda: kore_amd.gemm_fused(a2, b2, bias, "gelu")
    ab, bb = W.batched_inputs(4, 128, 256, 128, seed=3, device=dev)
    yield "batched", lambda: kore_amd.batched_gemm(ab, bb)
    for M in (16, 100, 512):
        xq, wq, xs, ws = W.fp8_inputs(M, 512, 1024, seed=M, device=dev)
        yield f"fp8 M={M}", (lambda xq=xq, wq=wq, xs=xs, ws=ws: kore_amd.gemm_a8w8_blockscale(xq, wq, xs, ws))
    args = W.moe_inputs(64, 8, 2, 256, 512, seed=4, device=dev, wscale=0.05)
    yield "fused_moe", lambda: kore_amd.fused_moe(*args)


def test_graph_replay_matches_eager(gpu):
    for name, fn in _cases(gpu):
        ref = fn().clone()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = fn()
        for rep in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"{name}: replay {rep} differs from eager"
            other = fn()  # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(other, ref), f"{name}: eager call after replay {rep} differs"
        del g
