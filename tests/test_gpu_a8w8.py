"""GPU parity: fp8 / int8 a8w8 GEMM (per-token, per-tensor, per-channel scales) vs the
CPU dequant oracle (kore/tasks/_quant_common.py:236-242), on the task shapes of
gemm_fp8_a8w8, gemm_fp8_a8w8_pertoken, gemm_fp8_a8w8_pertensor, gemm_int8_a8w8 and
genv_gemm_a8w8_{fp8,int8}."""

from __future__ import annotations

import pytest
import torch

import kore_amd
from kore_amd import workloads as W
from oracle.quant import matmul_a8w8_ref
from tests.fourprong import bit_equal, verdict

pytestmark = pytest.mark.gpu

ROW_SAMPLE_FLOPS = 3e11  # above this the oracle runs on a row sample of the output


def _check(gpu, kind, mode, M, N, K, seed=0, ta=False, task="a8w8"):
    xq, wq, xs, ws = W.a8w8_inputs(M, N, K, kind, mode, seed=seed, transpose_a=ta)
    out = kore_amd.gemm_a8w8(xq.to(gpu), wq.to(gpu), xs.to(gpu), ws.to(gpu)).cpu()
    assert out.shape == (M, N) and out.dtype == torch.bfloat16
    label = f"{kind} {mode} {M}x{N}x{K}{' TA' if ta else ''}"
    if 2.0 * M * N * K > ROW_SAMPLE_FLOPS:
        rows = torch.unique(torch.cat([torch.arange(0, M, max(1, M // 96)), torch.tensor([M - 1])]))
        ref = matmul_a8w8_ref(xq[rows], wq, xs[rows], ws)
        out = out[rows]
    else:
        ref = matmul_a8w8_ref(xq, wq, xs, ws)
    verdict(out, ref, task, kind, label)
    verdict(out, ref, "north_star", kind, label + " (1e-2)")
    return out


@pytest.mark.parametrize("M,N,K", [(8, 512, 512), (4096, 4096, 4096), (1, 4096, 4096), (8, 4096, 4096),
                                   (64, 4096, 4096)])
def test_gemm_fp8_a8w8_task(gpu, M, N, K):
    """gemm_fp8_a8w8/task.yaml shapes: per-tensor scales broadcast to [M,1] / [1,N]."""
    _check(gpu, "fp8", "pertensor", M, N, K)


@pytest.mark.parametrize("M,N,K,ta", [(8, 512, 512, False), (4096, 4096, 4096, False), (1, 4096, 4096, False),
                                      (17, 6144, 4096, False), (4097, 4096, 4096, False), (64, 4096, 4095, False),
                                      (16, 4096, 4096, True), (8192, 28672, 8192, False)])
def test_gemm_fp8_a8w8_pertoken_task(gpu, M, N, K, ta):
    """gemm_fp8_a8w8_pertoken/task.yaml shapes, incl. the K tail (4095), the M tail
    (4097), the transposed-A view and the 8192x28672x8192 gate_up shape (row-sampled)."""
    _check(gpu, "fp8", "pertoken", M, N, K, ta=ta)


@pytest.mark.parametrize("M,N,K", [(8, 512, 512), (1, 4096, 4096), (4097, 4096, 4096), (2048, 14336, 4096),
                                   (64, 4096, 4095)])
def test_gemm_fp8_a8w8_pertensor_task(gpu, M, N, K):
    _check(gpu, "fp8", "pertensor", M, N, K)


@pytest.mark.parametrize("M,N,K", [(8, 512, 512), (4096, 4096, 4096), (1, 4096, 4096), (17, 4096, 4096),
                                   (4097, 6144, 4096), (8192, 8192, 4096), (64, 4096, 4095)])
def test_gemm_int8_a8w8_task(gpu, M, N, K):
    """gemm_int8_a8w8/task.yaml shapes (per-token x, per-channel w, symmetric int8)."""
    _check(gpu, "int8", "pertoken", M, N, K)


@pytest.mark.parametrize("kind", ["fp8", "int8"])
@pytest.mark.parametrize("M,N,K", [(128, 128, 256), (4096, 4096, 4096), (8192, 8192, 1024), (2048, 14336, 8192),
                                   (4096, 4096, 4095)])
def test_genv_gemm_a8w8_task(gpu, kind, M, N, K):
    """genv_gemm_a8w8_{fp8,int8}/task.yaml shapes at the generated-task tolerance
    (per-tensor scales, kore/tasks/vendor_ops.py:266-288)."""
    _check(gpu, kind, "pertensor", M, N, K, task="a8w8_genv")


@pytest.mark.parametrize("kind", ["fp8", "int8"])
@pytest.mark.parametrize("M,N,K", [(1, 128, 128), (33, 256, 640), (100, 384, 1152), (128, 512, 256),
                                   (20, 8192, 256), (100, 8192, 384), (129, 256, 384), (300, 384, 640),
                                   (200, 300, 256), (96, 128, 100)])
def test_a8w8_paths(gpu, kind, M, N, K):
    """Every kernel path: skinny (M <= 128; 16-column workgroups below N = 8192,
    32-column ones from it), tiled (M > 128, 128x128 / 256x128 tiles), generic
    (N % 128 != 0, K % 128 != 0); ragged M throughout."""
    _check(gpu, kind, "pertoken", M, N, K, seed=M + K)


@pytest.mark.parametrize("kind", ["fp8", "int8"])
@pytest.mark.parametrize("M", [16, 512])
def test_a8w8_metamorphic_and_determinism(gpu, kind, M):
    """Bit-equal reruns; doubling x_scale doubles Y exactly; w_scale as [1,N], [N,1] or
    [N] is one operand; a padded-row view equals the contiguous operand; the generic
    kernel (reached through a column-major xq) and the MFMA kernel both meet the oracle."""
    N, K = 384, 1024
    xq, wq, xs, ws = W.a8w8_inputs(M, N, K, kind, "pertoken", seed=7)
    xg, wg, xsg, wsg = xq.to(gpu), wq.to(gpu), xs.to(gpu), ws.to(gpu)
    y = kore_amd.gemm_a8w8(xg, wg, xsg, wsg)
    assert bit_equal(kore_amd.gemm_a8w8(xg, wg, xsg, wsg), y)
    assert bit_equal(kore_amd.gemm_a8w8(xg, wg, xsg * 2, wsg), y * 2)
    assert bit_equal(kore_amd.gemm_a8w8(xg, wg, xsg, wsg.reshape(N, 1)), y)
    assert bit_equal(kore_amd.gemm_a8w8(xg, wg, xsg, wsg.reshape(N)), y)
    pad = torch.zeros(M, K + 128, dtype=xq.dtype)
    pad[:, :K] = xq
    assert bit_equal(kore_amd.gemm_a8w8(pad[:, :K].to(gpu), wg, xsg, wsg), y)
    xt = xq.t().contiguous().t().to(gpu)  # column-major xq: generic kernel
    ref = matmul_a8w8_ref(xq, wq, xs, ws)
    verdict(kore_amd.gemm_a8w8(xt, wg, xsg, wsg).cpu(), ref, "north_star", kind, f"{kind} generic kernel")
    verdict(y.cpu(), ref, "north_star", kind, f"{kind} MFMA kernel")


@pytest.mark.parametrize("kind", ["fp8", "int8"])
@pytest.mark.parametrize("regime", ["zeros", "ones", "large"])
def test_a8w8_adversarial(gpu, kind, regime):
    """Constant fills (kore/tasks/vendor_ops.py:526-543 battery) through the quantiser."""
    M, N, K = 256, 512, 1024
    val = {"zeros": 0.0, "ones": 1.0, "large": 10.0}[regime]
    xq, wq, xs, ws = W.a8w8_inputs(M, N, K, kind, "pertoken", seed=0)
    full = torch.full((M, K), val)
    qmax = 448.0 if kind == "fp8" else 127.0
    s = (full.abs().amax(-1, keepdim=True).clamp(min=1e-12) / qmax)
    xq = (full / s).clamp(-qmax, qmax)
    xq = xq.to(torch.float8_e4m3fn) if kind == "fp8" else xq.round().to(torch.int8)
    out = kore_amd.gemm_a8w8(xq.to(gpu), wq.to(gpu), s.to(gpu), ws.to(gpu)).cpu()
    verdict(out, matmul_a8w8_ref(xq, wq, s, ws), "a8w8", kind, f"{kind} {regime}")


@pytest.mark.parametrize("kind,M,N,K", [("fp8", 3000, 4096, 4096), ("fp8", 2048, 7168, 8192),
                                        ("fp8", 3000, 4096, 2048), ("int8", 3000, 4096, 2048),
                                        ("int8", 4000, 3840, 4096), ("int8", 3500, 4096, 1024)])
def test_a8w8_buffer_tile(gpu, kind, M, N, K):
    """The dense 4-wave 256x256 tile (N % 256 == 0, at least 192 tiles, K from 2048 for fp8
    and 1024 for int8): ragged M, and operands given as padded-row views, which must give
    the contiguous operands' output bit for bit; the oracle on a row sample."""
    xq, wq, xs, ws = W.a8w8_inputs(M, N, K, kind, "pertoken", seed=K + M)
    xg, wg, xsg, wsg = xq.to(gpu), wq.to(gpu), xs.to(gpu), ws.to(gpu)
    y = kore_amd.gemm_a8w8(xg, wg, xsg, wsg)
    xp = torch.zeros(M, K + 128, dtype=xq.dtype, device=gpu)
    xp[:, :K] = xg
    wp = torch.zeros(N, K + 256, dtype=wq.dtype, device=gpu)
    wp[:, :K] = wg
    assert bit_equal(kore_amd.gemm_a8w8(xp[:, :K], wp[:, :K], xsg, wsg), y)
    rows = torch.unique(torch.cat([torch.arange(0, M, max(1, M // 64)), torch.arange(M - 40, M)]))
    ref = matmul_a8w8_ref(xq[rows], wq, xs[rows], ws)
    out = y.cpu()[rows]
    label = f"{kind} buffer tile {M}x{N}x{K}"
    verdict(out, ref, "a8w8", kind, label)
    verdict(out, ref, "north_star", kind, label + " (1e-2)")


def test_a8w8_rejects_bad_inputs(gpu):
    xq, wq, xs, ws = W.a8w8_inputs(8, 128, 128, "fp8", "pertoken")
    with pytest.raises(ValueError):
        kore_amd.gemm_a8w8(xq.to(gpu), wq.to(torch.int8).to(gpu), xs.to(gpu), ws.to(gpu))
    with pytest.raises(ValueError):
        kore_amd.gemm_a8w8(xq.to(gpu), wq.to(gpu), xs[:4].to(gpu), ws.to(gpu))
