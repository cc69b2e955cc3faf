"""GPU parity: OCP-e4m3 a8w8 block-scaled GEMM vs the CPU dequant oracle."""

from __future__ import annotations

import pytest
import torch

import kore_amd
from kore_amd import workloads as W
from oracle.quant import matmul_blockscale_ref, quant_128x128_fp8, quant_1x128_fp8
from tests.fourprong import bit_equal, pair_only, verdict

pytestmark = pytest.mark.gpu


def _run(gpu, xq, wq, xs, ws):
    return kore_amd.gemm_a8w8_blockscale(xq.to(gpu), wq.to(gpu), xs.to(gpu), ws.to(gpu))


@pytest.mark.parametrize("M", [2048, 512, 128, 16])
def test_fp8_config_sweep(gpu, M):
    """X, W ~ N(0,1), N=7168, K=4096, M in {2048, 512, 128, 16}."""
    xq, wq, xs, ws = W.fp8_inputs(M, 7168, 4096, seed=0)
    out = _run(gpu, xq, wq, xs, ws)
    ref = matmul_blockscale_ref(xq, wq, xs, ws)
    verdict(out, ref, "blockscale", "fp8", f"M={M}")
    # |o-r| <= 1e-2 + 1e-2|r| as well as the task tolerance
    verdict(out, ref, "blockscale_genv", "fp8", f"M={M} (1e-2)")


@pytest.mark.parametrize("M,N,K", [(128, 256, 256), (4095, 512, 512), (300, 384, 640), (256, 128, 128), (200, 256, 128)])
@pytest.mark.parametrize("seed", range(3))
def test_fp8_task_shapes(gpu, M, N, K, seed):
    """gemm_fp8_a8w8_blockscale shapes incl. the non-aligned M=4095, task draw N(0,1)*0.2
    (kore/tasks/gemm_fp8_a8w8_blockscale/reference.py:46-59)."""
    xq, wq, xs, ws = W.fp8_inputs(M, N, K, seed=seed, scale=0.2)
    out = _run(gpu, xq, wq, xs, ws)
    ref = matmul_blockscale_ref(xq, wq, xs, ws)
    verdict(out, ref, "blockscale", "fp8", f"{M}x{N}x{K} seed {seed}")
    pair_only(out, ref, "fp8", f"{M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(128, 4096, 4096), (100, 7168, 4096), (65, 4096, 8192), (97, 7168, 5120)])
def test_fp8_skinny_ragged_rows(gpu, M, N, K):
    """The skinny (M <= 128) kernel at a full 128-row tile and at ragged row counts
    (rows past M repeat row M-1 and are never stored), K up to 64 blocks and K/128 not
    a multiple of the wave count.  Repeated calls must be bit-identical (fixed-order
    cross-wave sum)."""
    xq, wq, xs, ws = W.fp8_inputs(M, N, K, seed=M + N + K, scale=0.2)
    out = _run(gpu, xq, wq, xs, ws)
    ref = matmul_blockscale_ref(xq, wq, xs, ws)
    verdict(out, ref, "blockscale", "fp8", f"{M}x{N}x{K}")
    verdict(out, ref, "blockscale_genv", "fp8", f"{M}x{N}x{K} (1e-2)")
    assert bit_equal(out, _run(gpu, xq, wq, xs, ws)), "split-K result not reproducible"


@pytest.mark.parametrize("M,N,K", [(256, 7168, 4096), (384, 4096, 2048), (512, 1024, 512), (640, 2048, 1536)])
def test_fp8_128_tiles(gpu, M, N, K):
    """Problems with too few tiles for the 256-row kernels run 128x128 tiles on 4 waves
    (four LDS slots, four-block scale loads): K from 4 to 32 blocks, 80 to 112 tiles."""
    xq, wq, xs, ws = W.fp8_inputs(M, N, K, seed=M + N + K, scale=0.2)
    out = _run(gpu, xq, wq, xs, ws)
    ref = matmul_blockscale_ref(xq, wq, xs, ws)
    verdict(out, ref, "blockscale", "fp8", f"{M}x{N}x{K}")
    verdict(out, ref, "blockscale_genv", "fp8", f"{M}x{N}x{K} (1e-2)")
    assert bit_equal(out, _run(gpu, xq, wq, xs, ws)), "not reproducible"


@pytest.mark.parametrize("M,N,K", [(512, 7168, 4096), (512, 6144, 1024), (512, 7168, 1536), (256, 16384, 1024),
                                   (512, 7168, 512)])
def test_fp8_ksplit_tiles(gpu, M, N, K):
    """128 x 128 tiles covering three quarters of the CUs with contiguous scales run the K-split
    kernel: the two waves of a SIMD take the even and the odd K blocks of the same outputs
    and their partial sums are added once after the loop.  Parity at the task tolerance and
    the 1e-2 bound, bit-exact reruns, and power-of-two scale invariance (each block's scale
    multiplies its own partial exactly once); K from 4 to 32 blocks (2 to 16 stages).
    Not bit-equal to the other tile kernels: the even and odd K blocks are summed apart."""
    xq, wq, xs, ws = W.fp8_inputs(M, N, K, seed=M + N + K, scale=0.2)
    out = _run(gpu, xq, wq, xs, ws)
    ref = matmul_blockscale_ref(xq, wq, xs, ws)
    verdict(out, ref, "blockscale", "fp8", f"{M}x{N}x{K}")
    verdict(out, ref, "blockscale_genv", "fp8", f"{M}x{N}x{K} (1e-2)")
    pair_only(out, ref, "fp8", f"{M}x{N}x{K}")
    assert bit_equal(_run(gpu, xq, wq, xs, ws), out), "not reproducible"
    assert bit_equal(_run(gpu, xq, wq, xs * 4, ws), out * 4)
    assert bit_equal(_run(gpu, xq, wq, xs, ws * 0.5), out * 0.5)


@pytest.mark.parametrize("M,N,K", [(4000, 3072, 640), (4000, 3072, 512), (3840, 3072, 1024),
                                   (1100, 6016, 512), (1100, 6016, 640), (768, 7168, 1024), (700, 7168, 512)])
def test_fp8_wide_tiles(gpu, M, N, K):
    """Problems with at least 192 tiles of 256x256 run on the 256x256 (two-slot) kernel:
    a partial last M tile (M=4000), per-step scale loads (K/128 = 5) and four-step
    scale loads (K/128 = 4, 8).  N = 6016 (not a multiple of 256) with 235 tiles of
    256x128 runs the 256x128 (three-slot) kernel, and so do M = 768 / 700 at N = 7168
    (168 tiles, where 336 / 336 tiles of 128x128 would need two rounds of the CUs);
    smaller problems run 128x128 tiles."""
    xq, wq, xs, ws = W.fp8_inputs(M, N, K, seed=M + K, scale=0.2)
    out = _run(gpu, xq, wq, xs, ws)
    ref = matmul_blockscale_ref(xq, wq, xs, ws)
    verdict(out, ref, "blockscale", "fp8", f"{M}x{N}x{K}")
    pair_only(out, ref, "fp8", f"{M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(2048, 7168, 512), (1024, 7168, 2048), (2048, 4480, 1024), (4096, 7168, 512)])
def test_fp8_224_tiles(gpu, M, N, K):
    """M % 256 == 0, N % 224 == 0, K % 512 == 0 with contiguous scales, where 256 x 224
    tiles take fewer CU-rounds than 256 x 256 ones (one tile per CU at 2048 x 7168 and
    1024 x 7168; N = 4480 is not a multiple of 256; 4096 x 7168 runs two rounds):
    parity, bit-exact reruns and power-of-two scale invariance.  Every output element
    sums the same partial products in the same order as the 256 x 256 / 256 x 128
    kernels, which column-major x_scale views select: the two must agree bit for bit."""
    xq, wq, xs, ws = W.fp8_inputs(M, N, K, seed=M + N + K, scale=0.2)
    out = _run(gpu, xq, wq, xs, ws)
    ref = matmul_blockscale_ref(xq, wq, xs, ws)
    verdict(out, ref, "blockscale", "fp8", f"{M}x{N}x{K}")
    verdict(out, ref, "blockscale_genv", "fp8", f"{M}x{N}x{K} (1e-2)")
    pair_only(out, ref, "fp8", f"{M}x{N}x{K}")
    assert bit_equal(_run(gpu, xq, wq, xs, ws), out)
    assert bit_equal(_run(gpu, xq, wq, xs * 4, ws), out * 4)
    xs_cm = xs.t().contiguous().t()
    assert bit_equal(_run(gpu, xq, wq, xs_cm, ws), out), "differs from the 256-row tile kernels"


@pytest.mark.parametrize("regime", ["zeros", "ones", "large", "small"])
def test_fp8_adversarial(gpu, regime):
    """The task's authored adversarial battery (kore/tasks/vendor_ops.py:526-543)."""
    M, N, K = 256, 512, 1024
    val = {"zeros": 0.0, "ones": 1.0, "large": 10.0, "small": 1e-2}[regime]
    xq, xs = quant_1x128_fp8(torch.full((M, K), val))
    wq, ws = quant_128x128_fp8(torch.full((N, K), val))
    out = _run(gpu, xq, wq, xs, ws)
    verdict(out, matmul_blockscale_ref(xq, wq, xs, ws), "blockscale", "fp8", regime)


def test_fp8_scale_invariance_and_determinism(gpu):
    """Doubling x_scale doubles Y exactly (power-of-two scale invariance)."""
    xq, wq, xs, ws = W.fp8_inputs(512, 1024, 1024, seed=9)
    y1 = _run(gpu, xq, wq, xs, ws)
    y2 = _run(gpu, xq, wq, xs * 2, ws)
    assert bit_equal(y2, y1 * 2)
    assert bit_equal(_run(gpu, xq, wq, xs, ws), y1)


@pytest.mark.parametrize("M,K", [(512, 4096), (300, 1536), (256, 640)])
def test_fp8_scale_and_row_layouts(gpu, M, K):
    """Column-major scale tensors (x_scale stride (1, M), w_scale stride (1, N/128)) and
    padded operand rows give the same result as the contiguous layout: the kernel reads
    scales through their strides (per-K-step loads) and the contiguous case batches four
    K steps of x_scale per load when K/128 % 4 == 0."""
    N = 384
    xq, wq, xs, ws = W.fp8_inputs(M, N, K, seed=4)
    base = _run(gpu, xq, wq, xs, ws)
    verdict(base, matmul_blockscale_ref(xq, wq, xs, ws), "blockscale", "fp8", f"{M}x{N}x{K}")
    xs_t = xs.t().contiguous().t()
    ws_t = ws.t().contiguous().t()
    assert xs_t.stride() == (1, M)
    assert bit_equal(_run(gpu, xq, wq, xs_t, ws_t), base)
    pad = torch.zeros(M, K + 128, dtype=xq.dtype)
    pad[:, :K] = xq
    padw = torch.zeros(N, K + 256, dtype=wq.dtype)
    padw[:, :K] = wq
    assert bit_equal(_run(gpu, pad[:, :K], padw[:, :K], xs, ws), base)


def test_fp8_rejects_unaligned(gpu):
    xq, wq, xs, ws = W.fp8_inputs(64, 256, 256, seed=0)
    with pytest.raises(ValueError):
        kore_amd.gemm_a8w8_blockscale(xq[:, :200].to(gpu), wq[:, :200].to(gpu), xs.to(gpu), ws.to(gpu))


@pytest.mark.parametrize("M", [1, 7, 16, 17, 33, 64, 100, 128])
@pytest.mark.parametrize("N,K", [(128, 128), (384, 384), (1024, 1152), (256, 2048)])
def test_fp8_skinny(gpu, M, N, K):
    """M <= 128 runs the weight-streaming split-K kernel: ragged M (rows padded to 16,
    32, 64 or 128), K/128 blocks fewer than, not a multiple of, and a multiple of the
    8 waves that split them."""
    xq, wq, xs, ws = W.fp8_inputs(M, N, K, seed=M * 7 + K, scale=0.2)
    out = _run(gpu, xq, wq, xs, ws)
    ref = matmul_blockscale_ref(xq, wq, xs, ws)
    verdict(out, ref, "blockscale", "fp8", f"{M}x{N}x{K}")
    verdict(out, ref, "blockscale_genv", "fp8", f"{M}x{N}x{K} (1e-2)")
    assert bit_equal(_run(gpu, xq, wq, xs, ws), out)  # fixed-order cross-wave sum


@pytest.mark.parametrize("M", [16, 100])
def test_fp8_skinny_layouts(gpu, M):
    """Skinny kernel: column-major scales and padded operand rows match the contiguous
    layout bit for bit; doubling x_scale doubles Y exactly."""
    N, K = 384, 1536
    xq, wq, xs, ws = W.fp8_inputs(M, N, K, seed=11)
    base = _run(gpu, xq, wq, xs, ws)
    verdict(base, matmul_blockscale_ref(xq, wq, xs, ws), "blockscale", "fp8", f"{M}x{N}x{K}")
    xs_t = xs.t().contiguous().t()
    ws_t = ws.t().contiguous().t()
    assert bit_equal(_run(gpu, xq, wq, xs_t, ws_t), base)
    pad = torch.zeros(M, K + 128, dtype=xq.dtype)
    pad[:, :K] = xq
    padw = torch.zeros(N, K + 256, dtype=wq.dtype)
    padw[:, :K] = wq
    assert bit_equal(_run(gpu, pad[:, :K], padw[:, :K], xs, ws), base)
    assert bit_equal(_run(gpu, xq, wq, xs * 2, ws), base * 2)
