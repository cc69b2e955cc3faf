"""GPU parity: top-1 grouped expert GEMM (vs the fp32 oracle), token permute /
unpermute (bit-exact) and the expert / align offsets (exact)."""

from __future__ import annotations

import pytest
import torch

import kore_amd
from kore_amd import workloads as W
from oracle.moe import (expert_offsets_ref, grouped_gemm_fp8_ref, grouped_gemm_ref, permute_ref, trace32_bias,
                        unpermute_ref)
from tests.fourprong import bit_equal, verdict

pytestmark = pytest.mark.gpu

ROW_SAMPLE_FLOPS = 2e11  # above this the oracle runs on a row sample of the output


def _grouped(gpu, M, E, N, K, seed=0, ids=None):
    """Inputs are drawn on the GPU (the expert weights of the large shapes are GBs);
    the oracle gets the sampled rows and only the experts they use."""
    hidden, w, ti = W.grouped_inputs(M, E, N, K, seed=seed, device=gpu, router_bias=trace32_bias(E))
    if ids is not None:
        ti = ids.to(gpu)
    out = kore_amd.grouped_gemm(hidden, w, ti)
    assert out.shape == (M, N) and out.dtype == torch.bfloat16
    rows = torch.arange(M, device=gpu)
    if 2.0 * M * N * K > ROW_SAMPLE_FLOPS:
        rows = torch.unique(torch.cat([torch.arange(0, M, max(1, M // 96)), torch.tensor([M - 1])])).to(gpu)
    t = ti[rows].long()
    used = torch.unique(t[(t >= 0) & (t < E)])
    remap = torch.full((E,), -1, dtype=torch.long, device=gpu)
    remap[used] = torch.arange(used.numel(), device=gpu)
    local = torch.where((t >= 0) & (t < E), remap[t.clamp(0, E - 1)], torch.full_like(t, -1))
    wsub = w[used] if used.numel() else w[:1]
    ref = grouped_gemm_ref(hidden[rows].cpu(), wsub.cpu(), local.to(torch.int32).cpu())
    return out[rows].cpu(), ref


# moe_grouped_gemm_bf16/task.yaml:11-16 (minimal, primary, validation) and the breadth
# grouped-GEMM catalog (kore/tasks/breadth/moe_ext.py:220-224, K = 4095 included).
@pytest.mark.parametrize("M,E,N,K", [(64, 8, 128, 128), (4096, 32, 2048, 4096), (8192, 64, 1024, 2048),
                                     (1024, 256, 512, 2048), (512, 32, 1536, 4096), (64, 8, 256, 256),
                                     (4096, 256, 2048, 4096), (512, 64, 4096, 4095)])
def test_grouped_gemm_task_shapes(gpu, M, E, N, K):
    out, ref = _grouped(gpu, M, E, N, K)
    verdict(out, ref, "grouped", "bf16", f"M{M} E{E} N{N} K{K}")


@pytest.mark.parametrize("M,E,N,K", [(1, 4, 128, 64), (33, 3, 384, 200), (700, 5, 256, 512), (96, 2, 640, 136),
                                     (4000, 8, 100, 96)])
def test_grouped_gemm_ragged(gpu, M, E, N, K):
    """Decode (32-row) and prefill (256-row) tiles, K not a multiple of 64 (register-
    staged path), N padded to 128 on the host, one-token and empty experts."""
    out, ref = _grouped(gpu, M, E, N, K, seed=M)
    verdict(out, ref, "grouped", "bf16", f"M{M} E{E} N{N} K{K}")


def test_grouped_gemm_invalid_ids_and_determinism(gpu):
    M, E, N, K = 300, 6, 256, 256
    hg, wg, tg = W.grouped_inputs(M, E, N, K, seed=3, device=gpu)
    tg = tg.clone()
    tg[::7] = -1
    tg[3::11] = E + 2
    out, ref = _grouped(gpu, M, E, N, K, seed=3, ids=tg)
    assert (out[::7] == 0).all() and (out[3::11] == 0).all()
    verdict(out, ref, "grouped", "bf16", "invalid ids")
    a = kore_amd.grouped_gemm(hg, wg, tg)
    b = kore_amd.grouped_gemm(hg, wg, tg)
    assert bit_equal(a, b)


def test_grouped_gemm_all_one_expert(gpu):
    """Every token on one expert equals a dense GEMM with that expert's weight."""
    M, E, N, K = 777, 4, 512, 1024
    hidden, w, _ = W.grouped_inputs(M, E, N, K, seed=9)
    ti = torch.full((M,), 2, dtype=torch.int32)
    out = kore_amd.grouped_gemm(hidden.to(gpu), w.to(gpu), ti.to(gpu)).cpu()
    dense = (hidden.float() @ w[2].float().t()).to(torch.bfloat16)
    verdict(out, dense, "grouped", "bf16", "one expert")


def _grouped_fp8(gpu, M, E, N, K, seed=0, ids=None):
    xq, wq, xs, ws, ti = W.grouped_fp8_inputs(M, E, N, K, seed=seed, device=gpu, router_bias=trace32_bias(E))
    if ids is not None:
        ti = ids.to(gpu)
    out = kore_amd.grouped_gemm_fp8(xq, wq, xs, ws, ti)
    assert out.shape == (M, N) and out.dtype == torch.bfloat16
    rows = torch.arange(M, device=gpu)
    if 2.0 * M * N * K > ROW_SAMPLE_FLOPS:
        rows = torch.unique(torch.cat([torch.arange(0, M, max(1, M // 96)), torch.tensor([M - 1])])).to(gpu)
    t = ti[rows].long()
    valid = (t >= 0) & (t < E)
    used = torch.unique(t[valid])
    remap = torch.full((E,), -1, dtype=torch.long, device=gpu)
    remap[used] = torch.arange(used.numel(), device=gpu)
    local = torch.where(valid, remap[t.clamp(0, E - 1)], torch.full_like(t, -1))
    sel = used if used.numel() else torch.zeros(1, dtype=torch.long, device=gpu)
    ref = grouped_gemm_fp8_ref(xq[rows].cpu(), wq[sel].cpu(), xs[rows].cpu(), ws[sel].cpu(),
                               local.to(torch.int32).cpu())
    return out[rows].cpu(), ref


# moe_grouped_gemm_fp8/task.yaml:11-16 and the breadth fp8 grouped catalog
# (moe_ext.py:219-224, K = 4095 padded on the host).
@pytest.mark.parametrize("M,E,N,K", [(64, 8, 256, 256), (4096, 32, 2048, 4096), (8192, 64, 1024, 2048),
                                     (1024, 256, 512, 2048), (512, 32, 1536, 4096), (16384, 128, 4096, 4096),
                                     (4096, 256, 2048, 4096), (512, 64, 4096, 4095)])
def test_grouped_gemm_fp8_task_shapes(gpu, M, E, N, K):
    out, ref = _grouped_fp8(gpu, M, E, N, K)
    verdict(out, ref, "grouped_fp8", "fp8", f"M{M} E{E} N{N} K{K}")


@pytest.mark.parametrize("M,E,N,K", [(1, 4, 128, 128), (33, 3, 384, 256), (700, 5, 256, 512), (2000, 2, 640, 384),
                                     (9000, 4, 512, 256), (1100, 16, 768, 512), (300, 6, 200, 100)])
def test_grouped_gemm_fp8_ragged(gpu, M, E, N, K):
    """128-row and (M >= 64 E, N % 256 == 0) 256-row tiles, N not a multiple of 256,
    one-token experts, and odd N / K padded on the host."""
    out, ref = _grouped_fp8(gpu, M, E, N, K, seed=M)
    verdict(out, ref, "grouped_fp8", "fp8", f"M{M} E{E} N{N} K{K}")


def test_grouped_gemm_fp8_invalid_ids_one_expert_determinism(gpu):
    M, E, N, K = 600, 5, 512, 512
    xq, wq, xs, ws, ti = W.grouped_fp8_inputs(M, E, N, K, seed=4, device=gpu)
    bad = ti.clone()
    bad[::9] = -1
    bad[4::13] = E
    out, ref = _grouped_fp8(gpu, M, E, N, K, seed=4, ids=bad)
    assert (out[::9] == 0).all() and (out[4::13] == 0).all()
    verdict(out, ref, "grouped_fp8", "fp8", "invalid ids")
    a = kore_amd.grouped_gemm_fp8(xq, wq, xs, ws, ti)
    assert bit_equal(a, kore_amd.grouped_gemm_fp8(xq, wq, xs, ws, ti))
    # every token on expert 1 equals the dense a8w8 GEMM with that expert's weight
    one = torch.full((M,), 1, dtype=torch.int32, device=gpu)
    g1 = kore_amd.grouped_gemm_fp8(xq, wq, xs, ws, one)
    d1 = kore_amd.gemm_a8w8(xq, wq[1], xs, ws[1].reshape(1, N))
    assert bit_equal(g1, d1)


def test_registered_grouped_ops_reject_and_stride(gpu):
    """torch.ops.korehip.grouped_gemm_fp8 called directly (no Python layer): a short
    expert_ids raises ValueError before anything is launched, and a strided x_scale
    column is read with its real stride (bit-equal to the contiguous call)."""
    M, E, N, K = 256, 4, 256, 256
    xq, wq, xs, ws, ti = W.grouped_fp8_inputs(M, E, N, K, seed=7, device=gpu)
    ops = torch.ops.korehip
    with pytest.raises(ValueError, match="one id per row"):
        ops.grouped_gemm_fp8(xq, wq, xs, ws, ti[: M // 2])
    with pytest.raises(ValueError, match="w_scale"):
        ops.grouped_gemm_fp8(xq, wq, xs, ws[:, : N // 2], ti)
    ref = ops.grouped_gemm_fp8(xq, wq, xs, ws, ti)
    wide = torch.zeros((M, 3), dtype=torch.float32, device=gpu)
    wide[:, 1] = xs[:, 0]
    strided = wide[:, 1:2]  # [M,1], stride 3 along M
    assert strided.stride(0) == 3
    assert bit_equal(ops.grouped_gemm_fp8(xq, wq, strided, ws, ti), ref)
    hidden, w, ti16 = W.grouped_inputs(M, E, N, K, seed=7, device=gpu)
    with pytest.raises(ValueError, match="one id per row"):
        ops.grouped_gemm(hidden, w, ti16[:-1])
    with pytest.raises(ValueError, match="one src row per index"):
        ops.scatter_rows(hidden, torch.arange(M + 1, dtype=torch.int32, device=gpu))


def _sort_idx(M, E, seed):
    _, _, ti = W.grouped_inputs(M, E, 128, 8, seed=seed, router_bias=trace32_bias(E))
    return torch.argsort(ti, stable=True).to(torch.int32)


# moe_permute_bf16/task.yaml:12-17 and the breadth permute catalog (moe_ext.py:207-212).
@pytest.mark.parametrize("M,E,D", [(64, 8, 128), (8192, 256, 7168), (4096, 32, 4096), (2048, 64, 2048),
                                   (1024, 256, 5120), (4095, 64, 4096)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_permute_unpermute_task_shapes(gpu, M, E, D, dtype):
    g = torch.Generator().manual_seed(M + D)
    hidden = torch.randn((M, D), generator=g).to(dtype)
    sidx = _sort_idx(M, E, M)
    perm = kore_amd.moe_permute(hidden.to(gpu), sidx.to(gpu))
    assert bit_equal(perm.cpu(), permute_ref(hidden, sidx))
    back = kore_amd.moe_unpermute(perm, sidx.to(gpu))
    assert bit_equal(back.cpu(), unpermute_ref(permute_ref(hidden, sidx), sidx))
    assert bit_equal(back.cpu(), hidden)  # unpermute o permute = identity for a permutation


@pytest.mark.parametrize("M,D,dtype", [(5, 3, torch.bfloat16), (17, 1, torch.float16), (9, 7, torch.float32),
                                       (40, 13, torch.uint8)])
def test_permute_odd_rows(gpu, M, D, dtype):
    """Row sizes that are not a multiple of 16 bytes take the byte-copy path."""
    hidden = torch.arange(M * D, dtype=torch.float32).reshape(M, D).to(dtype)
    sidx = torch.randperm(M, generator=torch.Generator().manual_seed(M)).to(torch.int32)
    perm = kore_amd.moe_permute(hidden.to(gpu), sidx.to(gpu))
    assert bit_equal(perm.cpu(), permute_ref(hidden, sidx))
    assert bit_equal(kore_amd.moe_unpermute(perm, sidx.to(gpu)).cpu(), hidden)


# breadth offsets / align_offsets catalog (moe_ext.py:213-218), block 64 (ALIGN_BLOCK).
@pytest.mark.parametrize("M,E", [(64, 8), (4096, 64), (16384, 128), (8192, 256), (4095, 64)])
@pytest.mark.parametrize("block", [1, 64])
def test_expert_offsets_exact(gpu, M, E, block):
    _, _, ti = W.grouped_inputs(M, E, 128, 8, seed=E, router_bias=trace32_bias(E))
    if block == 1:
        off = kore_amd.moe_expert_offsets(ti.to(gpu), E)
    else:
        off = kore_amd.moe_align_block_offsets(ti.to(gpu), E, block)
    assert off.dtype == torch.int32 and off.shape == (E + 1,)
    assert torch.equal(off.cpu(), expert_offsets_ref(ti, E, block))
