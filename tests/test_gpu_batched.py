"""GPU parity: batched bf16 GEMM ``C[i] = A[i] @ B[i]^T`` vs the CPU oracle."""

from __future__ import annotations

import pytest
import torch

import kore_amd
from kore_amd import workloads as W
from oracle.gemm import batched_gemm_ref
from tests.fourprong import adversarial, bit_equal, pair_only, verdict

pytestmark = pytest.mark.gpu


def test_batched_config(gpu):
    """A[64,1024,128], B[64,128,1024] ~ N(0,1)*0.1, b = B.transpose(1,2)."""
    a, b = W.batched_inputs(64, 1024, 1024, 128, seed=0)
    out = kore_amd.batched_gemm(a.to(gpu), b.to(gpu))
    verdict(out, batched_gemm_ref(a, b), "batched_gemm", "bf16", "64x1024x1024x128")


@pytest.mark.parametrize("Bn,M,N,K", [(2, 128, 128, 256), (8, 512, 512, 512), (16, 256, 256, 1024),
                                      (4, 1024, 1024, 512), (8, 512, 513, 512)])
@pytest.mark.parametrize("seed", range(2))
def test_batched_task_shapes(gpu, Bn, M, N, K, seed):
    """genv_batched_gemm_bf16 shapes (kore/tasks/vendor_ops.py:83-89) with the task's
    [B,N,K] K-contiguous b, both scaled 1/sqrt(K) (vendor_ops.py:365-371)."""
    g = torch.Generator().manual_seed(seed)
    sc = 1.0 / K ** 0.5
    a = (torch.randn((Bn, M, K), generator=g) * sc).bfloat16()
    b = (torch.randn((Bn, N, K), generator=g) * sc).bfloat16()
    out = kore_amd.batched_gemm(a.to(gpu), b.to(gpu))
    ref = batched_gemm_ref(a, b)
    verdict(out, ref, "batched_gemm", "bf16", f"B{Bn} {M}x{N}x{K}")
    pair_only(out, ref, "bf16", f"B{Bn} {M}x{N}x{K}")


@pytest.mark.parametrize("Bn,M,N,K", [(64, 1024, 1024, 128), (4, 256, 384, 512)])
def test_batched_adversarial(gpu, Bn, M, N, K):
    """The generic adversarial fills (kore/tasks/_genops.py:855-879) through the
    persistent short-K kernel (the config's K = 128) and the tiled batched path:
    constant, alternating-sign, large (1e3: 1e8-scale sums) and small operands."""
    g = torch.Generator().manual_seed(Bn + K)
    a = (torch.randn((Bn, M, K), generator=g) * 0.1).bfloat16()
    b = (torch.randn((Bn, N, K), generator=g) * 0.1).bfloat16()
    for name, (aa, bb) in adversarial((a, b)):
        out = kore_amd.batched_gemm(aa.to(gpu), bb.to(gpu))
        verdict(out, batched_gemm_ref(aa, bb), "batched_gemm", "bf16", f"B{Bn} {M}x{N}x{K} adversarial {name}")


def test_batched_metamorphic_and_determinism(gpu):
    a, b = W.batched_inputs(12, 256, 384, 128, seed=7)
    a, b = a.to(gpu), b.to(gpu)
    full = kore_amd.batched_gemm(a, b)
    perm = torch.randperm(12, generator=torch.Generator().manual_seed(1)).to(gpu)
    permuted = kore_amd.batched_gemm(a[perm], b[perm])
    assert bit_equal(permuted, full[perm]), "batch permutation equivariance"
    assert bit_equal(kore_amd.batched_gemm(a, b), full), "determinism"


# Persistent short-K kernel (K of 64 or 128, >= 4 tiles of 128x128 per CU): ragged M/N,
# both B layouts, tile counts that are and are not multiples of 8 (the XCD schedule).
@pytest.mark.parametrize("Bn,M,N,K,bnc", [(40, 1000, 1016, 128, True), (20, 1000, 1024, 64, True),
                                          (33, 520, 1032, 64, False), (24, 1024, 1028, 128, False), (5, 4000, 1024, 128, False), (3, 3000, 2048, 64, True),
                                          (64, 1024, 1024, 128, False)])
def test_batched_short_k(gpu, Bn, M, N, K, bnc):
    g = torch.Generator().manual_seed(M + N + K)
    a = (torch.randn((Bn, M, K), generator=g) * 0.1).bfloat16()
    if bnc:
        b = (torch.randn((Bn, K, N), generator=g) * 0.1).bfloat16().transpose(1, 2)
    else:
        b = (torch.randn((Bn, N, K), generator=g) * 0.1).bfloat16()
    out = kore_amd.batched_gemm(a.to(gpu), b.to(gpu))
    ref = batched_gemm_ref(a, b)
    tag = f"short-K B{Bn} {M}x{N}x{K} {'NC' if bnc else 'KC'}"
    verdict(out, ref, "batched_gemm", "bf16", tag)
    pair_only(out, ref, "bf16", tag)
    assert bit_equal(kore_amd.batched_gemm(a.to(gpu), b.to(gpu)), out), "determinism"


def test_dense_short_k(gpu):
    """Dense A.W^T with K = 128 and enough tiles takes the persistent short-K kernel too
    (ragged M and N, 4-tile column segments)."""
    g = torch.Generator().manual_seed(5)
    a = (torch.randn((4000, 128), generator=g) * 0.1).bfloat16()
    w = (torch.randn((4104, 128), generator=g) * 0.1).bfloat16()
    out = kore_amd.gemm(a.to(gpu), w.to(gpu).t())
    from oracle.gemm import matmul_ref
    verdict(out, matmul_ref(a, w.t()), "gemm", "bf16", "short-K dense 4000x4104x128")
