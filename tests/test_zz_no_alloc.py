"""GPU: kore_gemm_noalloc, the GEMM entry point that allocates nothing, against kore_gemm.

Both entry points run the same kernels; the no-allocation one takes the scratch of its
packed-operand and split-K paths from a static device array instead of a workspace.
Each case calls it twice in a row through the C ABI, the second time on a smaller
problem (the array still holds the first call's contents), and both outputs must equal
kore_gemm's bit for bit; the first problem of each pair is also checked against the
CPU oracle at the reference tolerance.  A problem needing more scratch than the array
holds must fail with KORE_EWORKSPACE and leave the output untouched.
"""

from __future__ import annotations

import pytest
import torch

import kore_amd
from kore_amd import _lib
from kore_amd.ops import ACT_CODE, DT_CODE
from oracle.gemm import gemm_fusion_ref
from tests.fourprong import verdict

pytestmark = pytest.mark.gpu


def _noalloc(a, b, bias, act):
    lib = _lib.load()
    M, K = a.shape
    N = b.shape[1]
    c = torch.full((M, N), float("nan"), dtype=a.dtype, device=a.device)
    rc = lib.kore_gemm_noalloc(DT_CODE[a.dtype], ACT_CODE[act], a.data_ptr(), a.stride(0), a.stride(1),
                               b.data_ptr(), b.stride(0), b.stride(1),
                               bias.data_ptr() if bias is not None else None, c.data_ptr(), c.stride(0),
                               M, N, K, torch.cuda.current_stream(a.device).cuda_stream)
    return rc, c


def _inputs(M, N, K, dtype, layout, bias, seed, dev, a_t=False):
    g = torch.Generator().manual_seed(seed)
    sc = 1.0 / K ** 0.5
    a = (torch.randn((M, K), generator=g) * sc).to(dtype)
    if layout == "kn":  # the task's N-contiguous [K, N] B
        b = (torch.randn((K, N), generator=g) * sc).to(dtype)
        bd = b.to(dev)
    else:  # B = W.t(), K-contiguous
        w = (torch.randn((N, K), generator=g) * sc).to(dtype)
        b, bd = w.t(), w.to(dev).t()
    bs = torch.randn((N,), generator=g).to(dtype) if bias else None
    ad = a.t().contiguous().to(dev).t() if a_t else a.to(dev)  # a_t: A as an M-contiguous view
    return a, b, bs, ad, bd, (bs.to(dev) if bias else None)


# (first problem, second smaller problem), dtype, B layout, bias, act, path
CASES = [
    (((512, 1024, 4095), (200, 520, 2047)), torch.bfloat16, "kn", False, "none", "packed A"),
    (((384, 768, 999), (256, 640, 999)), torch.float16, "nk", True, "gelu", "packed A and B"),
    (((1, 2048, 4096), (1, 1024, 4096)), torch.bfloat16, "kn", False, "none", "split-K"),
    (((4, 4096, 4096), (2, 2048, 2048)), torch.float16, "nk", True, "silu", "split-K"),
    (((512, 1024, 4095), (300, 600, 1023)), torch.float32, "kn_at", True, "relu", "fp32 packed"),
    (((256, 256, 512), (128, 128, 256)), torch.bfloat16, "nk", False, "none", "no scratch"),
]


@pytest.mark.parametrize("shapes,dtype,layout,bias,act,path", CASES, ids=[c[-1] + f" {c[1]}" for c in CASES])
def test_noalloc_matches_kore_gemm(gpu, shapes, dtype, layout, bias, act, path):
    outs = []
    for i, (M, N, K) in enumerate(shapes):
        a, b, bs, ad, bd, bsd = _inputs(M, N, K, dtype, layout.removesuffix("_at"), bias, seed=M + N + K + i,
                                        dev=gpu, a_t=layout.endswith("_at"))
        rc, c = _noalloc(ad, bd, bsd, act)
        _lib.check(rc)
        outs.append((c, ad, bd, bsd, a, b, bs, (M, N, K)))
    torch.cuda.synchronize()
    for i, (c, ad, bd, bsd, a, b, bs, (M, N, K)) in enumerate(outs):
        ref = kore_amd.gemm_fused(ad, bd, bsd, act)
        torch.cuda.synchronize()
        assert torch.equal(c, ref), f"{path}: call {i} ({M}x{N}x{K}) differs from kore_gemm"
        if i == 0:
            name = "gemm_fusion_fp32" if dtype == torch.float32 else "gemm_fusion"
            dt = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[dtype]
            verdict(c.cpu(), gemm_fusion_ref(a, b, bs, act), name, dt, f"noalloc {path} {M}x{N}x{K}")


def test_noalloc_rejects_oversized_scratch(gpu):
    lib = _lib.load()
    cap = lib.kore_gemm_noalloc_scratch_bytes()
    assert cap == 64 << 20
    # 8200 x 1024 x 4095 with A an M-contiguous view and an unaligned K: A packs to
    # 8200 x 4096 bf16 (65.6 MB > 64 MiB)
    a = torch.zeros((4095, 8200), dtype=torch.bfloat16, device=gpu).t()
    b = torch.zeros((4095, 1024), dtype=torch.bfloat16, device=gpu)
    rc, c = _noalloc(a, b, None, "none")
    assert rc == 4, rc
    assert b"static scratch" in lib.kore_last_error()
    torch.cuda.synchronize()
    assert torch.isnan(c).all(), "nothing may be written when the scratch is too small"
