"""GPU parity: dense bf16/fp16 GEMM and the fused bias/activation epilogues.

Every case calls the gfx950 kernels through kore_amd (C ABI) and compares with the
CPU oracle (oracle/gemm.py) on identical seeded inputs, under the reference
drivers' verdict (allclose atol=rtol=1e-2, SNR >= 30 dB) and the four-prong pair
rule (bf16/fp16: worst |c-r|/(|r|+1e-2) <= 3e-2, SNR >= 30 dB, exact non-finite
structure).
"""

from __future__ import annotations

import pytest
import torch

import kore_amd
from kore_amd import workloads as W
from oracle.gemm import gemm_fusion_ref, matmul_ref
from tests.fourprong import adversarial, bit_equal, pair_only, verdict

pytestmark = pytest.mark.gpu


def _ref_style_inputs(M, N, K, seed, dtype=torch.bfloat16):
    """The reference task's own draw: a ~ N(0,1)/sqrt(K), b[K,N] ~ N(0,1) N-contiguous
    (kore/tasks/gemm_bf16/reference.py:28-36), drawn on the CPU here."""
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn((M, K), generator=g) / (K ** 0.5)).to(dtype)
    b = torch.randn((K, N), generator=g).to(dtype)
    return a, b


@pytest.mark.parametrize("seed", range(5))
def test_gemm_config_1024_bt(gpu, seed):
    """A, B [1024,1024] ~ N(0,1)*0.1, C = A.B^T (b = B.t())."""
    a, b = W.dense_inputs(1024, 1024, 1024, seed=seed)
    out = kore_amd.gemm(a.to(gpu), b.to(gpu))
    verdict(out, matmul_ref(a, b), "gemm", "bf16", f"1024^3 seed {seed}")


@pytest.mark.parametrize("M,N,K,dtype,op", [(1000, 1000, 1024, torch.bfloat16, "gemm"),
                                             (300, 520, 640, torch.float16, "gemm_bias_gelu"),
                                             (1, 4096, 4096, torch.bfloat16, "gemm"),
                                             (64, 4096, 4096, torch.float16, "gemm_bias_silu")])
def test_gemm_ring_small(gpu, M, N, K, dtype, op):
    """Few tiles and K >= 512 with b = W.t() run the 32x128 ring kernel: ragged M and N,
    a single row, and the fused epilogues on it."""
    g = torch.Generator().manual_seed(M + N)
    a = (torch.randn((M, K), generator=g) / K ** 0.5).to(dtype)
    w = (torch.randn((N, K), generator=g) / K ** 0.5).to(dtype)
    bias = (torch.randn((N,), generator=g) * 0.1).to(dtype)
    if op == "gemm":
        out = kore_amd.gemm_fused(a.to(gpu), w.to(gpu).t())
        ref = gemm_fusion_ref(a, w.t(), None, "none")
    else:
        out = getattr(kore_amd, op)(a.to(gpu), w.to(gpu).t(), bias.to(gpu))
        ref = gemm_fusion_ref(a, w.t(), bias, kore_amd.GEMM_FUSION_OPS[op][1])
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    verdict(out, ref, "gemm_fusion", dt, f"ring {op} {M}x{N}x{K}")
    pair_only(out, ref, dt, f"ring {op} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(64, 512, 512), (1, 4096, 4096), (4096, 4096, 4095),
                                   (513, 1000, 200), (4096, 4096, 4096)])
def test_gemm_reference_task_shapes(gpu, M, N, K):
    """gemm_bf16 task.yaml shapes (kore/tasks/gemm_bf16/task.yaml:8-14) with the task's
    natural N-contiguous B, plus a ragged shape; K = 4095 takes the in-place K-tail path
    (A rows read at 2-byte alignment, last stage from K - 64)."""
    a, b = _ref_style_inputs(M, N, K, seed=1)
    out = kore_amd.gemm(a.to(gpu), b.to(gpu))
    verdict(out, matmul_ref(a, b), "gemm", "bf16", f"{M}x{N}x{K}")


@pytest.mark.parametrize("K", [4095, 4033, 1000, 127, 65])
@pytest.mark.parametrize("layout", ["kn", "bt"])
def test_gemm_k_tail_in_place(gpu, K, layout):
    """K % 64 != 0 on the 256x256 grid (3072 x 4096: 192 tiles): the 16x16 engine reads A
    and B in place (rows at 2-byte alignment when K is odd) and starts its last 64-wide
    stage at K - 64; the 64 * ceil(K / 64) - K columns that stage shares with the one
    before (1 for K = 4095 and 127, 63 for 4033 and 65, 24 for 1000) are zeroed in LDS in
    both operands.  Column K - 64, inside that shared region, holds 4 in every row of A
    and every column of B (16 per output, against outputs of about unit size), so
    counting it twice, or missing it, fails the oracle check.  B: the task's [K,N] layout (kn) or W.t() of a [N,K] W (bt, rows of K
    elements)."""
    M, N = 3072, 4096
    g = torch.Generator().manual_seed(K)
    a = (torch.randn((M, K), generator=g) / K ** 0.5).to(torch.bfloat16)
    w = torch.randn((N, K), generator=g).to(torch.bfloat16)
    a[:, K - 64] = 4.0
    w[:, K - 64] = 4.0
    b = w.t().contiguous() if layout == "kn" else w.t()
    bd = w.t().contiguous().to(gpu) if layout == "kn" else w.to(gpu).t()
    out = kore_amd.gemm(a.to(gpu), bd)
    ref = matmul_ref(a, b)
    verdict(out, ref, "gemm", "bf16", f"K tail {K} {layout}")
    pair_only(out, ref, "bf16", f"K tail {K} {layout}")
    out2 = kore_amd.gemm(a.to(gpu), bd)
    assert bit_equal(out, out2), "determinism"


@pytest.mark.parametrize("M,N,K,dtype,op", [(512, 4096, 4095, torch.float16, "gemm_bias_gelu"),
                                             (512, 4096, 1000, torch.bfloat16, "gemm"),
                                             (512, 4096, 257, torch.bfloat16, "gemm_relu"),
                                             (2048, 2048, 2047, torch.float16, "gemm"),
                                             (1536, 4096, 1001, torch.bfloat16, "gemm_bias_silu")])
@pytest.mark.parametrize("layout", ["kn", "bt"])
def test_gemm_k_tail_deep_ring(gpu, M, N, K, dtype, op, layout):
    """K % 64 != 0 on mid-size grids runs the deep ring engine's K-tail mode at the tile
    pick_tile chooses (64x128 for 512 x 4096, 128x128 for 2048^2, 256x128 for 1536 x
    4096): both operands read in place, the last stage from K - 64, the repeated columns
    zeroed in LDS.  Column K - 64 holds 4 in every row of A and column of B (16 per
    output), so counting it twice or missing it fails the oracle check; fused epilogues
    on the same path."""
    g = torch.Generator().manual_seed(M + K)
    a = (torch.randn((M, K), generator=g) / K ** 0.5).to(dtype)
    w = torch.randn((N, K), generator=g).to(dtype)
    a[:, K - 64] = 4.0
    w[:, K - 64] = 4.0
    bias = torch.randn((N,), generator=g).to(dtype)
    b = w.t().contiguous() if layout == "kn" else w.t()
    bd = w.t().contiguous().to(gpu) if layout == "kn" else w.to(gpu).t()
    has_bias, act = kore_amd.GEMM_FUSION_OPS.get(op, (False, "none"))
    out = kore_amd.gemm_fused(a.to(gpu), bd, bias.to(gpu) if has_bias else None, act)
    ref = gemm_fusion_ref(a, b, bias if has_bias else None, act)
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    verdict(out, ref, "gemm_fusion", dt, f"deep K tail {op} {M}x{N}x{K} {layout}")
    pair_only(out, ref, dt, f"deep K tail {op} {M}x{N}x{K} {layout}")


@pytest.mark.parametrize("M,N,K,dtype,op", [(4096, 4096, 4096, torch.bfloat16, "gemm_bias_gelu"),
                                             (3000, 4104, 1024, torch.float16, "gemm_bias_silu"),
                                             (2048, 7168, 4096, torch.bfloat16, "gemm"),
                                             (3840, 3336, 1024, torch.float16, "gemm_relu")])
@pytest.mark.parametrize("strided", [False, True])
def test_gemm_nc_buffer_engine(gpu, M, N, K, dtype, op, strided):
    """N-contiguous B (the tasks' natural [K,N] layout) at >= 192 tiles of 256x256 runs the
    buffer-load engine with LDS transpose reads: ragged M and N (N % 256 != 0), fused
    epilogues, and a B view whose K-rows are wider than N (row stride N + 128)."""
    has_bias, act = kore_amd.GEMM_FUSION_OPS.get(op, (False, "none"))
    g = torch.Generator().manual_seed(M + N + K)
    sc = 1.0 / K ** 0.5
    a = (torch.randn((M, K), generator=g) * sc).to(dtype)
    bfull = (torch.randn((K, N + 128), generator=g) * sc).to(dtype)
    b = bfull[:, 64:64 + N] if strided else bfull[:, :N].contiguous()
    bias = torch.randn((N,), generator=g).to(dtype) if has_bias else None
    bd = bfull.to(gpu)[:, 64:64 + N] if strided else b.to(gpu)
    assert bd.stride(1) == 1 and bd.stride(0) == (N + 128 if strided else N)
    out = kore_amd.gemm_fused(a.to(gpu), bd, bias.to(gpu) if has_bias else None, act)
    ref = gemm_fusion_ref(a, b, bias, act)
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    verdict(out, ref, "gemm_fusion", dt, f"nc {op} {M}x{N}x{K} strided={strided}")
    pair_only(out, ref, dt, f"nc {op} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,dtype,op", [(4000, 3900, 4096, torch.bfloat16, "gemm_bias_gelu"),
                                             (3000, 4104, 1024, torch.float16, "gemm_bias_silu"),
                                             (2048, 7168, 4096, torch.bfloat16, "gemm"),
                                             (3841, 3336, 512, torch.float16, "gemm_relu")])
@pytest.mark.parametrize("strided", [False, True])
def test_gemm_kc_buffer_engine(gpu, M, N, K, dtype, op, strided):
    """K-contiguous B (a W[N,K].t() view) at >= 192 tiles of 256x256 runs the 4-wave tile with
    its accumulators in AGPRs: ragged M and N, fused epilogues, and W rows wider than K (row
    stride K + 64) read in place."""
    has_bias, act = kore_amd.GEMM_FUSION_OPS.get(op, (False, "none"))
    g = torch.Generator().manual_seed(M + N + K + 1)
    sc = 1.0 / K ** 0.5
    a = (torch.randn((M, K), generator=g) * sc).to(dtype)
    wfull = (torch.randn((N, K + 64), generator=g) * sc).to(dtype)
    w = wfull[:, 32:32 + K] if strided else wfull[:, :K].contiguous()
    bias = torch.randn((N,), generator=g).to(dtype) if has_bias else None
    wd = wfull.to(gpu)[:, 32:32 + K] if strided else w.to(gpu)
    assert wd.stride(1) == 1 and wd.stride(0) == (K + 64 if strided else K)
    out = kore_amd.gemm_fused(a.to(gpu), wd.t(), bias.to(gpu) if has_bias else None, act)
    ref = gemm_fusion_ref(a, w.t(), bias, act)
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    verdict(out, ref, "gemm_fusion", dt, f"kc {op} {M}x{N}x{K} strided={strided}")
    pair_only(out, ref, dt, f"kc {op} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,dtype,op", [(2048, 2048, 2048, torch.bfloat16, "gemm"),
                                             (1024, 4096, 4096, torch.float16, "gemm_bias_gelu"),
                                             (256, 14336, 4096, torch.bfloat16, "gemm_bias_silu"),
                                             (512, 4096, 4096, torch.bfloat16, "gemm_bias_gelu"),
                                             (1024, 2048, 2048, torch.float16, "gemm_sigmoid"),
                                             (500, 4000, 1024, torch.bfloat16, "gemm_bias"),
                                             (1000, 1000, 1024, torch.bfloat16, "gemm_tanh"),
                                             (1, 4096, 4096, torch.bfloat16, "gemm"),
                                             (1536, 4096, 4096, torch.bfloat16, "gemm"),
                                             (1500, 4000, 1024, torch.float16, "gemm_bias_gelu"),
                                             (768, 4096, 4096, torch.bfloat16, "gemm_bias_relu")])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_gemm_deep_ring(gpu, M, N, K, dtype, op, layout):
    """Mid-size and small problems with a long K on the deep-ring kernel (256x128,
    128x128, 64x128 or 32x128 tiles by weighted rounds over the CUs), both B layouts
    ([K,N] and the W.t() view), ragged M and N, fused epilogues."""
    has_bias, act = kore_amd.GEMM_FUSION_OPS.get(op, (False, "none"))
    g = torch.Generator().manual_seed(M * 7 + N + K)
    sc = 1.0 / K ** 0.5
    a = (torch.randn((M, K), generator=g) * sc).to(dtype)
    if layout == "kn":
        b = (torch.randn((K, N), generator=g) * sc).to(dtype)
        bd = b.to(gpu)
    else:
        w = (torch.randn((N, K), generator=g) * sc).to(dtype)
        b, bd = w.t(), w.to(gpu).t()
    bias = torch.randn((N,), generator=g).to(dtype) if has_bias else None
    out = kore_amd.gemm_fused(a.to(gpu), bd, bias.to(gpu) if has_bias else None, act)
    ref = gemm_fusion_ref(a, b, bias, act)
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    verdict(out, ref, "gemm_fusion", dt, f"deep {op} {M}x{N}x{K} {layout}")
    pair_only(out, ref, dt, f"deep {op} {M}x{N}x{K} {layout}")


def test_batched_deep_ring(gpu):
    """A batched problem with >= 224 tiles of 128x128 and K = 512 runs the deep ring per
    batch (batch strides on A, B and C)."""
    from oracle.gemm import batched_gemm_ref

    g = torch.Generator().manual_seed(5)
    a = (torch.randn((16, 512, 512), generator=g) / 512 ** 0.5).bfloat16()
    b = (torch.randn((16, 512, 512), generator=g) / 512 ** 0.5).bfloat16()
    out = kore_amd.batched_gemm(a.to(gpu), b.to(gpu))
    verdict(out, batched_gemm_ref(a, b), "gemm", "bf16", "batched deep 16x512x512x512")


@pytest.mark.parametrize("M,N,K,dtype,op,layout", [(512, 4096, 4095, torch.float16, "gemm_bias_gelu", "kn"),
                                                    (512, 4096, 4095, torch.bfloat16, "gemm_bias_silu", "nk"),
                                                    (1024, 2048, 2047, torch.bfloat16, "gemm_relu", "kn_at"),
                                                    (300, 1000, 777, torch.float16, "gemm_bias", "nk_at"),
                                                    (2048, 2048, 1000, torch.bfloat16, "gemm", "strided")])
def test_gemm_packed_path(gpu, M, N, K, dtype, op, layout):
    """Operands the engines cannot read in place -- K tails that leave rows unaligned (the
    gen_gemm_* K = 4095 validation shape), a transposed A, a B with a row stride that is
    not a multiple of 8 -- are packed into the caller's workspace first."""
    has_bias, act = kore_amd.GEMM_FUSION_OPS.get(op, (False, "none"))
    g = torch.Generator().manual_seed(M + 3 * N + K)
    sc = 1.0 / K ** 0.5
    a = (torch.randn((M, K), generator=g) * sc).to(dtype)
    ad = a.t().contiguous().to(gpu).t() if layout.endswith("_at") else a.to(gpu)
    if layout.startswith("kn"):
        b = (torch.randn((K, N), generator=g) * sc).to(dtype)
        bd = b.to(gpu)
    elif layout == "strided":
        full = (torch.randn((K, N + 3), generator=g) * sc).to(dtype)
        b, bd = full[:, :N], full.to(gpu)[:, :N]
    else:
        w = (torch.randn((N, K), generator=g) * sc).to(dtype)
        b, bd = w.t(), w.to(gpu).t()
    bias = torch.randn((N,), generator=g).to(dtype) if has_bias else None
    out = kore_amd.gemm_fused(ad, bd, bias.to(gpu) if has_bias else None, act)
    ref = gemm_fusion_ref(a, b, bias, act)
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    verdict(out, ref, "gemm_fusion", dt, f"packed {op} {M}x{N}x{K} {layout}")
    pair_only(out, ref, dt, f"packed {op} {M}x{N}x{K} {layout}")
    # a second call (with its own workspace): same result bit for bit
    again = kore_amd.gemm_fused(ad, bd, bias.to(gpu) if has_bias else None, act)
    assert torch.equal(out, again)


@pytest.mark.parametrize("M,N,K,dtype,op,layout", [(4096, 4096, 4096, torch.bfloat16, "gemm", "kn"),
                                                    (4096, 4096, 4096, torch.float16, "gemm_bias_gelu", "nk"),
                                                    (3000, 4104, 1024, torch.bfloat16, "gemm_bias_silu", "kn"),
                                                    (2048, 7168, 2048, torch.float16, "gemm_relu", "nk")])
def test_gemm_transposed_a_in_place(gpu, M, N, K, dtype, op, layout):
    """A transposed A (the a.t() view of a [K, M] tensor, M-contiguous) on a grid of at
    least 192 tiles of 256x256 is read in place by the buffer engine through LDS transpose
    reads (no workspace): ragged M and N, both B layouts, fused epilogues."""
    has_bias, act = kore_amd.GEMM_FUSION_OPS.get(op, (False, "none"))
    g = torch.Generator().manual_seed(M + 5 * N + K)
    sc = 1.0 / K ** 0.5
    a = (torch.randn((M, K), generator=g) * sc).to(dtype)
    ad = a.t().contiguous().to(gpu).t()
    assert ad.stride() == (1, M)
    if layout == "kn":
        b = (torch.randn((K, N), generator=g) * sc).to(dtype)
        bd = b.to(gpu)
    else:
        w = (torch.randn((N, K), generator=g) * sc).to(dtype)
        b, bd = w.t(), w.to(gpu).t()
    bias = torch.randn((N,), generator=g).to(dtype) if has_bias else None
    from kore_amd import _lib
    lib = _lib.load()
    assert lib.kore_gemm_workspace_bytes(0 if dtype == torch.bfloat16 else 1, 0, ad.data_ptr(), 1, M, bd.data_ptr(),
                                         bd.stride(0), bd.stride(1), None, ad.data_ptr(), N, M, N, K) == 0
    out = kore_amd.gemm_fused(ad, bd, bias.to(gpu) if has_bias else None, act)
    ref = gemm_fusion_ref(a, b, bias, act)
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    verdict(out, ref, "gemm_fusion", dt, f"transposed A {op} {M}x{N}x{K} {layout}")
    pair_only(out, ref, dt, f"transposed A {op} {M}x{N}x{K} {layout}")
    assert torch.equal(out, kore_amd.gemm_fused(ad, bd, bias.to(gpu) if has_bias else None, act))


@pytest.mark.parametrize("M,N,K,dtype,op,layout", [(1, 4096, 4096, torch.bfloat16, "gemm", "kn"),
                                                    (16, 11008, 4096, torch.float16, "gemm_bias_gelu", "kn"),
                                                    (7, 1002, 2048, torch.bfloat16, "gemm_bias_relu", "nk"),
                                                    (33, 3000, 1024, torch.float16, "gemm_sigmoid", "nk"),
                                                    (64, 4096, 4096, torch.bfloat16, "gemm_bias_silu", "kn"),
                                                    (1, 5120, 4096, torch.bfloat16, "gemm_bias", "nk")])
def test_gemm_splitk(gpu, M, N, K, dtype, op, layout):
    """Decode-sized M with a long K splits K over the CUs (32x128 ring per slice, fp32
    partials, fixed-order reduce with the epilogue): ragged N (not a multiple of 4 on the
    W.t() layout: the 8-column scalar reduce), 2, 4, 6 and 8 slices (the 4-column reduce's
    unrolled and remainder loops), and bit-identical repeated calls."""
    has_bias, act = kore_amd.GEMM_FUSION_OPS.get(op, (False, "none"))
    g = torch.Generator().manual_seed(M + N + K + 1)
    sc = 1.0 / K ** 0.5
    a = (torch.randn((M, K), generator=g) * sc).to(dtype)
    if layout == "kn":
        b = (torch.randn((K, N), generator=g) * sc).to(dtype)
        bd = b.to(gpu)
    else:
        w = (torch.randn((N, K), generator=g) * sc).to(dtype)
        b, bd = w.t(), w.to(gpu).t()
    bias = torch.randn((N,), generator=g).to(dtype) if has_bias else None
    args = (a.to(gpu), bd, bias.to(gpu) if has_bias else None, act)
    out = kore_amd.gemm_fused(*args)
    ref = gemm_fusion_ref(a, b, bias, act)
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    verdict(out, ref, "gemm_fusion", dt, f"splitk {op} {M}x{N}x{K} {layout}")
    pair_only(out, ref, dt, f"splitk {op} {M}x{N}x{K} {layout}")
    assert torch.equal(out, kore_amd.gemm_fused(*args))


@pytest.mark.parametrize("M,N,K,dtype,op,a_t,b_layout", [(512, 512, 511, torch.bfloat16, "gemm_bias_gelu", False, "kn"),
                                                           (200, 300, 1001, torch.float16, "gemm_relu", True, "nk"),
                                                           (130, 129, 77, torch.bfloat16, "gemm", True, "odd"),
                                                           (1, 257, 33, torch.float16, "gemm_bias_silu", False, "odd")])
def test_gemm_generic_mfma(gpu, M, N, K, dtype, op, a_t, b_layout):
    """Problems too small for a pack pass in layouts the engines cannot read (odd K,
    transposed A, B rows with an odd stride) run the generic MFMA kernel: element reads
    along the unit-stride index, every read bounds-checked, ragged tiles on every edge."""
    has_bias, act = kore_amd.GEMM_FUSION_OPS.get(op, (False, "none"))
    g = torch.Generator().manual_seed(M + N + K + 7)
    sc = 1.0 / K ** 0.5
    a = (torch.randn((M, K), generator=g) * sc).to(dtype)
    ad = a.t().contiguous().to(gpu).t() if a_t else a.to(gpu)
    if b_layout == "kn":
        b = (torch.randn((K, N), generator=g) * sc).to(dtype)
        bd = b.to(gpu)
    elif b_layout == "nk":
        w = (torch.randn((N, K), generator=g) * sc).to(dtype)
        b, bd = w.t(), w.to(gpu).t()
    else:
        full = (torch.randn((K, N + 5), generator=g) * sc).to(dtype)
        b, bd = full[:, 2:2 + N], full.to(gpu)[:, 2:2 + N]
    bias = torch.randn((N,), generator=g).to(dtype) if has_bias else None
    out = kore_amd.gemm_fused(ad, bd, bias.to(gpu) if has_bias else None, act)
    ref = gemm_fusion_ref(a, b, bias, act)
    dt = "bf16" if dtype == torch.bfloat16 else "fp16"
    verdict(out, ref, "gemm_fusion", dt, f"generic {op} {M}x{N}x{K} a_t={a_t} {b_layout}")
    pair_only(out, ref, dt, f"generic {op} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,op,a_t,b_layout", [(300, 200, 77, "gemm_bias_gelu", True, "kn"),
                                                    (257, 130, 1001, "gemm_sigmoid", False, "odd"),
                                                    (1, 300, 64, "gemm_bias", False, "nk"),
                                                    (129, 257, 130, "gemm_relu", True, "odd")])
def test_gemm_fp32_generic_mfma(gpu, M, N, K, op, a_t, b_layout):
    """fp32 problems the ring kernel cannot read and too small for a pack pass run the
    generic fp32 MFMA kernel (element reads along the unit-stride index, bounds-checked,
    ragged tiles on every edge) at the fp32 gate."""
    has_bias, act = kore_amd.GEMM_FUSION_OPS.get(op, (False, "none"))
    g = torch.Generator().manual_seed(M * 3 + N + K)
    sc = 1.0 / K ** 0.5
    a = torch.randn((M, K), generator=g) * sc
    ad = a.t().contiguous().to(gpu).t() if a_t else a.to(gpu)
    if b_layout == "kn":
        b = torch.randn((K, N), generator=g) * sc
        bd = b.to(gpu)
    elif b_layout == "nk":
        w = torch.randn((N, K), generator=g) * sc
        b, bd = w.t(), w.to(gpu).t()
    else:
        full = torch.randn((K, N + 3), generator=g) * sc
        b, bd = full[:, 1:1 + N], full.to(gpu)[:, 1:1 + N]
    bias = torch.randn((N,), generator=g) if has_bias else None
    out = kore_amd.gemm_fused(ad, bd, bias.to(gpu) if has_bias else None, act)
    ref = gemm_fusion_ref(a, b, bias, act)
    verdict(out, ref, "gemm_fusion_fp32", "fp32", f"fp32 generic {op} {M}x{N}x{K} a_t={a_t} {b_layout}")


@pytest.mark.parametrize("K", [4095, 1000, 96, 33])
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_gemm_fp32_k_tail_in_place(gpu, K, layout):
    """fp32 K % 64 != 0 at 512 x 4096 (the gen_gemm_*_fp32 shape class): the ring kernel
    reads A and B in place (rows at 4-byte alignment when K % 4 != 0) and starts its last
    32-float stage at K - 32; the 32 * ceil(K / 32) - K columns it shares with the stage
    before (1, 8, 0 and 31 here) are zeroed in LDS in both operands.  Column K - 32 holds 4
    in every row of A and column of B, so a twice-counted or missing product (16 per
    output) fails the fp32 gate."""
    M, N = 512, 4096
    g = torch.Generator().manual_seed(K + 7)
    a = torch.randn((M, K), generator=g) / K ** 0.5
    w = torch.randn((N, K), generator=g)
    a[:, K - 32] = 4.0
    w[:, K - 32] = 4.0
    bias = torch.randn((N,), generator=g)
    if layout == "kn":
        b = w.t().contiguous()
        bd = b.to(gpu)
    else:
        b, bd = w.t(), w.to(gpu).t()
    out = kore_amd.gemm_fused(a.to(gpu), bd, bias.to(gpu), "none")
    ref = gemm_fusion_ref(a, b, bias, "none")
    verdict(out, ref, "gemm_fusion_fp32", "fp32", f"fp32 K tail {K} {layout}")
    pair_only(out, ref, "fp32", f"fp32 K tail {K} {layout}")


def test_batched_packed_path(gpu):
    """A batched problem with an odd K runs the packed path per batch."""
    from oracle.gemm import batched_gemm_ref

    g = torch.Generator().manual_seed(9)
    a = (torch.randn((4, 512, 999), generator=g) / 999 ** 0.5).bfloat16()
    b = (torch.randn((4, 384, 999), generator=g) / 999 ** 0.5).bfloat16()
    out = kore_amd.batched_gemm(a.to(gpu), b.to(gpu))
    verdict(out, batched_gemm_ref(a, b), "gemm", "bf16", "batched packed 4x512x384x999")


@pytest.mark.parametrize("B,M,N,K", [(4, 1024, 1024, 1023), (4, 2048, 2048, 2047)])
def test_batched_k_tail_in_place(gpu, B, M, N, K):
    """Batched problems with K % 64 != 0 on the K-tail modes, per-batch operand offsets
    included: 4 x 1024^2 (256 tiles of 128x128: deep ring) and 4 x 2048^2 (256 tiles of
    256x256: the 16x16 engine); column K - 64 of every batch holds 4 in A and B, so a
    twice-counted or missing shared column fails the check."""
    from oracle.gemm import batched_gemm_ref

    g = torch.Generator().manual_seed(B + K)
    a = (torch.randn((B, M, K), generator=g) / K ** 0.5).bfloat16()
    b = torch.randn((B, N, K), generator=g).bfloat16()
    a[:, :, K - 64] = 4.0
    b[:, :, K - 64] = 4.0
    out = kore_amd.batched_gemm(a.to(gpu), b.to(gpu))
    ref = batched_gemm_ref(a, b)
    verdict(out, ref, "gemm", "bf16", f"batched K tail {B}x{M}x{N}x{K}")
    pair_only(out, ref, "bf16", f"batched K tail {B}x{M}x{N}x{K}")


def test_gemm_metric_4096_bt(gpu):
    a, b = W.dense_inputs(4096, 4096, 4096, seed=0)
    out = kore_amd.gemm(a.to(gpu), b.to(gpu))
    verdict(out, matmul_ref(a, b), "gemm", "bf16", "4096^3 A.B^T")


@pytest.mark.parametrize("act", ["gelu", "relu", "silu"])
def test_fused_fp16_config_4096(gpu, act):
    """fp16 A, W [4096,4096] ~ N(0,1)/64, bias ~ N(0,1)*0.1,
    out = act(A.W^T + bias)."""
    a, b, bias = W.fused_inputs(4096, 4096, 4096, seed=0)
    out = kore_amd.gemm_fused(a.to(gpu), b.to(gpu), bias.to(gpu), act)
    verdict(out, gemm_fusion_ref(a, b, bias, act), "gemm_fusion", "fp16", f"fp16 4096^3 bias+{act}")


@pytest.mark.parametrize("op", sorted(kore_amd.GEMM_FUSION_OPS))
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_fusion_ops(gpu, op, dtype):
    """Every gemm_fusion op (kore/tasks/_genops.py:274-290), 3 seeds, on the task's minimal
    shape and a ragged shape, with the task's own distribution (A, B ~ N(0,1)/sqrt(K),
    B N-contiguous, bias ~ N(0,1); kore/tasks/_genops.py:430-443)."""
    has_bias, act = kore_amd.GEMM_FUSION_OPS[op]
    fn = getattr(kore_amd, op)
    for (M, N, K) in [(64, 256, 256), (300, 520, 200)]:
        for seed in range(3):
            g = torch.Generator().manual_seed(seed)
            sc = 1.0 / K ** 0.5
            a = (torch.randn((M, K), generator=g) * sc).to(dtype)
            b = (torch.randn((K, N), generator=g) * sc).to(dtype)
            bias = torch.randn((N,), generator=g).to(dtype) if has_bias else None
            args = (a, b, bias) if has_bias else (a, b)
            out = fn(*[t.to(gpu) for t in args])
            ref = gemm_fusion_ref(a, b, bias, act)
            verdict(out, ref, "gemm_fusion", str(dtype), f"{op} {M}x{N}x{K} seed {seed}")
            pair_only(out, ref, str(dtype), f"{op} {M}x{N}x{K}")


@pytest.mark.parametrize("op", ["gemm_bias_gelu", "gemm_bias_relu", "gemm_bias_silu", "gemm_bias",
                                "gemm_tanh", "gemm_sigmoid"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gemm_fusion_adversarial(gpu, op, dtype):
    """Generic adversarial fills (kore/tasks/_genops.py:855-879): with K=512 the 'large'
    fill gives 5e8 accumulators, i.e. +-inf after the fp16 cast in both paths."""
    has_bias, act = kore_amd.GEMM_FUSION_OPS[op]
    M, N, K = 128, 256, 512
    g = torch.Generator().manual_seed(0)
    a = torch.randn((M, K), generator=g).to(dtype)
    b = torch.randn((K, N), generator=g).to(dtype)
    bias = torch.randn((N,), generator=g).to(dtype)
    base = (a, b, bias) if has_bias else (a, b)
    for name, adv in adversarial(base):
        out = kore_amd.gemm_fused(adv[0].to(gpu), adv[1].to(gpu), adv[2].to(gpu) if has_bias else None, act)
        ref = gemm_fusion_ref(adv[0], adv[1], adv[2] if has_bias else None, act)
        verdict(out, ref, "gemm_fusion", str(dtype), f"{op} adversarial {name}")


def test_gemm_metamorphic(gpu):
    """Row split, column permutation and power-of-two scaling identities."""
    a, b = W.dense_inputs(768, 640, 512, seed=3)
    a, b = a.to(gpu), b.to(gpu)
    full = kore_amd.gemm(a, b)
    top, bot = kore_amd.gemm(a[:300], b), kore_amd.gemm(a[300:], b)
    pair_only(torch.cat([top, bot]).cpu(), full.cpu(), "bf16", "row split", "metamorphic")
    perm = torch.randperm(640, generator=torch.Generator().manual_seed(0)).to(gpu)
    pcols = kore_amd.gemm(a, b[:, perm].contiguous())
    pair_only(pcols.cpu(), full[:, perm].cpu(), "bf16", "column permutation", "metamorphic")
    # x2 on A is exact in bf16 and commutes with RNE rounding: bit-identical result.
    assert bit_equal(kore_amd.gemm(a * 2, b), full * 2)


def test_gemm_determinism(gpu):
    a, b = W.dense_inputs(2048, 2048, 2048, seed=4)
    a, b = a.to(gpu), b.to(gpu)
    r1 = kore_amd.gemm(a, b)
    r2 = kore_amd.gemm(a, b)
    assert bit_equal(r1, r2)
    a16, b16, bias = W.fused_inputs(1024, 1024, 1024, seed=4)
    x1 = kore_amd.gemm_fused(a16.to(gpu), b16.to(gpu), bias.to(gpu), "gelu")
    x2 = kore_amd.gemm_fused(a16.to(gpu), b16.to(gpu), bias.to(gpu), "gelu")
    assert bit_equal(x1, x2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("K,start", [(4089, 1), (4095, 0), (4093, 3), (1031, 1)])
def test_gemm_repitch_k_tails(gpu, dtype, K, start):
    """Packed path through the row re-stride kernels: A as a view of a wider tensor
    starting `start` elements in (row 0 at a 2 mod 4 byte address for odd starts in 16-bit
    types), row stride K + 9, K % 8 in {1, 3, 7}; B given as W.t() with W [N, K] in the
    same layout, so B^T is re-strided too (fp32: B read in place when N-contiguous, here
    packed).  Zero K tails padded to the kernels' K step."""
    M, N = 512, 1024
    g = torch.Generator().manual_seed(K + start)
    afull = (torch.randn((M, K + 9), generator=g) / 16).to(dtype)
    wfull = (torch.randn((N, K + 9), generator=g) / 16).to(dtype)
    a, w = afull[:, start:start + K], wfull[:, start:start + K]
    ad, wd = afull.to(gpu)[:, start:start + K], wfull.to(gpu)[:, start:start + K]
    assert ad.stride() == (K + 9, 1) and wd.stride() == (K + 9, 1)
    out = kore_amd.gemm_fused(ad, wd.t(), None, "none")
    ref = gemm_fusion_ref(a, w.t(), None, "none")
    verdict(out, ref, "gemm_fusion", str(dtype), f"re-stride {M}x{N}x{K} start {start}")
    assert bit_equal(kore_amd.gemm_fused(ad, wd.t(), None, "none"), out), "determinism"


def test_batched_repitch_k_tail(gpu):
    """Batched packed path with a K tail (K = 1001): per-batch re-stride of A and B^T."""
    Bn, M, N, K = 4, 512, 512, 1001
    g = torch.Generator().manual_seed(1)
    a = (torch.randn((Bn, M, K), generator=g) * 0.1).bfloat16()
    b = (torch.randn((Bn, N, K), generator=g) * 0.1).bfloat16()
    out = kore_amd.batched_gemm(a.to(gpu), b.to(gpu))
    from oracle.gemm import batched_gemm_ref
    verdict(out, batched_gemm_ref(a, b), "batched_gemm", "bf16", f"re-stride B{Bn} {M}x{N}x{K}")


def test_gemm_strided_and_degenerate(gpu):
    """Non-unit strides on both operands (generic kernel), K=0 and empty outputs."""
    g = torch.Generator().manual_seed(5)
    big = torch.randn((200, 300), generator=g).to(torch.bfloat16)
    a = big[::2, ::3]          # [100, 100], strides (600, 3)
    b = big.t()[::3, ::2]      # [100, 100]
    out = kore_amd.gemm(a.to(gpu), b.to(gpu))
    verdict(out, matmul_ref(a, b), "gemm", "bf16", "strided")
    z = kore_amd.gemm_fused(torch.empty((7, 0), dtype=torch.float16, device=gpu),
                            torch.empty((0, 9), dtype=torch.float16, device=gpu),
                            torch.ones(9, dtype=torch.float16, device=gpu), "relu")
    assert torch.equal(z.cpu(), torch.ones((7, 9), dtype=torch.float16))
    assert kore_amd.gemm(torch.empty((0, 8), dtype=torch.bfloat16, device=gpu),
                         torch.empty((8, 5), dtype=torch.bfloat16, device=gpu)).shape == (0, 5)


def test_gemm_errors(gpu):
    a = torch.zeros((4, 8), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        kore_amd.gemm(a, torch.zeros((7, 4), dtype=torch.bfloat16, device=gpu))
    with pytest.raises(ValueError):
        kore_amd.gemm(a, torch.zeros((8, 4), dtype=torch.float16, device=gpu))
    with pytest.raises(ValueError):
        kore_amd.gemm(a.cpu(), torch.zeros((8, 4), dtype=torch.bfloat16))


# gen_gemm_<op>_fp32 tasks (kore/tasks/gen_gemm_bias_fp32/task.yaml: minimal 64x256x256,
# primary 512x4096x4096, validation 1024x2048x2048, 256x14336x4096, 512x4096x4095)
@pytest.mark.parametrize("op", sorted(kore_amd.GEMM_FUSION_OPS))
def test_gemm_fusion_fp32_ops(gpu, op):
    """fp32 operands on the fp32 MFMA: every op on the minimal shape and a ragged one
    (N-contiguous b, the task's draw), at the fp32 gate (40 dB, allclose 1e-2) and the
    strict fp32 pair rule."""
    has_bias, act = kore_amd.GEMM_FUSION_OPS[op]
    fn = getattr(kore_amd, op)
    for (M, N, K) in [(64, 256, 256), (300, 520, 224), (77, 132, 100)]:
        g = torch.Generator().manual_seed(M)
        sc = 1.0 / K ** 0.5
        a = torch.randn((M, K), generator=g) * sc
        b = torch.randn((K, N), generator=g) * sc
        bias = torch.randn((N,), generator=g) if has_bias else None
        args = (a, b, bias) if has_bias else (a, b)
        out = fn(*[t.to(gpu) for t in args])
        assert out.dtype == torch.float32
        ref = gemm_fusion_ref(a, b, bias, act)
        verdict(out, ref, "gemm_fusion_fp32", "fp32", f"{op} fp32 {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(512, 4096, 4096), (1024, 2048, 2048), (256, 14336, 4096), (512, 4096, 4095)])
@pytest.mark.parametrize("bt", [False, True])
def test_gemm_fp32_task_shapes(gpu, M, N, K, bt):
    """The fp32 task shapes, with b N-contiguous (the task's layout) or a W.t() view;
    K = 4095 runs the ring kernel's in-place K-tail mode.  Rows are sampled for the
    oracle."""
    g = torch.Generator(device=gpu).manual_seed(K)
    sc = 1.0 / K ** 0.5
    a = torch.randn((M, K), generator=g, device=gpu) * sc
    b = (torch.randn((N, K), generator=g, device=gpu) * sc).t() if bt else torch.randn((K, N), generator=g, device=gpu) * sc
    bias = torch.randn((N,), generator=g, device=gpu)
    out = kore_amd.gemm_bias_gelu(a, b, bias)
    rows = torch.unique(torch.cat([torch.arange(0, M, max(1, M // 64)), torch.tensor([M - 1])])).to(gpu)
    ref = gemm_fusion_ref(a[rows].cpu(), b.cpu(), bias.cpu(), "gelu")
    verdict(out[rows].cpu(), ref, "gemm_fusion_fp32", "fp32", f"fp32 {M}x{N}x{K} bt={bt}")
    pair_only(out[rows].cpu(), ref, "fp32", f"fp32 {M}x{N}x{K}")


# gemm_backward_bf16 (kore/tasks/gemm_backward_bf16/task.yaml: minimal 256^3, primary
# 8192x4096x4096, validation 32768x4096x4096, 4096x14336x4096, 8192x4096x8192,
# 4096x4095x4096) plus a ragged small shape
@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (8192, 4096, 4096), (4096, 4095, 4096), (4096, 14336, 4096),
                                   (300, 200, 136)])
def test_gemm_backward_task_shapes(gpu, M, N, K):
    """dX = dY.W and dW = dY^T.X against the fp32 oracle at the task tolerances (dx
    atol 5e-2, dw atol 2e-1, rtol 2e-2, SNR >= 25 dB); the multi-GB shapes are checked
    on sampled rows of dX and columns of dW, plus determinism."""
    from oracle.gemm import gemm_backward_ref

    x, w, dy = W.backward_inputs(M, N, K, seed=M + N)
    xg, wg, dyg = x.to(gpu), w.to(gpu), dy.to(gpu)
    dx, dw = kore_amd.gemm_backward(xg, wg, dyg)
    assert dx.shape == (M, K) and dw.shape == (N, K) and dx.dtype == dw.dtype == torch.bfloat16
    step_m, step_k = max(1, M // 48), max(1, K // 48)
    rows = torch.unique(torch.cat([torch.arange(0, M, step_m), torch.tensor([M - 1])]))
    cols = torch.unique(torch.cat([torch.arange(0, K, step_k), torch.tensor([K - 1])]))
    rdx, _ = gemm_backward_ref(x[rows], w, dy[rows])
    _, rdw = gemm_backward_ref(x[:, cols], w[:, cols], dy)
    verdict(dx[rows.to(gpu)].cpu(), rdx, "gemm_backward_dx", "bf16", f"dx {M}x{N}x{K}")
    verdict(dw[:, cols.to(gpu)].cpu(), rdw, "gemm_backward_dw", "bf16", f"dw {M}x{N}x{K}")
    dx2, dw2 = kore_amd.gemm_backward(xg, wg, dyg)
    assert bit_equal(dx2, dx) and bit_equal(dw2, dw), "determinism"


def test_gemm_backward_errors(gpu):
    x = torch.zeros((8, 16), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError):
        kore_amd.gemm_backward(x, torch.zeros((4, 8), dtype=torch.bfloat16, device=gpu),
                               torch.zeros((8, 4), dtype=torch.bfloat16, device=gpu))
    with pytest.raises(ValueError):
        kore_amd.gemm_backward(x, torch.zeros((4, 16), dtype=torch.float16, device=gpu),
                               torch.zeros((8, 4), dtype=torch.bfloat16, device=gpu))


@pytest.mark.skip(reason="two GPU runs of this test ended in an illegal memory access while the library "
                         "recorded stream-ordered allocations (hipMallocAsync / hipFreeAsync graph nodes) "
                         "in the captured graph; that mechanism is removed (the caller now passes the "
                         "workspace) and this case stays off the GPU")
def test_scratch_paths_under_graph_capture(gpu):
    """Historical case, kept skipped: the packed path (K = 4095) and split-K (M = 1)
    captured on a fresh stream, replayed on another stream beside eager work on the
    capture stream.  When it faulted, the library took its scratch under capture from
    hipMallocAsync (graph allocation nodes); the library no longer allocates at all --
    the caller's workspace comes from torch (under capture: the graph's private pool),
    which test_workspace_paths_under_graph_capture covers."""
    g = torch.Generator().manual_seed(11)
    a = (torch.randn((512, 4095), generator=g) / 64).bfloat16().to(gpu)
    b = (torch.randn((4095, 1024), generator=g) / 64).bfloat16().to(gpu)
    a1 = (torch.randn((1, 4096), generator=g) / 64).bfloat16().to(gpu)
    b1 = (torch.randn((4096, 2048), generator=g) / 64).bfloat16().to(gpu)
    e_packed, e_split = kore_amd.gemm(a, b), kore_amd.gemm(a1, b1)
    torch.cuda.synchronize()
    cap = torch.cuda.Stream()
    with torch.cuda.stream(cap):  # the capture stream owns a cached buffer before capture
        assert torch.equal(kore_amd.gemm(a, b), e_packed)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        y_packed = kore_amd.gemm(a, b)
        y_split = kore_amd.gemm(a1, b1)
    other_stream = torch.cuda.Stream()
    for r in range(4):
        with torch.cuda.stream(other_stream):
            graph.replay()  # replayed on another stream while the capture stream works
        with torch.cuda.stream(cap):
            eager = kore_amd.gemm(a, b)
        torch.cuda.synchronize()
        assert torch.equal(y_packed, e_packed), f"packed replay {r}"
        assert torch.equal(y_split, e_split), f"split-K replay {r}"
        assert torch.equal(eager, e_packed), f"eager on the capture stream {r}"
        other = kore_amd.gemm(a1, b1)  # eager work on the default stream between replays
        torch.cuda.synchronize()
        assert torch.equal(other, e_split)


def test_workspace_paths_under_graph_capture(gpu):
    """The packed path (K = 4095, unaligned A rows) and split-K (M = 1) captured with
    torch.cuda.graph: the workspace ops.py allocates comes from the graph's private
    pool, so the captured kernels are the eager ones (no fallback path).  Every replay
    matches the eager result bit for bit -- on the capture's own stream with eager
    calls in between, then on a second stream while eager calls run on the default
    stream."""
    g = torch.Generator().manual_seed(11)
    a = (torch.randn((512, 4095), generator=g) / 64).bfloat16().to(gpu)
    b = (torch.randn((4095, 1024), generator=g) / 64).bfloat16().to(gpu)
    a1 = (torch.randn((1, 4096), generator=g) / 64).bfloat16().to(gpu)
    b1 = (torch.randn((4096, 2048), generator=g) / 64).bfloat16().to(gpu)
    e_packed, e_split = kore_amd.gemm(a, b), kore_amd.gemm(a1, b1)
    torch.cuda.synchronize()
    verdict(e_packed.cpu(), matmul_ref(a.cpu(), b.cpu()), "gemm", "bf16", "packed 512x1024x4095")
    verdict(e_split.cpu(), matmul_ref(a1.cpu(), b1.cpu()), "gemm", "bf16", "split-K 1x2048x4096")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_packed = kore_amd.gemm(a, b)
        y_split = kore_amd.gemm(a1, b1)
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_packed, e_packed), f"packed replay {r}"
        assert torch.equal(y_split, e_split), f"split-K replay {r}"
        assert torch.equal(kore_amd.gemm(a, b), e_packed), f"eager packed after replay {r}"
        torch.cuda.synchronize()
    other = torch.cuda.Stream()
    for r in range(3):
        y_packed.zero_()
        y_split.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(other):
            graph.replay()
        eager = kore_amd.gemm(a1, b1)  # default stream, beside the replay
        torch.cuda.synchronize()
        assert torch.equal(y_packed, e_packed), f"packed replay {r} on a second stream"
        assert torch.equal(y_split, e_split), f"split-K replay {r} on a second stream"
        assert torch.equal(eager, e_split), f"eager split-K beside replay {r}"
    del graph
