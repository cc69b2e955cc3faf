"""OCP e4m3 fp8 codec and the DeepSeek-style block-scaled GEMM oracle (CPU).

Test infrastructure only (see ``oracle/__init__.py``).

gfx950 uses the OCP ``float8_e4m3fn`` encoding with finite max 448
(``kore/tasks/aiter_ref.py:37-62``).  Scales are fp32 ``amax/448`` with a 1e-8
floor; activations are quantised per 1x128 K-group, weights per 128x128 block.
"""

from __future__ import annotations

import numpy as np
import torch

BLK = 128            # kore/tasks/_quant_common.py BLK (1x128 act, 128x128 weight)
FP8_MAX = 448.0      # OCP e4m3fn largest finite value
FP8_DTYPE = torch.float8_e4m3fn


def e4m3_decode_table() -> np.ndarray:
    """All 256 OCP e4m3fn codes -> float64, from the format definition.

    Sign bit 7, exponent bits 6..3 (bias 7), mantissa bits 2..0; exponent 0 is
    subnormal (m * 2^-9); code 0x7f / 0xff is NaN (no infinities).  Written from the
    OCP 8-bit floating point specification; used to pin torch's fp8 cast.
    """
    out = np.empty(256, dtype=np.float64)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            out[c] = np.nan
        elif e == 0:
            out[c] = s * m * 2.0 ** -9
        else:
            out[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


def quant_1x128_fp8(x: torch.Tensor):
    """Per-token 1x128-group fp8 quantiser: x[M,K] -> (xq[M,K] e4m3, xs[M,K/128] f32).

    Follows ``kore/tasks/_quant_common.py:104-112``: ``s = max(amax, 1e-8)/448``,
    ``q = clamp(x/s, +-448).to(e4m3fn)``.  Pinned by the decode table
    (round-trip error <= half an e4m3 ulp) in ``tests/test_oracle_quant.py``.
    """
    M, K = x.shape
    if K % BLK:
        raise ValueError(f"block-scale needs K % {BLK} == 0 (got K={K})")
    xb = x.float().view(M, K // BLK, BLK)
    amax = xb.abs().amax(-1, keepdim=True).clamp(min=1e-8)
    s = amax / FP8_MAX
    xq = (xb / s).clamp(-FP8_MAX, FP8_MAX).to(FP8_DTYPE).view(M, K)
    return xq, s.squeeze(-1).to(torch.float32).contiguous()


def quant_128x128_fp8(w: torch.Tensor):
    """Per-128x128-block fp8 quantiser: w[N,K] -> (wq[N,K] e4m3, ws[N/128,K/128] f32).

    Follows ``kore/tasks/_quant_common.py:115-123``.
    """
    N, K = w.shape
    if K % BLK or N % BLK:
        raise ValueError(f"block-scale needs N, K % {BLK} == 0 (got N={N}, K={K})")
    wb = w.float().view(N // BLK, BLK, K // BLK, BLK)
    amax = wb.abs().amax(dim=(1, 3), keepdim=True).clamp(min=1e-8)
    s = amax / FP8_MAX
    wq = (wb / s).clamp(-FP8_MAX, FP8_MAX).to(FP8_DTYPE).view(N, K)
    return wq, s.squeeze(1).squeeze(-1).to(torch.float32).contiguous()


def matmul_blockscale_ref(xq, wq, xs, ws) -> torch.Tensor:
    """Block-scaled fp8 GEMM oracle -> bf16 [M,N].

    ``xd[m,k] = xq[m,k]*xs[m,k//128]``, ``wd[n,k] = wq[n,k]*ws[n//128,k//128]``,
    ``Y = (xd @ wd^T).to(bf16)``; each scale applied exactly once.  Follows
    ``kore/tasks/_quant_common.py:245-252`` (``matmul_blockscale_fp32``).
    Pinned by an independent ``repeat_interleave``+``einsum`` path, power-of-two
    scale invariance and the reference's explicit-dequant check
    (``tests/test_vendor_ops.py:49-65``), all in ``tests/test_oracle_quant.py``.
    """
    M, K = xq.shape
    N = wq.shape[0]
    if K % BLK or N % BLK:
        raise ValueError(f"block-scale needs N, K % {BLK} == 0 (got N={N}, K={K})")
    xd = (xq.view(M, K // BLK, BLK).float() * xs.float()[:, :, None]).view(M, K)
    wd = (wq.view(N // BLK, BLK, K // BLK, BLK).float()
          * ws.float()[:, None, :, None]).view(N, K)
    return (xd @ wd.t()).to(torch.bfloat16)


# --------------------------------------------------------------------------- #
# a8w8 GEMM with per-row activation and per-column weight scales (fp8 / int8)
# --------------------------------------------------------------------------- #
INT8_MAX = 127.0     # kore/tasks/_quant_common.py INT8_MAX (symmetric int8)


def quant_per_tensor_fp8(x: torch.Tensor):
    """Per-tensor fp8: x -> (xq e4m3, scalar fp32 scale); ``amax`` floored at 1e-12.

    Follows ``kore/tasks/_quant_common.py:77-83`` (``quant_per_tensor_fp8``).
    """
    amax = x.float().abs().max().clamp(min=1e-12)
    s = (amax / FP8_MAX).to(torch.float32)
    xq = (x.float() / s).clamp(-FP8_MAX, FP8_MAX).to(FP8_DTYPE)
    return xq, s.reshape(())


def quant_rowwise_fp8(x: torch.Tensor):
    """Per-row fp8: x[R,K] -> (xq[R,K] e4m3, scale[R,1] fp32); ``x ~= xq * scale``.

    Follows ``kore/tasks/_quant_common.py:86-93`` (``quant_rowwise_fp8``).
    """
    amax = x.float().abs().amax(dim=-1, keepdim=True).clamp(min=1e-12)
    s = (amax / FP8_MAX).to(torch.float32)
    return (x.float() / s).clamp(-FP8_MAX, FP8_MAX).to(FP8_DTYPE), s


def quant_rowwise_int8(x: torch.Tensor):
    """Per-row symmetric int8: x[R,K] -> (xq[R,K] int8, scale[R,1] fp32).

    ``q = clamp(round(x / s), +-127)`` with round-half-even, ``s = max(amax, 1e-12)/127``;
    follows ``kore/tasks/_quant_common.py:96-101`` (``quant_rowwise_int8``).
    """
    amax = x.float().abs().amax(dim=-1, keepdim=True).clamp(min=1e-12)
    s = (amax / INT8_MAX).to(torch.float32)
    return (x.float() / s).round().clamp(-INT8_MAX, INT8_MAX).to(torch.int8), s


def quant_per_tensor_int8(x: torch.Tensor):
    """Per-tensor symmetric int8 (``kore/tasks/vendor_ops.py:163-177``, int8 branch)."""
    amax = x.float().abs().max().clamp(min=1e-12)
    s = (amax / INT8_MAX).to(torch.float32)
    return (x.float() / s).round().clamp(-INT8_MAX, INT8_MAX).to(torch.int8), s.reshape(())


def matmul_a8w8_ref(xq, wq, x_scale, w_scale) -> torch.Tensor:
    """8-bit (fp8 / int8) a8w8 GEMM oracle -> bf16 [M,N].

    ``(xq * x_scale[M,1]) @ (wq * w_scale.reshape(-1,1))^T`` in fp32, one cast; covers
    per-tensor (equal scales), per-token / per-channel and int8.  Follows
    ``kore/tasks/_quant_common.py:236-242`` (``matmul_a8w8_fp32``).  Pinned in
    ``tests/test_oracle_quant.py`` by the reference test's explicit dequant
    (``tests/test_vendor_ops.py:38-65``), exact int64 arithmetic for int8 on small K,
    and power-of-two scale invariance.
    """
    a = xq.float() * x_scale.float().reshape(-1, 1)
    w = wq.float() * w_scale.float().reshape(-1, 1)
    return (a @ w.t()).to(torch.bfloat16)
