"""Pin the fp8 codec, the quantisers and the block-scaled GEMM oracle on the CPU."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kore_amd import workloads as W
from oracle.quant import (FP8_MAX, e4m3_decode_table, matmul_blockscale_ref, quant_128x128_fp8,
                          quant_1x128_fp8)


def test_e4m3_decode_table_matches_torch():
    table = e4m3_decode_table()
    codes = torch.arange(256, dtype=torch.uint8)
    got = codes.view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    nan = np.isnan(table)
    assert np.array_equal(np.isnan(got), nan) and nan.sum() == 2
    assert np.array_equal(got[~nan], table[~nan])
    assert np.nanmax(table) == FP8_MAX and np.nanmin(table) == -FP8_MAX


def test_e4m3_encode_is_round_to_nearest_even():
    table = e4m3_decode_table()
    finite = np.where(~np.isnan(table))[0]
    vals = table[finite]
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-448, 448, 4000), rng.uniform(-1, 1, 4000) * 2.0 ** -6]).astype(np.float32)
    # exact midpoints between neighbours (ties) as well
    pos = np.unique(np.abs(vals))
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mids, -mids])
    codes = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    for xi, c in zip(x, codes):
        d = np.abs(pos - abs(float(xi)))
        best = d.min()
        cands = pos[np.isclose(d, best, rtol=0, atol=0)]
        dec = abs(table[c])
        assert dec in cands, (xi, dec, cands)
        if len(cands) == 2:  # tie: even mantissa (last bit 0)
            assert (c & 1) == 0


@pytest.mark.parametrize("M,K", [(3, 128), (5, 256), (2, 512)])
def test_quant_1x128_roundtrip(M, K):
    g = torch.Generator().manual_seed(M)
    x = torch.randn((M, K), generator=g) * 3
    xq, xs = quant_1x128_fp8(x)
    assert xq.dtype == torch.float8_e4m3fn and xs.shape == (M, K // 128)
    deq = xq.float().view(M, K // 128, 128) * xs[:, :, None]
    err = (deq.view(M, K) - x).abs()
    # half an e4m3 ulp at the top binade (32 at 448) relative to 448, per group
    bound = (xs[:, :, None] * 16.0).expand(M, K // 128, 128).reshape(M, K)
    assert (err <= bound + 1e-12).all()
    amax = x.view(M, K // 128, 128).abs().amax(-1)
    assert torch.allclose(xs, amax / 448.0)
    assert (xq.float().view(M, K // 128, 128).abs().amax(-1) == 448.0).all()


def test_quant_128x128_shapes_and_block_scale():
    g = torch.Generator().manual_seed(7)
    w = torch.randn((256, 384), generator=g)
    wq, ws = quant_128x128_fp8(w)
    assert wq.shape == (256, 384) and ws.shape == (2, 3)
    blk = w.view(2, 128, 3, 128).abs().amax(dim=(1, 3))
    assert torch.allclose(ws, blk / 448.0)


def test_quant_zero_block_uses_floor():
    xq, xs = quant_1x128_fp8(torch.zeros((1, 128)))
    assert (xq.float() == 0).all() and torch.allclose(xs, torch.tensor([[1e-8 / 448.0]]))


def _blockscale_independent(xq, wq, xs, ws):
    """repeat_interleave + einsum path (the reference draft sanity check's second path)."""
    xsf = xs.repeat_interleave(128, dim=1)                                   # [M,K]
    wsf = ws.repeat_interleave(128, dim=0).repeat_interleave(128, dim=1)     # [N,K]
    return torch.einsum("mk,nk->mn", xq.float() * xsf, wq.float() * wsf).to(torch.bfloat16)


@pytest.mark.parametrize("M,N,K", [(3, 128, 128), (5, 256, 256), (7, 384, 256)])
def test_blockscale_ref_independent_path(M, N, K):
    g = torch.Generator().manual_seed(M * N)
    xq, xs = quant_1x128_fp8(torch.randn((M, K), generator=g))
    wq, ws = quant_128x128_fp8(torch.randn((N, K), generator=g))
    got = matmul_blockscale_ref(xq, wq, xs, ws)
    want = _blockscale_independent(xq, wq, xs, ws)
    assert got.shape == (M, N) and got.dtype == torch.bfloat16
    assert torch.allclose(got.float(), want.float(), atol=1e-2, rtol=1e-2)


def test_blockscale_each_scale_applied_once():
    """Doubling one x-scale group doubles exactly that group's contribution."""
    g = torch.Generator().manual_seed(11)
    xq, xs = quant_1x128_fp8(torch.randn((4, 256), generator=g))
    wq, ws = quant_128x128_fp8(torch.randn((128, 256), generator=g))
    y = matmul_blockscale_ref(xq, wq, xs, ws).float()
    assert torch.equal(matmul_blockscale_ref(xq, wq, xs * 2, ws).float(), y * 2)   # pow2 invariance
    xs2 = xs.clone()
    xs2[:, 1] = 0
    part0 = matmul_blockscale_ref(xq, wq, xs2, ws).float()
    xs3 = xs.clone()
    xs3[:, 0] = 0
    part1 = matmul_blockscale_ref(xq, wq, xs3, ws).float()
    # each of the three results carries one bf16 rounding (half an ulp, 2^-9 relative)
    bound = 2.0 ** -8 * (part0.abs() + part1.abs() + y.abs()) + 1e-6
    assert ((part0 + part1 - y).abs() <= bound).all()


def test_blockscale_vs_explicit_dequant_like_reference_test():
    """The reference's own check (tests/test_vendor_ops.py:49-65): oracle == explicit
    dequantised fp32 matmul within allclose(1e-2)."""
    g = torch.Generator().manual_seed(0)
    X = torch.randn((8, 256), generator=g) * 0.2
    Wt = torch.randn((128, 256), generator=g) * 0.2
    xq, xs = quant_1x128_fp8(X)
    wq, ws = quant_128x128_fp8(Wt)
    out = matmul_blockscale_ref(xq, wq, xs, ws)
    xd = xq.float() * xs.repeat_interleave(128, 1)
    wd = wq.float() * ws.repeat_interleave(128, 0).repeat_interleave(128, 1)
    assert torch.allclose(out.float(), xd @ wd.t(), atol=1e-2, rtol=1e-2)


def test_blockscale_rejects_k_not_multiple_of_128():
    with pytest.raises(ValueError):
        quant_1x128_fp8(torch.zeros((4, 4095)))
    with pytest.raises(ValueError):
        matmul_blockscale_ref(torch.zeros((4, 4095), dtype=torch.float8_e4m3fn),
                              torch.zeros((128, 4095), dtype=torch.float8_e4m3fn),
                              torch.ones((4, 31)), torch.ones((1, 31)))


def test_workload_quantisers_match_oracle_bit_exact():
    g = torch.Generator().manual_seed(5)
    x = torch.randn((64, 512), generator=g)
    w = torch.randn((256, 512), generator=g)
    a1, s1 = W.quant_1x128(x)
    a2, s2 = quant_1x128_fp8(x)
    assert torch.equal(a1.view(torch.uint8), a2.view(torch.uint8)) and torch.equal(s1, s2)
    b1, t1 = W.quant_128x128(w)
    b2, t2 = quant_128x128_fp8(w)
    assert torch.equal(b1.view(torch.uint8), b2.view(torch.uint8)) and torch.equal(t1, t2)
