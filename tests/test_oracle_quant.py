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


# ---------------------------------------------------------------------------
# a8w8 (per-row / per-column scales, fp8 and int8)
# ---------------------------------------------------------------------------
from oracle.quant import (  # noqa: E402
    matmul_a8w8_ref, quant_per_tensor_fp8, quant_per_tensor_int8, quant_rowwise_fp8, quant_rowwise_int8,
)


def test_int8_quantiser_rounding_and_clamp():
    """Symmetric int8: s = amax/127, q = clamp(round-half-even(x/s), +-127)."""
    x = torch.tensor([[127.0, 0.5, 1.5, -2.5, 63.5, -127.0]])
    q, s = quant_rowwise_int8(x)
    assert s.shape == (1, 1) and float(s) == 1.0
    assert q.tolist() == [[127, 0, 2, -2, 64, -127]]
    z, sz = quant_rowwise_int8(torch.zeros(2, 4))
    assert torch.all(z == 0) and torch.all(sz == 1e-12 / 127.0)
    qt, st = quant_per_tensor_int8(torch.tensor([[1.0, -254.0]]))
    assert float(st) == 2.0 and qt.tolist() == [[0, -127]]


def test_rowwise_fp8_quantiser_roundtrip():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(16, 96, generator=g) * 3
    q, s = quant_rowwise_fp8(x)
    assert q.dtype == torch.float8_e4m3fn and s.shape == (16, 1)
    assert torch.allclose(s[:, 0], x.abs().amax(-1) / 448.0)
    assert torch.all(q.float().abs().amax(-1) == 448.0)  # each row's amax maps to 448
    # relative error of an e4m3 normal is at most half an ulp (2^-4)
    rel = ((q.float() * s - x).abs() / x.abs().clamp(min=1e-3 * float(s.max())))
    assert float(rel.max()) <= 2.0 ** -4 + 1e-6
    qt, st = quant_per_tensor_fp8(x)
    assert st.shape == () and float(qt.float().abs().max()) == 448.0


@pytest.mark.parametrize("kind", ["fp8", "int8"])
def test_a8w8_oracle_matches_explicit_dequant(kind):
    """The reference's own checks (tests/test_vendor_ops.py:38-65): the oracle equals the
    explicit dequantised matmul at M=8, N=16, K=32."""
    g = torch.Generator().manual_seed(0)
    a, w = torch.randn(8, 32, generator=g), torch.randn(16, 32, generator=g)
    quant = quant_rowwise_fp8 if kind == "fp8" else quant_rowwise_int8
    xq, xs = quant(a)
    wq, wsc = quant(w)
    ws = wsc.reshape(1, 16)
    out = matmul_a8w8_ref(xq, wq, xs, ws)
    assert out.shape == (8, 16) and out.dtype == torch.bfloat16
    exp = (xq.float() * xs.float()) @ (wq.float() * ws.float().reshape(-1, 1)).t()
    assert torch.allclose(out.float(), exp, atol=1e-2, rtol=1e-2)
    # the weight scale belongs to output columns: applying it per row must differ
    wrong = ((xq.float() * ws.float().reshape(1, -1)[:, :8].reshape(-1, 1)) @ (wq.float() * xs.float()[:1]).t())
    assert not torch.allclose(out.float(), wrong, atol=1e-2, rtol=1e-2)


def test_a8w8_int8_exact_and_scale_invariance():
    """int8 products and sums up to K=64 are exact integers in fp32: with unit scales the
    oracle is the int64 matmul rounded once to bf16; doubling x_scale doubles Y exactly."""
    g = torch.Generator().manual_seed(5)
    xq = torch.randint(-127, 128, (12, 64), generator=g, dtype=torch.int8)
    wq = torch.randint(-127, 128, (20, 64), generator=g, dtype=torch.int8)
    one_x, one_w = torch.ones(12, 1), torch.ones(1, 20)
    exact = (xq.long() @ wq.long().t()).double().float().to(torch.bfloat16)
    assert torch.equal(matmul_a8w8_ref(xq, wq, one_x, one_w), exact)
    xs = torch.rand(12, 1, generator=g) + 0.5
    ws = torch.rand(1, 20, generator=g) + 0.5
    y1 = matmul_a8w8_ref(xq, wq, xs, ws)
    assert torch.equal(matmul_a8w8_ref(xq, wq, xs * 2, ws), (y1.float() * 2).to(torch.bfloat16))
    # w_scale given as [N,1] or [N] is the same operand
    assert torch.equal(matmul_a8w8_ref(xq, wq, xs, ws.reshape(20, 1)), y1)
    assert torch.equal(matmul_a8w8_ref(xq, wq, xs, ws.reshape(20)), y1)
