"""Pin the dense / fused / batched GEMM oracles (oracle/gemm.py) on the CPU.

Each check is independent of the formula it pins: fp64 triple loops, a bit-level
numpy round-to-nearest-even bf16/fp16 cast, closed-form activations in fp64, and
cases built so a plausible mistake (transposed operand, bias after the activation,
exact GELU instead of tanh GELU, a missing final cast) fails.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.gemm import act_fp32, batched_gemm_ref, gemm_backward_ref, gemm_fusion_ref, matmul_ref


def bf16_rne(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 -> fp32 by bit manipulation: round to nearest, ties to even."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) & 0xFFFF0000).astype(np.uint32)
    out = r.view(np.float32).copy()
    out[np.isnan(x)] = np.nan
    return out


def matmul_f64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    M, K = a.shape
    N = b.shape[1]
    out = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        for n in range(N):
            s = 0.0
            for k in range(K):
                s += float(a[m, k]) * float(b[k, n])
            out[m, n] = s
    return out


def test_bf16_cast_is_rne():
    """torch's fp32->bf16 cast (used by every oracle) is RNE, including ties and overflow."""
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(20000) * 10.0 ** rng.integers(-30, 30, 20000)).astype(np.float32)
    ties = np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -(1.0 + 2 ** -8), 3.3895314e38, 3.4e38], dtype=np.float32)
    x = np.concatenate([x, ties])
    got = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    want = bf16_rne(x)
    assert np.array_equal(got, want)
    assert got[-5] == 1.0 and got[-4] == 1.0 + 2 ** -6  # ties go to the even neighbour
    assert np.isinf(got[-1])                           # overflow rounds to inf


def test_matmul_ref_matches_fp64_bruteforce():
    g = torch.Generator().manual_seed(0)
    a = torch.randn((7, 13), generator=g).to(torch.bfloat16)
    b = torch.randn((13, 5), generator=g).to(torch.bfloat16)   # non-square: a transpose fails
    got = matmul_ref(a, b)
    assert got.dtype == torch.bfloat16 and got.shape == (7, 5)
    want = bf16_rne(matmul_f64(a.float().numpy(), b.float().numpy()).astype(np.float32))
    # fp32 accumulation vs exact fp64: the bf16 results may differ by one ulp at most
    ulp = np.abs(want) * 2 ** -7 + 1e-30
    assert (np.abs(got.float().numpy() - want) <= ulp).all()


def test_matmul_ref_strided_views():
    """b = B.t() views give the same result as a contiguous copy (A.B^T convention)."""
    g = torch.Generator().manual_seed(1)
    a = torch.randn((6, 9), generator=g).to(torch.bfloat16)
    B = torch.randn((4, 9), generator=g).to(torch.bfloat16)
    assert torch.equal(matmul_ref(a, B.t()), matmul_ref(a, B.t().contiguous()))


def _gelu_tanh(x: float) -> float:
    return 0.5 * x * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


CLOSED = {
    "none": lambda x: x,
    "relu": lambda x: max(x, 0.0),
    "gelu": _gelu_tanh,
    "silu": lambda x: x / (1.0 + math.exp(-x)),
    "tanh": math.tanh,
    "sigmoid": lambda x: 1.0 / (1.0 + math.exp(-x)),
}


@pytest.mark.parametrize("act", list(CLOSED))
def test_activation_closed_forms(act):
    xs = np.linspace(-8, 8, 321, dtype=np.float32)
    got = act_fp32(act, torch.from_numpy(xs)).numpy()
    want = np.array([CLOSED[act](float(v)) for v in xs])
    assert np.allclose(got, want, rtol=2e-6, atol=2e-7)


def test_gelu_is_tanh_approximation_not_exact():
    x = torch.tensor([1.5])
    exact = 0.5 * 1.5 * (1 + math.erf(1.5 / math.sqrt(2)))
    got = act_fp32("gelu", x).item()
    assert abs(got - _gelu_tanh(1.5)) < 1e-6 and abs(got - exact) > 1e-4


@pytest.mark.parametrize("act", ["relu", "gelu", "silu", "tanh", "sigmoid"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_gemm_fusion_ref_closed_form(act, dtype):
    g = torch.Generator().manual_seed(2)
    a = (torch.randn((5, 11), generator=g) * 0.5).to(dtype)
    b = (torch.randn((11, 6), generator=g) * 0.5).to(dtype)
    bias = torch.randn((6,), generator=g).to(dtype)
    got = gemm_fusion_ref(a, b, bias, act)
    assert got.dtype == dtype
    y = matmul_f64(a.float().numpy(), b.float().numpy()) + bias.float().numpy()[None, :]
    want = np.vectorize(CLOSED[act])(y)
    cast = torch.from_numpy(want.astype(np.float32)).to(dtype).float().numpy()
    ulp = np.abs(cast) * (2 ** -7 if dtype == torch.bfloat16 else 2 ** -10) + 1e-6
    assert (np.abs(got.float().numpy() - cast) <= ulp).all()


def test_bias_is_added_before_the_activation():
    a = torch.tensor([[1.0]], dtype=torch.float16)
    b = torch.tensor([[-2.0]], dtype=torch.float16)
    bias = torch.tensor([3.0], dtype=torch.float16)
    assert gemm_fusion_ref(a, b, bias, "relu").item() == 1.0   # relu(-2+3); relu(-2)+3 would be 3


def test_gemm_fusion_overflow_gives_inf_in_fp16():
    """The generic 'large' adversarial fill overflows fp16 to +-inf in the oracle."""
    a = torch.full((2, 512), 1e3, dtype=torch.float16)
    b = torch.full((512, 3), 1e3, dtype=torch.float16)
    out = gemm_fusion_ref(a, b, None, "none")
    assert torch.isinf(out).all() and (out > 0).all()
    neg = gemm_fusion_ref(a, -b, None, "gelu")      # gelu(-5e8) -> -0 (finite)
    assert torch.isfinite(neg).all() and (neg.float() == 0).all()


def test_batched_ref_per_batch_and_permutation():
    g = torch.Generator().manual_seed(3)
    a = torch.randn((4, 6, 8), generator=g).to(torch.bfloat16)
    b = torch.randn((4, 5, 8), generator=g).to(torch.bfloat16)
    got = batched_gemm_ref(a, b)
    assert got.shape == (4, 6, 5)
    for i in range(4):
        assert torch.equal(got[i], matmul_ref(a[i], b[i].t()))
    perm = torch.tensor([2, 0, 3, 1])
    assert torch.equal(batched_gemm_ref(a[perm], b[perm]), got[perm])


def test_gemm_backward_oracle_is_the_autograd_gradient():
    """The backward oracle equals torch autograd of the fp32 forward X @ W^T (the
    reference's oracle, kore/tasks/gemm_backward_bf16/reference.py:64-72) and central
    finite differences of L = sum(dY * (X @ W^T)) in float64; swapping the two
    gradients (or dropping the transpose on dY) fails both."""
    from kore_amd import workloads as W

    x, w, dy = W.backward_inputs(16, 12, 20, seed=3)
    dx, dw = gemm_backward_ref(x, w, dy)
    assert dx.shape == (16, 20) and dw.shape == (12, 20) and dx.dtype == torch.float32
    xf = x.float().requires_grad_(True)
    wf = w.float().requires_grad_(True)
    (xf @ wf.t()).backward(dy.float())
    assert torch.allclose(dx, xf.grad, rtol=1e-5, atol=1e-6)
    assert torch.allclose(dw, wf.grad, rtol=1e-5, atol=1e-6)
    xd, wd, dyd = x.double(), w.double(), dy.double()

    def loss(a, b):
        return float((dyd * (a @ b.t())).sum())

    h = 1e-3
    for i, j in [(0, 0), (5, 7), (15, 19)]:
        e = torch.zeros_like(xd)
        e[i, j] = h
        assert abs((loss(xd + e, wd) - loss(xd - e, wd)) / (2 * h) - float(dx[i, j])) < 1e-4
    for i, j in [(0, 0), (3, 11), (11, 19)]:
        e = torch.zeros_like(wd)
        e[i, j] = h
        assert abs((loss(xd, wd + e) - loss(xd, wd - e)) / (2 * h) - float(dw[i, j])) < 1e-4
