"""Dense, fused-epilogue and batched GEMM oracles (CPU, torch fp32).

Test infrastructure only (see ``oracle/__init__.py``).

Every oracle upcasts its low-precision inputs to fp32, runs one fp32 matmul, and
casts the result once (round-to-nearest-even) to the output dtype -- exactly the
reference's recipe.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

ACTS = ("none", "relu", "gelu", "silu", "tanh", "sigmoid")


def act_fp32(name: str, y: torch.Tensor) -> torch.Tensor:
    """fp32 activation by KORE act code.

    Follows ``kore/tasks/_genops.py:294-304`` (``_torch_act``): gelu is the tanh
    approximation (``F.gelu(approximate="tanh")``), silu is ``F.silu``.
    Pinned by closed forms in ``tests/test_oracle_gemm.py``.
    """
    if name == "none":
        return y
    if name == "relu":
        return torch.relu(y)
    if name == "gelu":
        return F.gelu(y, approximate="tanh")
    if name == "silu":
        return F.silu(y)
    if name == "tanh":
        return torch.tanh(y)
    if name == "sigmoid":
        return torch.sigmoid(y)
    raise ValueError(f"unknown activation {name!r}")


def matmul_ref(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Dense bf16 GEMM oracle: ``(a.float() @ b.float()).to(bf16)``.

    a[M,K], b[K,N] (any strides).  Follows ``kore/tasks/gemm_bf16/reference.py:39-41``.
    Pinned by an fp64 brute force (``tests/test_oracle_gemm.py``).
    """
    return (a.float() @ b.float()).to(torch.bfloat16)


def gemm_fusion_ref(a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None,
                    act: str) -> torch.Tensor:
    """GEMM + fused bias/activation oracle: ``act(a@b [+bias]).to(a.dtype)``.

    Follows ``kore/tasks/_genops.py:446-451`` (gemm_fusion ``ref_fn``): bias is
    added in fp32 before the activation, one final cast to the input dtype.
    Pinned by closed-form activations on an fp64 GEMM (``tests/test_oracle_gemm.py``).
    """
    y = a.float() @ b.float()
    if bias is not None:
        y = y + bias.float()
    return act_fp32(act, y).to(a.dtype)


def batched_gemm_ref(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Batched GEMM oracle: ``C[i] = A[i] @ B[i]^T``; a[B,M,K], b[B,N,K].

    Follows ``kore/tasks/vendor_ops.py:373-374`` and
    ``kore/tasks/_moe_common.py:252-258`` (``batched_gemm_fp32``).
    Pinned per batch against ``matmul_ref`` and a batch-permutation relation.
    """
    return torch.bmm(a.float(), b.float().transpose(1, 2)).to(a.dtype)


def gemm_backward_ref(x: torch.Tensor, w: torch.Tensor, dy: torch.Tensor):
    """Linear-layer backward oracle for ``Y = X @ W^T``: fp32 ``(dX, dW)``.

    ``dX = dY @ W`` and ``dW = dY^T @ X`` on fp32 upcasts -- the gradients torch
    autograd gives for the fp32 forward, which is the reference's oracle
    (``kore/tasks/gemm_backward_bf16/reference.py:64-72``).  Pinned against autograd
    and central finite differences in ``tests/test_oracle_gemm.py``.
    """
    xf, wf, dyf = x.float(), w.float(), dy.float()
    return dyf @ wf, dyf.t() @ xf
