"""Fake (shape-only) implementations of the ``torch.ops.korehip`` operators.

The operators are registered in C++ (``kore_amd/ext/kore_ops.cpp``) with one
CompositeExplicitAutograd kernel that insists on HIP tensors.  Tracing (FakeTensor,
``torch.compile``, ``make_fx``) must not run that kernel: it would take data pointers
of storage-less tensors.  Each function here returns empty tensors of the shape and
dtype the real operator returns, computed from the input shapes only, and applies the
same shape checks so that a trace fails where the call would.
"""

from __future__ import annotations

import torch

_FP8 = torch.float8_e4m3fn


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _align_capacity(slots: int, experts: int, block: int) -> int:
    """Slots after padding every expert to a multiple of ``block`` (the C ABI's
    ``kore_moe_align_capacity``): ``align_up(slots + E*(block-1), block)``."""
    n = slots + experts * (block - 1)
    return -(-n // block) * block


def _register() -> None:
    reg = torch.library.register_fake

    @reg("korehip::gemm")
    def _gemm(a, b):
        _check(a.dim() == 2 and b.dim() == 2 and a.shape[1] == b.shape[0], "gemm expects a[M,K] @ b[K,N]")
        return a.new_empty((a.shape[0], b.shape[1]))

    @reg("korehip::gemm_fused")
    def _gemm_fused(a, b, bias, act):
        _check(a.dim() == 2 and b.dim() == 2 and a.shape[1] == b.shape[0], "gemm expects a[M,K] @ b[K,N]")
        _check(bias is None or (bias.dim() == 1 and bias.shape[0] == b.shape[1]), "bias must be [N]")
        return a.new_empty((a.shape[0], b.shape[1]))

    @reg("korehip::batched_gemm")
    def _batched(a, b):
        _check(a.dim() == 3 and b.dim() == 3 and a.shape[0] == b.shape[0] and a.shape[2] == b.shape[2],
               "batched_gemm expects a[B,M,K], b[B,N,K]")
        return a.new_empty((a.shape[0], a.shape[1], b.shape[1]))

    @reg("korehip::gemm_backward")
    def _backward(x, w, dy):
        _check(x.dim() == 2 and w.dim() == 2 and dy.dim() == 2 and w.shape[1] == x.shape[1]
               and dy.shape[0] == x.shape[0] and dy.shape[1] == w.shape[0],
               "gemm_backward expects x[M,K], w[N,K], dy[M,N]")
        return x.new_empty(tuple(x.shape)), x.new_empty(tuple(w.shape))

    @reg("korehip::gemm_a8w8_blockscale")
    def _blockscale(xq, wq, x_scale, w_scale):
        _check(xq.dim() == 2 and wq.dim() == 2 and xq.shape[1] == wq.shape[1], "expected xq[M,K], wq[N,K]")
        return xq.new_empty((xq.shape[0], wq.shape[0]), dtype=torch.bfloat16)

    @reg("korehip::gemm_a8w8")
    def _a8w8(xq, wq, x_scale, w_scale):
        _check(xq.dim() == 2 and wq.dim() == 2 and xq.shape[1] == wq.shape[1], "expected xq[M,K], wq[N,K]")
        return xq.new_empty((xq.shape[0], wq.shape[0]), dtype=torch.bfloat16)

    @reg("korehip::moe_align")
    def _align(topk_ids, num_experts, block):
        _check(topk_ids.dim() == 2 and num_experts > 0 and block > 0, "moe_align expects topk_ids[T, topk]")
        cap = _align_capacity(topk_ids.shape[0] * topk_ids.shape[1], num_experts, block)
        i32 = torch.int32
        return (topk_ids.new_empty((num_experts + 1,), dtype=i32), topk_ids.new_empty((cap,), dtype=i32),
                topk_ids.new_empty((cap // block,), dtype=i32))

    @reg("korehip::fused_moe")
    def _fused_moe(hidden, w1, w2, topk_weight, topk_ids):
        _check(hidden.dim() == 2 and w1.dim() == 3 and w2.dim() == 3, "expected hidden[T,D], w1[E,2I,D], w2[E,D,I]")
        return hidden.new_empty(tuple(hidden.shape))

    @reg("korehip::grouped_gemm")
    def _grouped(hidden, w, expert_ids):
        _check(hidden.dim() == 2 and w.dim() == 3 and w.shape[2] == hidden.shape[1],
               "grouped_gemm expects hidden[M,K], w[E,N,K]")
        _check(expert_ids.numel() == hidden.shape[0], "expert_ids must hold one id per row")
        return hidden.new_empty((hidden.shape[0], w.shape[1]))

    @reg("korehip::grouped_gemm_fp8")
    def _grouped_fp8(xq, wq, x_scale, w_scale, expert_ids):
        _check(xq.dim() == 2 and wq.dim() == 3 and wq.shape[2] == xq.shape[1],
               "grouped_gemm_fp8 expects xq[M,K], wq[E,N,K]")
        _check(expert_ids.numel() == xq.shape[0] and x_scale.numel() == xq.shape[0]
               and w_scale.numel() == wq.shape[0] * wq.shape[1], "expected expert_ids[M], x_scale[M], w_scale[E,N]")
        return xq.new_empty((xq.shape[0], wq.shape[1]), dtype=torch.bfloat16)

    @reg("korehip::gather_rows")
    def _gather(src, idx):
        _check(src.dim() == 2 and idx.dim() == 1, "gather_rows expects src[rows, D], idx[n]")
        return src.new_empty((idx.shape[0], src.shape[1]))

    @reg("korehip::scatter_rows")
    def _scatter(src, idx):
        _check(src.dim() == 2 and idx.dim() == 1 and idx.shape[0] <= src.shape[0],
               "scatter_rows expects src[rows, D], idx[n <= rows]")
        return src.new_empty(tuple(src.shape))


_register()
