"""Fused top-k MoE (SiLU gated MLP) oracle, router and sort/align oracle (CPU).

Test infrastructure only (see ``oracle/__init__.py``).

Weight layout follows the reference task (``kore/tasks/fused_moe_silu_bf16/
reference.py:1-22``): ``w1[E, 2I, D]`` with the gate rows first and the up rows
second, ``w2[E, D, I]``.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

# Jagged per-expert weighting used as a router bias by the reference so the token
# counts are unbalanced and the last expert is dead
# (kore/tasks/fused_moe_silu_bf16/reference.py:34-38, _moe_common.py:93-97).
TRACE32 = [
    16053, 105, 1843, 2724, 327, 88, 4102, 51, 9210, 61, 3020, 44, 1502, 990,
    233, 77, 6740, 120, 410, 58, 2210, 39, 812, 175, 5030, 66, 1360, 92, 3550,
    47, 1180, 0,
]


def jagged_counts(E: int) -> list[int]:
    """Per-expert count pattern of length E with a dead last expert.

    Follows ``kore/tasks/_moe_common.py:100-113`` (``jagged_counts``).
    """
    if E <= len(TRACE32):
        c = list(TRACE32[:E])
    else:
        tile = [x for x in TRACE32 if x > 0]
        c = [tile[i % len(tile)] for i in range(E)]
    c[-1] = 0
    return c


def trace32_bias(E: int) -> torch.Tensor:
    """Router bias ``log(count + 1e-6)`` with ``-inf`` on dead experts.

    Follows ``kore/tasks/_moe_common.py:123-125``.
    """
    counts = torch.tensor([float(x) for x in jagged_counts(E)], dtype=torch.float32)
    bias = torch.log(counts + 1e-6)
    bias[counts == 0] = float("-inf")
    return bias


def route(logits: torch.Tensor, topk: int, renorm: bool = True):
    """softmax -> top-k -> (optional) renormalisation.

    Returns ``(topk_weight[T,topk] f32, topk_ids[T,topk] int32)``.  Follows
    ``kore/tasks/_moe_common.py:126-132`` (``make_routing``) and
    ``fused_moe_silu_bf16/reference.py:62-66``.  Pinned by invariants in
    ``tests/test_oracle_moe.py`` (weights sum to one, ids are the arg-max set).
    """
    probs = torch.softmax(logits.float(), dim=-1)
    tw, ti = torch.topk(probs, topk, dim=-1)
    if renorm:
        tw = tw / tw.sum(dim=-1, keepdim=True)
    return tw.to(torch.float32), ti.to(torch.int32)


def silu_fp32(x: torch.Tensor) -> torch.Tensor:
    return F.silu(x.float())


def moe_ref(hidden, w1, w2, topk_weight, topk_ids) -> torch.Tensor:
    """Exact fp32 top-k fused-MoE oracle -> hidden.dtype [T, D].

    Per expert e (ascending): ``gu = x_e @ w1[e]^T``; ``h = silu(gu[:, :I]) * gu[:, I:]``;
    ``y = h @ w2[e]^T``; ``out[idx] += y * w_e`` where ``w_e`` sums the token's
    router weights over the slots that chose e.  Experts with no token are skipped;
    ids outside ``[0, E)`` match no expert and contribute nothing.  Follows
    ``kore/tasks/fused_moe_silu_bf16/reference.py:81-105`` (identical to
    ``_moe_common.gated_mlp_fp32``, ``_moe_common.py:165-200``).
    Pinned against two independent paths (per-(token, slot) loop and a dense
    all-experts formulation) in ``tests/test_oracle_moe.py``.
    """
    T, D = hidden.shape
    E = w1.shape[0]
    I = w2.shape[2]
    x = hidden.float()
    w1f = w1.float()
    w2f = w2.float()
    out = torch.zeros((T, D), dtype=torch.float32)
    ids = topk_ids.long()
    tw = topk_weight.float()
    for e in range(E):
        mask = ids == e
        tok = mask.any(dim=1)
        if not bool(tok.any()):
            continue
        idx = tok.nonzero(as_tuple=True)[0]
        gate_up = x[idx] @ w1f[e].t()
        h = silu_fp32(gate_up[:, :I]) * gate_up[:, I:]
        ye = h @ w2f[e].t()
        w_e = (tw * mask.float()).sum(dim=1)[idx]
        out[idx] += ye * w_e[:, None]
    return out.to(hidden.dtype)


def moe_align_ref(topk_ids, E: int, block: int):
    """Sort/align oracle for the MoE dispatch (brute force).

    Slots are ``s = t*topk + k``.  Returns numpy int32 arrays:
      ``offsets[E+1]``: exclusive cumsum of ``ceil(count_e/block)*block``
                        (``kore/tasks/breadth/moe_ext.py:617-621``, ``align_offsets``);
      ``sorted_slots[offsets[E]]``: slots grouped by expert ascending, stable
                        (ascending slot order within an expert, as in
                        ``_moe_common.permute_tokens`` ``:317-329``), each expert's
                        run padded to a block multiple with the sentinel ``T*topk``;
      ``block_expert[offsets[E]//block]``: the expert owning each block.
    Ids outside ``[0, E)`` are dropped (they match no expert in ``moe_ref``).
    """
    ids = np.asarray(topk_ids, dtype=np.int64)
    T, topk = ids.shape
    flat = ids.reshape(-1)
    S = T * topk
    valid = (flat >= 0) & (flat < E)
    counts = np.bincount(flat[valid], minlength=E)[:E]
    padded = (counts + block - 1) // block * block
    offsets = np.zeros(E + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(padded)
    total = int(offsets[-1])
    sorted_slots = np.full(total, S, dtype=np.int64)
    block_expert = np.zeros(total // block, dtype=np.int64)
    slots = np.arange(S)
    for e in range(E):
        mine = slots[valid & (flat == e)]
        sorted_slots[offsets[e]:offsets[e] + mine.size] = mine
        block_expert[offsets[e] // block: offsets[e + 1] // block] = e
    return (offsets.astype(np.int32), sorted_slots.astype(np.int32),
            block_expert.astype(np.int32))


def grouped_gemm_ref(hidden, w, expert_ids) -> torch.Tensor:
    """Top-1 grouped expert GEMM oracle -> hidden.dtype [M, N] in token order.

    ``out[m] = hidden[m] @ w[expert_ids[m]]^T`` in fp32, one cast; experts with no
    token are never visited and ids outside ``[0, E)`` leave a zero row.  Follows
    ``kore/tasks/_moe_common.py:203-226`` (``grouped_gemm_fp32``).  Pinned in
    ``tests/test_oracle_moe.py`` by per-token matvecs (an independent gather path) and
    the dense one-hot form.
    """
    M, K = hidden.shape
    E, N, _ = w.shape
    x, wf = hidden.float(), w.float()
    out = torch.zeros((M, N), dtype=torch.float32)
    eids = expert_ids.reshape(-1).long()
    for e in range(E):
        idx = (eids == e).nonzero(as_tuple=True)[0]
        if idx.numel():
            out[idx] = x[idx] @ wf[e].t()
    return out.to(hidden.dtype)


def grouped_gemm_fp8_ref(xq, wq, x_scale, w_scale, expert_ids) -> torch.Tensor:
    """Top-1 grouped fp8 a8w8 expert GEMM oracle -> bf16 [M, N] in token order.

    ``out[m] = (xq[m]*x_scale[m]) @ (wq[e]*w_scale[e])^T`` with ``e = expert_ids[m]``,
    fp32 of the dequantised operands, one cast; ids outside ``[0, E)`` leave a zero row.
    Follows ``kore/tasks/_moe_common.py:228-249`` (``grouped_gemm_fp8_fp32``).  Pinned in
    ``tests/test_oracle_moe.py`` by per-token dequantised matvecs and, with every token
    on one expert, the dense a8w8 oracle.
    """
    M, K = xq.shape
    E, N, _ = wq.shape
    xd = xq.float() * x_scale.float().reshape(M, 1)
    wd = wq.float() * w_scale.float().reshape(E, N, 1)
    out = torch.zeros((M, N), dtype=torch.float32)
    eids = expert_ids.reshape(-1).long()
    for e in range(E):
        idx = (eids == e).nonzero(as_tuple=True)[0]
        if idx.numel():
            out[idx] = xd[idx] @ wd[e].t()
    return out.to(torch.bfloat16)


def permute_ref(hidden, sort_idx) -> torch.Tensor:
    """``out[i] = hidden[sort_idx[i]]`` (``kore/tasks/moe_permute_bf16/reference.py:56-59``)."""
    return hidden[sort_idx.long()]


def unpermute_ref(permuted, sort_idx) -> torch.Tensor:
    """``out[sort_idx[i]] = permuted[i]`` (``kore/tasks/breadth/moe_ext.py:567-570``)."""
    out = torch.zeros_like(permuted)
    out[sort_idx.long()] = permuted
    return out


def expert_offsets_ref(expert_ids, E: int, block: int = 1) -> torch.Tensor:
    """``offsets[E+1]`` int32: exclusive cumsum of per-expert counts rounded up to a
    multiple of ``block`` (``kore/tasks/breadth/moe_ext.py:597-621``, ``offsets`` /
    ``align_offsets``)."""
    counts = torch.bincount(expert_ids.reshape(-1).long(), minlength=E)[:E]
    padded = (counts + block - 1) // block * block
    off = torch.zeros(E + 1, dtype=torch.int64)
    off[1:] = torch.cumsum(padded, 0)
    return off.to(torch.int32)
