"""Seeded synthetic inputs for the GEMM-family configurations.

Each generator draws fp32 normals from ``torch.Generator(device).manual_seed(seed)``
and casts/quantises them exactly as the reference's ``get_inputs`` does, in the
layout the operator's entry takes.  With ``device="cpu"`` the draws are
reproducible on any machine (tests copy them to the GPU); large benchmark inputs
are drawn directly on the GPU.

Configurations:
  dense     A[M,K], B[N,K] ~ N(0,1)*0.1 bf16; entry gets b = B.t()          (C = A.B^T)
  fused     A[M,K], W[N,K] ~ N(0,1)/sqrt(K) fp16, bias[N] ~ N(0,1)*0.1; b = W.t()
  batched   A[B,M,K], B[B,K,N] ~ N(0,1)*0.1 bf16; entry gets b = B.transpose(1,2)
  fp8       X[M,K], W[N,K] ~ N(0,1) fp32, quantised 1x128 / 128x128 to e4m3
  moe       logits[T,E] ~ N(0,1) -> softmax -> top-k -> renorm; hidden ~ N(0,1) bf16;
            W_gate, W_up [I,D], W_down [D,I] ~ N(0,1)*0.02 bf16; w1 = cat(gate, up)
"""

from __future__ import annotations

from typing import Callable, NamedTuple

import torch

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0
BLK = 128


def _gen(device, seed: int) -> torch.Generator:
    return torch.Generator(device=device).manual_seed(seed)


def dense_inputs(M: int, N: int, K: int, seed: int = 0, device="cpu", dtype=torch.bfloat16,
                 scale: float = 0.1):
    g = _gen(device, seed)
    a = (torch.randn((M, K), generator=g, device=device) * scale).to(dtype)
    bt = (torch.randn((N, K), generator=g, device=device) * scale).to(dtype)
    return a, bt.t()


def backward_inputs(M: int, N: int, K: int, seed: int = 0, device="cpu", dtype=torch.bfloat16):
    """gemm_backward inputs (x[M,K], w[N,K], dy[M,N]): x, w ~ N(0,1)/sqrt(K), dy ~ N(0,1),
    as the reference draws them (kore/tasks/gemm_backward_bf16/reference.py:39-55), from
    one CPU generator here."""
    g = _gen(device, seed)
    sc = 1.0 / (K ** 0.5)
    x = (torch.randn((M, K), generator=g, device=device) * sc).to(dtype)
    w = (torch.randn((N, K), generator=g, device=device) * sc).to(dtype)
    dy = torch.randn((M, N), generator=g, device=device).to(dtype)
    return x, w, dy


def fused_inputs(M: int, N: int, K: int, seed: int = 0, device="cpu", dtype=torch.float16,
                 with_bias: bool = True):
    g = _gen(device, seed)
    sc = 1.0 / (K ** 0.5)
    a = (torch.randn((M, K), generator=g, device=device) * sc).to(dtype)
    w = (torch.randn((N, K), generator=g, device=device) * sc).to(dtype)
    bias = (torch.randn((N,), generator=g, device=device) * 0.1).to(dtype) if with_bias else None
    return a, w.t(), bias


def batched_inputs(B: int, M: int, N: int, K: int, seed: int = 0, device="cpu",
                   dtype=torch.bfloat16):
    g = _gen(device, seed)
    a = (torch.randn((B, M, K), generator=g, device=device) * 0.1).to(dtype)
    bm = (torch.randn((B, K, N), generator=g, device=device) * 0.1).to(dtype)
    return a, bm.transpose(1, 2)


def quant_1x128(x: torch.Tensor):
    """x[M,K] fp32 -> (e4m3 [M,K], fp32 scales [M,K/128]); amax/448 with a 1e-8 floor."""
    M, K = x.shape
    xb = x.float().view(M, K // BLK, BLK)
    s = xb.abs().amax(-1, keepdim=True).clamp(min=1e-8) / FP8_MAX
    q = (xb / s).clamp(-FP8_MAX, FP8_MAX).to(FP8).view(M, K)
    return q, s.squeeze(-1).to(torch.float32).contiguous()


def quant_128x128(w: torch.Tensor):
    """w[N,K] fp32 -> (e4m3 [N,K], fp32 scales [N/128,K/128])."""
    N, K = w.shape
    wb = w.float().view(N // BLK, BLK, K // BLK, BLK)
    s = wb.abs().amax(dim=(1, 3), keepdim=True).clamp(min=1e-8) / FP8_MAX
    q = (wb / s).clamp(-FP8_MAX, FP8_MAX).to(FP8).view(N, K)
    return q, s.squeeze(1).squeeze(-1).to(torch.float32).contiguous()


def fp8_inputs(M: int, N: int, K: int, seed: int = 0, device="cpu", scale: float = 1.0):
    g = _gen(device, seed)
    X = torch.randn((M, K), generator=g, device=device) * scale
    W = torch.randn((N, K), generator=g, device=device) * scale
    xq, xs = quant_1x128(X)
    wq, ws = quant_128x128(W)
    return xq, wq, xs, ws


def _q8_rowwise(x: torch.Tensor, kind: str):
    """Per-row symmetric quantisation (fp8 e4m3 max 448 / int8 max 127); scale [R,1]."""
    qmax = 448.0 if kind == "fp8" else 127.0
    s = (x.float().abs().amax(dim=-1, keepdim=True).clamp(min=1e-12) / qmax).to(torch.float32)
    if kind == "fp8":
        return (x.float() / s).clamp(-qmax, qmax).to(FP8), s
    return (x.float() / s).round().clamp(-qmax, qmax).to(torch.int8), s


def a8w8_inputs(M: int, N: int, K: int, kind: str = "fp8", mode: str = "pertoken", seed: int = 0,
                device="cpu", transpose_a: bool = False):
    """(xq[M,K], wq[N,K], x_scale[M,1], w_scale[1,N]) of the a8w8 tasks: X, W ~ N(0,1);
    ``pertoken`` quantises X per row and W per output channel, ``pertensor`` uses one
    scale per tensor broadcast to those shapes.  ``transpose_a`` returns xq as a
    non-contiguous [M,K] view of a [K,M] buffer (the per-token task's TA case)."""
    g = _gen(device, seed)
    X = torch.randn((K, M) if transpose_a else (M, K), generator=g, device=device)
    W = torch.randn((N, K), generator=g, device=device)
    if mode == "pertensor":
        qmax = 448.0 if kind == "fp8" else 127.0
        sx = (X.abs().max().clamp(min=1e-12) / qmax).to(torch.float32)
        sw = (W.abs().max().clamp(min=1e-12) / qmax).to(torch.float32)
        xq = (X / sx).clamp(-qmax, qmax)
        wq = (W / sw).clamp(-qmax, qmax)
        xq = xq.to(FP8) if kind == "fp8" else xq.round().to(torch.int8)
        wq = wq.to(FP8) if kind == "fp8" else wq.round().to(torch.int8)
        if transpose_a:
            xq = xq.t()
        return xq, wq, sx.reshape(1, 1).repeat(M, 1).contiguous(), sw.reshape(1, 1).repeat(1, N).contiguous()
    if transpose_a:
        xq_t, xs_t = _q8_rowwise(X.t().contiguous(), kind)
        xq = xq_t.t().contiguous().t()  # [M,K] view of a [K,M] buffer
        xs = xs_t
    else:
        xq, xs = _q8_rowwise(X, kind)
    wq, ws = _q8_rowwise(W, kind)
    return xq, wq, xs, ws.reshape(1, N).contiguous()


def route(logits: torch.Tensor, topk: int, renorm: bool = True):
    probs = torch.softmax(logits.float(), dim=-1)
    tw, ti = torch.topk(probs, topk, dim=-1)
    if renorm:
        tw = tw / tw.sum(dim=-1, keepdim=True)
    return tw.to(torch.float32), ti.to(torch.int32)


def moe_inputs(T: int, E: int, topk: int, D: int, I: int, seed: int = 0, device="cpu",
               wscale: float = 0.02, router_bias: torch.Tensor | None = None):
    """Returns (hidden[T,D], w1[E,2I,D], w2[E,D,I], topk_weight[T,topk], topk_ids[T,topk])."""
    g = _gen(device, seed)
    hidden = torch.randn((T, D), generator=g, device=device).to(torch.bfloat16)
    w1 = torch.empty((E, 2 * I, D), dtype=torch.bfloat16, device=device)
    w2 = torch.empty((E, D, I), dtype=torch.bfloat16, device=device)
    for e in range(E):  # per expert keeps the fp32 temporaries small
        w1[e, :I] = (torch.randn((I, D), generator=g, device=device) * wscale).to(torch.bfloat16)
        w1[e, I:] = (torch.randn((I, D), generator=g, device=device) * wscale).to(torch.bfloat16)
        w2[e] = (torch.randn((D, I), generator=g, device=device) * wscale).to(torch.bfloat16)
    logits = torch.randn((T, E), generator=g, device=device)
    if router_bias is not None:
        logits = logits + router_bias.to(device)
    tw, ti = route(logits, topk)
    return hidden, w1, w2, tw, ti


# --------------------------------------------------------------------------- #
# Benchmark workloads: one entry per BASELINE configuration (inputs drawn on the
# device so they are resident in HBM before timing starts).
# --------------------------------------------------------------------------- #
# Per-expert token-count trace of the reference's MoE tasks (``kore/tasks/
# _moe_common.py:93-113``): unbalanced, the last expert dead; tiled past 32 experts.
ROUTER_TRACE = (16053, 105, 1843, 2724, 327, 88, 4102, 51, 9210, 61, 3020, 44, 1502, 990, 233, 77,
                6740, 120, 410, 58, 2210, 39, 812, 175, 5030, 66, 1360, 92, 3550, 47, 1180, 0)


def jagged_bias(E: int) -> torch.Tensor:
    """Router bias ``log(count)`` over ``ROUTER_TRACE`` (``-inf`` on the dead last
    expert), added to N(0,1) logits to make the reference's unbalanced routing."""
    live = [c for c in ROUTER_TRACE if c > 0]
    counts = list(ROUTER_TRACE[:E]) if E <= len(ROUTER_TRACE) else [live[i % len(live)] for i in range(E)]
    counts[-1] = 0
    c = torch.tensor(counts, dtype=torch.float32)
    bias = torch.log(c + 1e-6)
    bias[c == 0] = float("-inf")
    return bias


def grouped_inputs(M: int, E: int, N: int, K: int, seed: int = 0, device="cpu",
                   router_bias: torch.Tensor | None = None):
    """(hidden[M,K] bf16, w[E,N,K] bf16, expert_ids[M] int32) of the top-1 grouped GEMM
    task: hidden, w ~ N(0,1)/sqrt(K); ids = argmax of softmax(N(0,1) logits + bias)."""
    g = _gen(device, seed)
    sc = 1.0 / K ** 0.5
    hidden = (torch.randn((M, K), generator=g, device=device) * sc).to(torch.bfloat16)
    w = (torch.randn((E, N, K), generator=g, device=device) * sc).to(torch.bfloat16)
    logits = torch.randn((M, E), generator=g, device=device)
    if router_bias is not None:
        logits = logits + router_bias.to(device)
    _, ti = route(logits, 1, renorm=False)
    return hidden, w, ti[:, 0].contiguous()


def grouped_fp8_inputs(M: int, E: int, N: int, K: int, seed: int = 0, device="cpu",
                       router_bias: torch.Tensor | None = None):
    """(xq[M,K], wq[E,N,K] e4m3, x_scale[M,1], w_scale[E,N,1] fp32, expert_ids[M] int32)
    of the fp8 grouped GEMM task: x ~ N(0,1), w ~ N(0,1)/sqrt(K), each quantised per
    last-dim row (``scale = max(amax, 1e-12)/448``)."""
    g = _gen(device, seed)
    xf = torch.randn((M, K), generator=g, device=device)
    wq = torch.empty((E, N, K), dtype=torch.float8_e4m3fn, device=device)
    ws = torch.empty((E, N, 1), dtype=torch.float32, device=device)
    for e in range(E):  # per expert keeps the fp32 temporaries small
        wq[e], ws[e] = _q8_rowwise(torch.randn((N, K), generator=g, device=device) / K ** 0.5, "fp8")
    xq, xs = _q8_rowwise(xf, "fp8")
    logits = torch.randn((M, E), generator=g, device=device)
    if router_bias is not None:
        logits = logits + router_bias.to(device)
    _, ti = route(logits, 1, renorm=False)
    return xq, wq, xs, ws, ti[:, 0].contiguous()


class Workload(NamedTuple):
    """One benchmark step: ``fn()`` runs the operator once on ``args`` (its device
    inputs); ``(op, dims, dtype)`` key the roofline model (``kore_amd.roofline``)."""
    fn: Callable[[], object]
    op: str
    dims: dict
    dtype: str
    args: tuple


def bench_workloads():
    """Ordered ``name -> builder(device)``; a builder returns a :class:`Workload`."""
    import kore_amd  # deferred: the package imports this module

    def fp8(M):
        def build(dev):
            xq, wq, xs, ws = fp8_inputs(M, 7168, 4096, seed=0, device=dev)
            return Workload(lambda: kore_amd.gemm_a8w8_blockscale(xq, wq, xs, ws), "gemm_fp8",
                            {"M": M, "N": 7168, "K": 4096}, "fp8", (xq, wq, xs, ws))
        return build

    def dense(n):
        def build(dev):
            a, b = dense_inputs(n, n, n, seed=0, device=dev)
            return Workload(lambda: kore_amd.gemm(a, b), "gemm", {"M": n, "N": n, "K": n}, "bf16",
                            (a, b, None, "none"))
        return build

    def dense_kn(n):
        # the gemm_bf16 task's own operands: b is a contiguous [K, N] tensor
        # (kore/tasks/gemm_bf16/reference.py:28-36)
        def build(dev):
            g = _gen(dev, 0)
            a = (torch.randn((n, n), generator=g, device=dev) / n ** 0.5).to(torch.bfloat16)
            b = torch.randn((n, n), generator=g, device=dev).to(torch.bfloat16)
            return Workload(lambda: kore_amd.gemm(a, b), "gemm", {"M": n, "N": n, "K": n}, "bf16",
                            (a, b, None, "none"))
        return build

    def fused(act):
        def build(dev):
            a, b, bias = fused_inputs(4096, 4096, 4096, seed=0, device=dev)
            return Workload(lambda: kore_amd.gemm_fused(a, b, bias, act), "gemm",
                            {"M": 4096, "N": 4096, "K": 4096}, "fp16", (a, b, bias, act))
        return build

    def batched(dev):
        a, b = batched_inputs(64, 1024, 1024, 128, seed=0, device=dev)
        return Workload(lambda: kore_amd.batched_gemm(a, b), "batched_gemm",
                        {"B": 64, "M": 1024, "N": 1024, "K": 128}, "bf16", (a, b))

    def moe(T):
        def build(dev):
            args = moe_inputs(T, 8, 2, 4096, 14336, seed=0, device=dev)
            return Workload(lambda: kore_amd.fused_moe(*args), "fused_moe",
                            {"M": T, "E": 8, "topk": 2, "D": 4096, "I": 14336}, "bf16", tuple(args))
        return build

    w = {"fp8_blockscale_2048x7168x4096": fp8(2048),
         "bf16_gemm_4096": dense(4096),
         "bf16_gemm_1024": dense(1024),
         "bf16_gemm_4096_kn": dense_kn(4096)}
    for act in ("gelu", "relu", "silu"):
        w[f"fp16_gemm_bias_{act}_4096"] = fused(act)
    w["bf16_batched_64x1024x1024x128"] = batched

    def backward(M, N, K):
        def build(dev):
            x, wt, dy = backward_inputs(M, N, K, seed=0, device=dev)
            return Workload(lambda: kore_amd.gemm_backward(x, wt, dy), "gemm_backward", {"M": M, "N": N, "K": K},
                            "bf16", (x, wt, dy))
        return build

    # gemm_backward_bf16 primary shape (task.yaml): dX = dY.W and dW = dY^T.X
    w["bf16_gemm_backward_8192x4096x4096"] = backward(8192, 4096, 4096)

    def fp32_bias(M, N, K):
        def build(dev):
            g = _gen(dev, 0)
            a = torch.randn((M, K), generator=g, device=dev) / K ** 0.5
            b = torch.randn((K, N), generator=g, device=dev) / K ** 0.5
            bias = torch.randn((N,), generator=g, device=dev)
            return Workload(lambda: kore_amd.gemm_bias(a, b, bias), "gemm", {"M": M, "N": N, "K": K}, "fp32",
                            (a, b, bias, "none"))
        return build

    def task_kn(M, N, K, dtype, op):
        # a gemm_bf16 / gen_gemm_* task's own operands: a, b[K,N] ~ N(0,1)/sqrt(K) with
        # b contiguous (kore/tasks/_genops.py:434-443), bias ~ N(0,1)
        def build(dev):
            g = _gen(dev, 0)
            has_bias, act = kore_amd.GEMM_FUSION_OPS.get(op, (False, "none"))
            a = (torch.randn((M, K), generator=g, device=dev) / K ** 0.5).to(dtype)
            b = (torch.randn((K, N), generator=g, device=dev) / K ** 0.5).to(dtype)
            bias = torch.randn((N,), generator=g, device=dev).to(dtype) if has_bias else None
            return Workload(lambda: kore_amd.gemm_fused(a, b, bias, act), "gemm", {"M": M, "N": N, "K": K},
                            "bf16" if dtype == torch.bfloat16 else "fp16", (a, b, bias, act))
        return build

    # the gen_gemm_* primary (deep ring), its K-tail validation shape (packed path) and
    # gemm_bf16's decode validation shape (split-K), all with the tasks' [K,N] B
    w["fp16_gemm_bias_gelu_512x4096x4096_kn"] = task_kn(512, 4096, 4096, torch.float16, "gemm_bias_gelu")
    w["bf16_gemm_bias_gelu_512x4096x4095_kn"] = task_kn(512, 4096, 4095, torch.bfloat16, "gemm_bias_gelu")
    w["bf16_gemm_1x4096x4096_kn"] = task_kn(1, 4096, 4096, torch.bfloat16, "gemm")

    # fp32 epilogue GEMM on the fp32 matrix cores (gen_gemm_bias_fp32 primary)
    w["fp32_gemm_bias_512x4096x4096"] = fp32_bias(512, 4096, 4096)
    for M in (512, 128, 16):
        w[f"fp8_blockscale_{M}x7168x4096"] = fp8(M)
    def a8w8(M, N, K, kind):
        def build(dev):
            xq, wq, xs, ws = a8w8_inputs(M, N, K, kind, "pertoken", seed=0, device=dev)
            return Workload(lambda: kore_amd.gemm_a8w8(xq, wq, xs, ws), "gemm_a8w8",
                            {"M": M, "N": N, "K": K}, kind, (xq, wq, xs, ws))
        return build

    # a8w8 with per-token / per-channel scales (task primaries + decode)
    w["fp8_a8w8_pertoken_4096"] = a8w8(4096, 4096, 4096, "fp8")
    w["int8_a8w8_4096"] = a8w8(4096, 4096, 4096, "int8")
    w["fp8_a8w8_pertoken_16x4096x4096"] = a8w8(16, 4096, 4096, "fp8")
    w["moe_decode_T64"] = moe(64)
    w["moe_prefill_T4096"] = moe(4096)

    def moe_task(T, E, topk, D, I):
        # the fused_moe_silu_bf16 task's primary shape and inputs (weights ~ N(0,1) * 0.05)
        def build(dev):
            args = moe_inputs(T, E, topk, D, I, seed=0, device=dev, wscale=0.05)
            return Workload(lambda: kore_amd.fused_moe(*args), "fused_moe",
                            {"M": T, "E": E, "topk": topk, "D": D, "I": I}, "bf16", tuple(args))
        return build

    w["fused_moe_M256_E32_top8_D1024_I768"] = moe_task(256, 32, 8, 1024, 768)

    def grouped(M, E, N, K):
        def build(dev):
            hidden, wt, ids = grouped_inputs(M, E, N, K, seed=0, device=dev, router_bias=jagged_bias(E))
            used = int(torch.unique(ids).numel())
            return Workload(lambda: kore_amd.grouped_gemm(hidden, wt, ids), "moe_grouped_gemm",
                            {"M": M, "E": E, "N": N, "K": K, "E_used": used}, "bf16", (hidden, wt, ids))
        return build

    def permute(M, E, D):
        def build(dev):
            g = _gen(dev, 0)
            hidden = torch.randn((M, D), generator=g, device=dev).to(torch.bfloat16)
            _, _, ids = grouped_inputs(M, E, 128, 8, seed=1, device=dev, router_bias=jagged_bias(E))
            sidx = torch.argsort(ids, stable=True).to(torch.int32)
            return Workload(lambda: kore_amd.moe_permute(hidden, sidx), "moe_permute", {"M": M, "D": D}, "bf16",
                            (hidden, sidx))
        return build

    # expert-dispatch stages: top-1 grouped GEMM and the token permute (task primaries)
    w["moe_grouped_gemm_4096x32x2048x4096"] = grouped(4096, 32, 2048, 4096)
    w["moe_permute_8192x7168"] = permute(8192, 256, 7168)

    def grouped_fp8(M, E, N, K):
        def build(dev):
            xq, wq, xs, ws, ids = grouped_fp8_inputs(M, E, N, K, seed=0, device=dev, router_bias=jagged_bias(E))
            used = int(torch.unique(ids).numel())
            return Workload(lambda: kore_amd.grouped_gemm_fp8(xq, wq, xs, ws, ids), "moe_grouped_gemm",
                            {"M": M, "E": E, "N": N, "K": K, "E_used": used}, "fp8", (xq, wq, xs, ws, ids))
        return build

    w["moe_grouped_gemm_fp8_4096x32x2048x4096"] = grouped_fp8(4096, 32, 2048, 4096)
    return w
