"""Host-side operators with the KORE task suite's entry signatures.

Each function validates its tensors, allocates the output with torch (the caching
allocator owns it), and launches the gfx950 kernels of ``libkore_amd.so`` through
the C ABI on torch's current HIP stream.  There is no non-HIP fallback: a missing
library raises, and unsupported shapes raise ``ValueError`` /
``NotImplementedError`` (the reference drivers turn a raised exception into a
failing verdict, ``kore/tasks/gemm_bf16/driver.py:115-118``).

Entry points and the reference callables they replace:

=========================  =======================================================
``gemm(a, b)``             ``kore/tasks/gemm_bf16/seed_triton.py:64-86``
``gemm_<act>(a, b)``,      ``kore/tasks/_genops.py:715-731`` (``_GEMM_TMPL``;
``gemm_bias_<act>(a,b,c)``  op list ``_genops.py:274-290``)
``batched_gemm(a, b)``     ``kore/tasks/vendor_ops.py:914-920``
``gemm_a8w8_blockscale``   ``kore/tasks/gemm_fp8_a8w8_blockscale/seed_triton.py:49-60``
(task entry name ``gemm``)
``gemm_a8w8``              ``kore/tasks/gemm_{fp8_a8w8,fp8_a8w8_pertoken,fp8_a8w8_pertensor,
                           int8_a8w8}/seed_triton.py``; ``kore/tasks/vendor_ops.py:697-760``
``fused_moe(...)``         ``kore/tasks/fused_moe_silu_bf16/seed_triton.py:69-86``
``moe_align(ids, E, blk)`` sort/align stage (``kore/tasks/breadth/moe_ext.py:617-621``)
``grouped_gemm``           ``kore/tasks/moe_grouped_gemm_bf16/seed_triton.py``; breadth ``moe_grouped_gemm``
``moe_permute``            ``kore/tasks/moe_permute_bf16/seed_triton.py``; breadth ``moe_permute`` /
``moe_unpermute``          ``moe_unpermute`` (``kore/tasks/breadth/moe_ext.py:546-571``)
``moe_align_block_offsets`` breadth ``moe_align_block_offsets`` / ``moe_expert_offsets``
=========================  =======================================================
"""

from __future__ import annotations

import torch

from . import _lib

DT_CODE = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
ACT_CODE = {"none": 0, "relu": 1, "gelu": 2, "silu": 3, "tanh": 4, "sigmoid": 5}
FP8_DTYPE = torch.float8_e4m3fn  # OCP e4m3 on gfx950 (kore/tasks/aiter_ref.py:37-62)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _workspace(nbytes: int, device: torch.device):
    """Device scratch of one call (a uint8 tensor, or None when the path needs none),
    owned by torch's caching allocator -- under graph capture by the graph's private
    pool.  The caller keeps it alive until the launch is enqueued."""
    if nbytes == 0:
        return None
    return torch.empty((nbytes,), dtype=torch.uint8, device=device)


def _ws_args(ws):
    return (None, 0) if ws is None else (ws.data_ptr(), ws.numel())


def _require_cuda(*ts: torch.Tensor) -> None:
    dev = None
    for t in ts:
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"expected a torch.Tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise ValueError(f"kore_amd operators need HIP device tensors (got {t.device})")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")


# --------------------------------------------------------------------------- #
# Dense GEMM + fused epilogue
# --------------------------------------------------------------------------- #
def gemm_fused(a: torch.Tensor, b: torch.Tensor, bias: torch.Tensor | None = None,
               act: str = "none") -> torch.Tensor:
    """``act(a @ b + bias)`` in ``a.dtype`` (bf16 / fp16 / fp32), fp32 accumulate.

    a[M,K], b[K,N] with any strides (``b = W.t()`` views and N-contiguous ``b`` are the
    fast paths), bias[N].  fp32 runs on the fp32 matrix cores (full fp32 products).
    """
    _require_cuda(a, b)
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError(f"gemm expects 2-D operands, got {tuple(a.shape)} and {tuple(b.shape)}")
    if a.shape[1] != b.shape[0]:
        raise ValueError(f"incompatible dims: a {tuple(a.shape)} @ b {tuple(b.shape)}")
    if a.dtype not in DT_CODE or b.dtype != a.dtype:
        raise ValueError(f"gemm supports bf16/fp16/fp32 operands of one dtype (got {a.dtype}, {b.dtype})")
    if act not in ACT_CODE:
        raise ValueError(f"unknown activation {act!r}")
    M, K = a.shape
    N = b.shape[1]
    if bias is not None:
        _require_cuda(bias)
        if bias.shape != (N,) or bias.dtype != a.dtype:
            raise ValueError(f"bias must be [{N}] {a.dtype} (got {tuple(bias.shape)} {bias.dtype})")
        bias = bias.contiguous()
    c = torch.empty((M, N), dtype=a.dtype, device=a.device)
    if M == 0 or N == 0:
        return c
    lib = _lib.load()
    args = (DT_CODE[a.dtype], ACT_CODE[act], a.data_ptr(), a.stride(0), a.stride(1),
            b.data_ptr(), b.stride(0), b.stride(1), bias.data_ptr() if bias is not None else None,
            c.data_ptr(), c.stride(0), M, N, K)
    ws = _workspace(lib.kore_gemm_workspace_bytes(*args), a.device)
    _lib.check(lib.kore_gemm(*args, *_ws_args(ws), _stream(a)))
    return c


def gemm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Dense bf16 GEMM ``C = A @ B`` (the ``gemm_bf16`` task entry)."""
    if a.dtype != torch.bfloat16 or b.dtype != torch.bfloat16:
        raise ValueError(f"gemm (gemm_bf16 task) takes bf16 operands (got {a.dtype}, {b.dtype})")
    return gemm_fused(a, b, None, "none")


def _make_fusion_entry(name: str, has_bias: bool, act: str):
    if has_bias:
        def entry(a, b, bias):
            return gemm_fused(a, b, bias, act)
    else:
        def entry(a, b):
            return gemm_fused(a, b, None, act)
    entry.__name__ = name
    entry.__qualname__ = name
    entry.__doc__ = (f"``{name}``: {act}(a @ b{' + bias' if has_bias else ''}) in a.dtype "
                     "(gemm_fusion op, kore/tasks/_genops.py:274-290).")
    return entry


# gemm_fusion op registry (kore/tasks/_genops.py:274-290): name -> (has_bias, act)
GEMM_FUSION_OPS = {
    "gemm_bias": (True, "none"),
    "gemm_relu": (False, "relu"),
    "gemm_gelu": (False, "gelu"),
    "gemm_silu": (False, "silu"),
    "gemm_bias_relu": (True, "relu"),
    "gemm_bias_gelu": (True, "gelu"),
    "gemm_bias_silu": (True, "silu"),
    "gemm_tanh": (False, "tanh"),
    "gemm_sigmoid": (False, "sigmoid"),
    "gemm_bias_tanh": (True, "tanh"),
    "gemm_bias_sigmoid": (True, "sigmoid"),
}

for _name, (_hb, _act) in GEMM_FUSION_OPS.items():
    globals()[_name] = _make_fusion_entry(_name, _hb, _act)


# --------------------------------------------------------------------------- #
# Batched GEMM
# --------------------------------------------------------------------------- #
def batched_gemm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``C[i] = A[i] @ B[i]^T``; a[B,M,K], b[B,N,K] (any strides) -> [B,M,N] a.dtype."""
    _require_cuda(a, b)
    if a.dim() != 3 or b.dim() != 3 or a.shape[0] != b.shape[0] or a.shape[2] != b.shape[2]:
        raise ValueError(f"batched_gemm expects a[B,M,K], b[B,N,K] (got {tuple(a.shape)}, {tuple(b.shape)})")
    if a.dtype not in (torch.bfloat16, torch.float16) or b.dtype != a.dtype:
        raise ValueError(f"batched_gemm supports bf16/fp16 (got {a.dtype}, {b.dtype})")
    Bn, M, K = a.shape
    N = b.shape[1]
    c = torch.empty((Bn, M, N), dtype=a.dtype, device=a.device)
    if Bn == 0 or M == 0 or N == 0:
        return c
    lib = _lib.load()
    args = (DT_CODE[a.dtype], a.data_ptr(), a.stride(0), a.stride(1), a.stride(2),
            b.data_ptr(), b.stride(0), b.stride(1), b.stride(2),
            c.data_ptr(), c.stride(0), c.stride(1), Bn, M, N, K)
    ws = _workspace(lib.kore_batched_gemm_workspace_bytes(*args), a.device)
    _lib.check(lib.kore_batched_gemm(*args, *_ws_args(ws), _stream(a)))
    return c


# --------------------------------------------------------------------------- #
# GEMM backward (linear layer Y = X @ W^T)
# --------------------------------------------------------------------------- #
def gemm_backward(x: torch.Tensor, w: torch.Tensor, dy: torch.Tensor):
    """``(dx, dw) = (dy @ w, dy^T @ x)`` in ``x.dtype`` (bf16/fp16), fp32 accumulate.

    x[M,K], w[N,K], dy[M,N] with unit stride along rows (the task's layouts); the
    entry of ``kore/tasks/gemm_backward_bf16`` (``gemm_backward(x, w, dy)``).
    """
    _require_cuda(x, w, dy)
    if x.dim() != 2 or w.dim() != 2 or dy.dim() != 2:
        raise ValueError("gemm_backward expects 2-D x[M,K], w[N,K], dy[M,N]")
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K or tuple(dy.shape) != (M, N):
        raise ValueError(f"incompatible shapes x{tuple(x.shape)} w{tuple(w.shape)} dy{tuple(dy.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float16) or w.dtype != x.dtype or dy.dtype != x.dtype:
        raise ValueError(f"gemm_backward takes bf16/fp16 tensors of one dtype (got {x.dtype}, {w.dtype}, {dy.dtype})")
    x, w, dy = (t if t.stride(1) == 1 else t.contiguous() for t in (x, w, dy))
    dx = torch.empty((M, K), dtype=x.dtype, device=x.device)
    dw = torch.empty((N, K), dtype=x.dtype, device=x.device)
    if M == 0 or N == 0 or K == 0:
        return dx.zero_(), dw.zero_()
    lib = _lib.load()
    args = (DT_CODE[x.dtype], x.data_ptr(), x.stride(0), w.data_ptr(), w.stride(0),
            dy.data_ptr(), dy.stride(0), dx.data_ptr(), dx.stride(0), dw.data_ptr(), dw.stride(0), M, N, K)
    ws = _workspace(lib.kore_gemm_backward_workspace_bytes(*args), x.device)
    _lib.check(lib.kore_gemm_backward(*args, *_ws_args(ws), _stream(x)))
    return dx, dw


# --------------------------------------------------------------------------- #
# fp8 a8w8 block-scaled GEMM
# --------------------------------------------------------------------------- #
def gemm_a8w8_blockscale(xq: torch.Tensor, wq: torch.Tensor, x_scale: torch.Tensor,
                         w_scale: torch.Tensor) -> torch.Tensor:
    """Block-scaled fp8 GEMM -> bf16 [M,N].

    xq[M,K] e4m3, wq[N,K] e4m3 (row-contiguous), x_scale[M,K/128] fp32,
    w_scale[N/128,K/128] fp32.  K and N must be multiples of 128.
    """
    _require_cuda(xq, wq, x_scale, w_scale)
    if xq.dtype != FP8_DTYPE or wq.dtype != FP8_DTYPE:
        raise ValueError(f"xq/wq must be {FP8_DTYPE} (got {xq.dtype}, {wq.dtype})")
    if x_scale.dtype != torch.float32 or w_scale.dtype != torch.float32:
        raise ValueError("scales must be fp32")
    if xq.dim() != 2 or wq.dim() != 2 or xq.shape[1] != wq.shape[1]:
        raise ValueError(f"expected xq[M,K], wq[N,K] (got {tuple(xq.shape)}, {tuple(wq.shape)})")
    M, K = xq.shape
    N = wq.shape[0]
    if K % 128 or N % 128:
        raise ValueError(f"block-scale needs K % 128 == 0 and N % 128 == 0 (got N={N}, K={K})")
    if tuple(x_scale.shape) != (M, K // 128) or tuple(w_scale.shape) != (N // 128, K // 128):
        raise ValueError(f"scale shapes must be [{M},{K // 128}] and [{N // 128},{K // 128}] "
                         f"(got {tuple(x_scale.shape)}, {tuple(w_scale.shape)})")
    if xq.stride(1) != 1 or wq.stride(1) != 1:
        xq, wq = xq.contiguous(), wq.contiguous()
    y = torch.empty((M, N), dtype=torch.bfloat16, device=xq.device)
    if M == 0:
        return y
    lib = _lib.load()
    rc = lib.kore_gemm_a8w8_blockscale(xq.data_ptr(), xq.stride(0), wq.data_ptr(), wq.stride(0),
                                       x_scale.data_ptr(), x_scale.stride(0), x_scale.stride(1),
                                       w_scale.data_ptr(), w_scale.stride(0), w_scale.stride(1),
                                       y.data_ptr(), y.stride(0), M, N, K, _stream(xq))
    _lib.check(rc)
    return y


# --------------------------------------------------------------------------- #
# a8w8 GEMM with per-row / per-column scales (fp8 e4m3 or int8)
# --------------------------------------------------------------------------- #
Q_CODE = {FP8_DTYPE: 0, torch.int8: 1}


def _scale_vector(s: torch.Tensor, n: int, what: str) -> tuple[torch.Tensor, int]:
    """A [n,1] / [1,n] / [n] fp32 scale as (tensor, element stride along n)."""
    if s.dtype != torch.float32:
        raise ValueError(f"{what} must be fp32 (got {s.dtype})")
    if s.numel() != n or not (s.dim() == 1 or (s.dim() == 2 and 1 in s.shape)):
        raise ValueError(f"{what} must hold {n} values as [{n},1], [1,{n}] or [{n}] (got {tuple(s.shape)})")
    along_dim0 = s.dim() == 1 or s.shape[0] == n
    return s, s.stride(0) if along_dim0 else s.stride(1)


def gemm_a8w8(xq: torch.Tensor, wq: torch.Tensor, x_scale: torch.Tensor,
              w_scale: torch.Tensor) -> torch.Tensor:
    """8-bit a8w8 GEMM -> bf16 [M,N]: ``(xq * x_scale) @ (wq * w_scale)^T``.

    xq[M,K], wq[N,K] both ``float8_e4m3fn`` or both ``int8`` (any strides),
    x_scale [M,1] (per token; per tensor = equal entries), w_scale [1,N] / [N,1] / [N]
    (per output channel), fp32.  Each scale is applied once to the fp32 (int8: exact
    int32) accumulator.
    """
    _require_cuda(xq, wq, x_scale, w_scale)
    if xq.dtype not in Q_CODE or wq.dtype != xq.dtype:
        raise ValueError(f"xq/wq must both be float8_e4m3fn or both int8 (got {xq.dtype}, {wq.dtype})")
    if xq.dim() != 2 or wq.dim() != 2 or xq.shape[1] != wq.shape[1]:
        raise ValueError(f"expected xq[M,K], wq[N,K] (got {tuple(xq.shape)}, {tuple(wq.shape)})")
    M, K = xq.shape
    N = wq.shape[0]
    xs, xs_st = _scale_vector(x_scale, M, "x_scale")
    ws, ws_st = _scale_vector(w_scale, N, "w_scale")
    y = torch.empty((M, N), dtype=torch.bfloat16, device=xq.device)
    if M == 0 or N == 0:
        return y
    if K == 0:
        return y.zero_()
    lib = _lib.load()
    rc = lib.kore_gemm_a8w8(Q_CODE[xq.dtype], xq.data_ptr(), xq.stride(0), xq.stride(1), wq.data_ptr(),
                            wq.stride(0), wq.stride(1), xs.data_ptr(), xs_st, ws.data_ptr(), ws_st,
                            y.data_ptr(), y.stride(0), M, N, K, _stream(xq))
    _lib.check(rc)
    return y


# --------------------------------------------------------------------------- #
# MoE
# --------------------------------------------------------------------------- #
def moe_align(topk_ids: torch.Tensor, num_experts: int, block: int):
    """Sort/align: returns ``(offsets[E+1], sorted_slots[cap], block_expert[cap/block])``.

    Slots ``s = t*topk + k`` grouped by expert (ascending), stable, each expert padded
    to a multiple of ``block`` with the sentinel ``T*topk``; ``offsets`` is the
    exclusive cumsum of the padded counts.  int32 tensors on the ids' device.
    """
    _require_cuda(topk_ids)
    if topk_ids.dim() != 2 or topk_ids.dtype != torch.int32:
        raise ValueError("topk_ids must be int32 [T, topk]")
    ids = topk_ids.contiguous()
    T, topk = ids.shape
    lib = _lib.load()
    cap = lib.kore_moe_align_capacity(T, topk, num_experts, block)
    if cap < 0:
        raise ValueError("bad moe_align sizes")
    dev = ids.device
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    sorted_slots = torch.empty(max(cap, 1), dtype=torch.int32, device=dev)
    block_expert = torch.empty(max(cap // block, 1), dtype=torch.int32, device=dev)
    rc = lib.kore_moe_align(ids.data_ptr(), T, topk, num_experts, block, offsets.data_ptr(),
                            sorted_slots.data_ptr(), block_expert.data_ptr(), cap, _stream(ids))
    _lib.check(rc)
    return offsets, sorted_slots[:cap], block_expert[:cap // block]


def fused_moe(hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
              topk_weight: torch.Tensor, topk_ids: torch.Tensor) -> torch.Tensor:
    """Top-k fused MoE (SiLU gated MLP) -> bf16 [T, D].

    hidden[T,D] bf16, w1[E,2I,D] bf16 (gate rows then up rows), w2[E,D,I] bf16,
    topk_weight[T,topk] fp32, topk_ids[T,topk] int32.
    """
    _require_cuda(hidden_states, w1, w2, topk_weight, topk_ids)
    if hidden_states.dtype != torch.bfloat16 or w1.dtype != torch.bfloat16 or w2.dtype != torch.bfloat16:
        raise ValueError("fused_moe takes bf16 hidden/w1/w2")
    if hidden_states.dim() != 2 or w1.dim() != 3 or w2.dim() != 3:
        raise ValueError("expected hidden[T,D], w1[E,2I,D], w2[E,D,I]")
    T, D = hidden_states.shape
    E, twoI, D1 = w1.shape
    I = twoI // 2
    if D1 != D or twoI != 2 * I or tuple(w2.shape) != (E, D, I):
        raise ValueError(f"shape mismatch: hidden {tuple(hidden_states.shape)}, w1 {tuple(w1.shape)}, "
                         f"w2 {tuple(w2.shape)}")
    if topk_ids.dim() != 2 or topk_ids.shape[0] != T or topk_weight.shape != topk_ids.shape:
        raise ValueError("topk_weight/topk_ids must both be [T, topk]")
    topk = topk_ids.shape[1]
    tw = topk_weight.to(torch.float32).contiguous()
    ti = topk_ids.to(torch.int32).contiguous()
    x = hidden_states if hidden_states.stride(1) == 1 else hidden_states.contiguous()
    w1c, w2c = w1.contiguous(), w2.contiguous()
    out = torch.empty((T, D), dtype=torch.bfloat16, device=x.device)
    if T == 0 or topk == 0:
        return out.zero_()
    lib = _lib.load()
    nbytes = lib.kore_fused_moe_workspace_bytes(T, topk, E, D, I)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    rc = lib.kore_fused_moe(x.data_ptr(), x.stride(0), w1c.data_ptr(), w2c.data_ptr(), tw.data_ptr(),
                            ti.data_ptr(), out.data_ptr(), T, D, I, E, topk, ws.data_ptr(), nbytes,
                            _stream(x))
    _lib.check(rc)
    return out


def grouped_gemm(hidden: torch.Tensor, w: torch.Tensor, expert_ids: torch.Tensor) -> torch.Tensor:
    """Top-1 grouped expert GEMM -> bf16 [M,N]: ``out[m] = hidden[m] @ w[expert_ids[m]]^T``.

    hidden[M,K] bf16, w[E,N,K] bf16, expert_ids[M] int; output rows in token order.
    Rows whose id is outside [0, E) are zero.  The kernels need N % 128 == 0 and
    K % 8 == 0; other shapes are zero-padded here first (a copy of ``w``).
    """
    _require_cuda(hidden, w, expert_ids)
    if hidden.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise NotImplementedError(f"grouped_gemm runs bf16 operands (got {hidden.dtype}, {w.dtype})")
    if hidden.dim() != 2 or w.dim() != 3 or w.shape[2] != hidden.shape[1]:
        raise ValueError(f"expected hidden[M,K], w[E,N,K] (got {tuple(hidden.shape)}, {tuple(w.shape)})")
    M, K = hidden.shape
    E, N, _ = w.shape
    if expert_ids.numel() != M:
        raise ValueError(f"expert_ids must hold {M} ids (got {tuple(expert_ids.shape)})")
    ids = expert_ids.reshape(M).to(torch.int32).contiguous()
    if M == 0 or N == 0:
        return torch.zeros((M, N), dtype=torch.bfloat16, device=hidden.device)
    Kp, Np = -(-K // 8) * 8, -(-N // 128) * 128
    if Kp != K or Np != N:
        xp = torch.zeros((M, Kp), dtype=torch.bfloat16, device=hidden.device)
        xp[:, :K] = hidden
        wp = torch.zeros((E, Np, Kp), dtype=torch.bfloat16, device=w.device)
        wp[:, :N, :K] = w
        return grouped_gemm(xp, wp, ids)[:, :N].contiguous()
    x = hidden if hidden.stride(1) == 1 and hidden.stride(0) % 8 == 0 else hidden.contiguous()
    wc = w.contiguous()
    out = torch.zeros((M, N), dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    nbytes = lib.kore_moe_grouped_gemm_workspace_bytes(M, E)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    rc = lib.kore_moe_grouped_gemm(x.data_ptr(), x.stride(0), wc.data_ptr(), ids.data_ptr(), out.data_ptr(),
                                   out.stride(0), M, N, K, E, ws.data_ptr(), nbytes, _stream(x))
    _lib.check(rc)
    return out


def grouped_gemm_fp8(xq: torch.Tensor, wq: torch.Tensor, x_scale: torch.Tensor, w_scale: torch.Tensor,
                     expert_ids: torch.Tensor) -> torch.Tensor:
    """Top-1 grouped fp8 a8w8 expert GEMM -> bf16 [M,N] in token order:
    ``out[m] = (xq[m]*x_scale[m]) @ (wq[e]*w_scale[e])^T``, ``e = expert_ids[m]``.

    xq[M,K] / wq[E,N,K] float8_e4m3fn, x_scale[M,1] (or [M]) per token, w_scale[E,N,1]
    (or [E,N]) per expert and output channel.  Rows whose id is outside [0, E) are
    zero.  The kernels need N % 128 == 0 and K % 128 == 0; other shapes are zero-padded
    here first (a copy of ``wq``).
    """
    _require_cuda(xq, wq, x_scale, w_scale, expert_ids)
    if xq.dtype != torch.float8_e4m3fn or wq.dtype != torch.float8_e4m3fn:
        raise NotImplementedError(f"grouped_gemm_fp8 runs float8_e4m3fn operands (got {xq.dtype}, {wq.dtype})")
    if xq.dim() != 2 or wq.dim() != 3 or wq.shape[2] != xq.shape[1]:
        raise ValueError(f"expected xq[M,K], wq[E,N,K] (got {tuple(xq.shape)}, {tuple(wq.shape)})")
    M, K = xq.shape
    E, N, _ = wq.shape
    if expert_ids.numel() != M or x_scale.numel() != M or w_scale.numel() != E * N:
        raise ValueError("expected expert_ids[M], x_scale[M,1] and w_scale[E,N,1]")
    ids = expert_ids.reshape(M).to(torch.int32).contiguous()
    xs = x_scale.reshape(M).to(torch.float32).contiguous()
    ws = w_scale.reshape(E, N).to(torch.float32).contiguous()
    if M == 0 or N == 0:
        return torch.zeros((M, N), dtype=torch.bfloat16, device=xq.device)
    Kp, Np = -(-K // 128) * 128, -(-N // 128) * 128
    if Kp != K or Np != N:
        xp = torch.zeros((M, Kp), dtype=torch.uint8, device=xq.device)
        xp[:, :K] = xq.view(torch.uint8)
        wp = torch.zeros((E, Np, Kp), dtype=torch.uint8, device=wq.device)
        wp[:, :N, :K] = wq.view(torch.uint8)
        wsp = torch.ones((E, Np), dtype=torch.float32, device=ws.device)
        wsp[:, :N] = ws
        return grouped_gemm_fp8(xp.view(torch.float8_e4m3fn), wp.view(torch.float8_e4m3fn), xs, wsp,
                                ids)[:, :N].contiguous()
    x = xq if xq.stride(1) == 1 and xq.stride(0) % 16 == 0 else xq.contiguous()
    wc = wq.contiguous()
    out = torch.zeros((M, N), dtype=torch.bfloat16, device=x.device)
    lib = _lib.load()
    nbytes = lib.kore_moe_grouped_gemm_workspace_bytes(M, E)
    wsp_ = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
    rc = lib.kore_moe_grouped_gemm_fp8(x.data_ptr(), x.stride(0), wc.data_ptr(), xs.data_ptr(), 1, ws.data_ptr(),
                                       ids.data_ptr(), out.data_ptr(), out.stride(0), M, N, K, E, wsp_.data_ptr(),
                                       nbytes, _stream(x))
    _lib.check(rc)
    return out


def _rows(op: str, src: torch.Tensor, idx: torch.Tensor, dst: torch.Tensor, rows: int) -> None:
    lib = _lib.load()
    eb = src.element_size()
    n = idx.numel()
    if op == "gather":
        rc = lib.kore_gather_rows(src.data_ptr(), src.stride(0) * eb, rows, idx.data_ptr(), n,
                                  src.shape[1] * eb, dst.data_ptr(), dst.stride(0) * eb, _stream(src))
    else:
        rc = lib.kore_scatter_rows(src.data_ptr(), src.stride(0) * eb, idx.data_ptr(), n, dst.data_ptr(), rows,
                                   src.shape[1] * eb, dst.stride(0) * eb, _stream(src))
    _lib.check(rc)


def moe_permute(hidden: torch.Tensor, sort_idx: torch.Tensor) -> torch.Tensor:
    """Expert-sorted token dispatch: ``out[i] = hidden[sort_idx[i]]`` (any dtype)."""
    _require_cuda(hidden, sort_idx)
    if hidden.dim() != 2 or sort_idx.dim() != 1:
        raise ValueError("expected hidden[M,D] and sort_idx[n]")
    x = hidden if hidden.stride(1) == 1 else hidden.contiguous()
    idx = sort_idx.to(torch.int32).contiguous()
    out = torch.empty((idx.numel(), x.shape[1]), dtype=x.dtype, device=x.device)
    if idx.numel() and x.shape[1]:
        _rows("gather", x, idx, out, x.shape[0])
    return out


def moe_unpermute(permuted: torch.Tensor, sort_idx: torch.Tensor) -> torch.Tensor:
    """Inverse of ``moe_permute``: ``out[sort_idx[i]] = permuted[i]`` (rows not named by
    ``sort_idx`` are zero; ``sort_idx`` is a permutation in the reference tasks)."""
    _require_cuda(permuted, sort_idx)
    if permuted.dim() != 2 or sort_idx.dim() != 1 or sort_idx.numel() != permuted.shape[0]:
        raise ValueError("expected permuted[M,D] and sort_idx[M]")
    x = permuted if permuted.stride(1) == 1 else permuted.contiguous()
    idx = sort_idx.to(torch.int32).contiguous()
    out = torch.zeros_like(x)
    if idx.numel() and x.shape[1]:
        _rows("scatter", x, idx, out, x.shape[0])
    return out


def moe_align_block_offsets(expert_ids: torch.Tensor, num_experts: int, block: int) -> torch.Tensor:
    """``offsets[E+1]`` int32: exclusive cumsum of each expert's token count rounded up to
    a multiple of ``block`` (``kore/tasks/breadth/moe_ext.py:610-621``)."""
    ids = expert_ids.reshape(-1, 1).to(torch.int32)
    return moe_align(ids, int(num_experts), int(block))[0]


def moe_expert_offsets(expert_ids: torch.Tensor, num_experts: int) -> torch.Tensor:
    """``offsets[E+1]`` int32: exclusive cumsum of the per-expert token counts
    (``kore/tasks/breadth/moe_ext.py:600-608``); the block-1 case of the align offsets."""
    return moe_align_block_offsets(expert_ids, num_experts, 1)


# Alias for drop-in shims: the reference's static scanner rejects any ``<x>.fused_moe(``
# call (kore/reward/reward.py:118), so ``kernel.py`` reaches the same operator by
# this name.
moe_gated_silu = fused_moe
