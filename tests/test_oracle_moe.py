"""Pin the MoE oracles (router, fused MoE, sort/align) on the CPU.

The fused-MoE oracle is checked against two independent formulations (a per
(token, slot) loop and a dense all-experts sum weighted by a scattered [T, E]
router matrix, as in the reference's own checks ``kore/tasks/breadth/tests/
test_moe_ext.py:617-642`` and ``_drafts/moe/_cpu_sanity_check.py:60-80``) and
against structural invariants.  The align oracle is checked against a second brute
force and its defining properties.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from kore_amd import workloads as W
from oracle.moe import TRACE32, jagged_counts, moe_align_ref, moe_ref, route, trace32_bias
from oracle.moe import grouped_gemm_fp8_ref


def _inputs(T=12, E=4, topk=2, D=32, I=24, seed=0, bias=None):
    return W.moe_inputs(T, E, topk, D, I, seed=seed, wscale=0.2, router_bias=bias)


def _per_slot(hidden, w1, w2, tw, ti):
    T, D = hidden.shape
    I = w2.shape[2]
    out = torch.zeros((T, D), dtype=torch.float64)
    for t in range(T):
        x = hidden[t].double()
        for k in range(ti.shape[1]):
            e = int(ti[t, k])
            if not (0 <= e < w1.shape[0]):
                continue
            gu = w1[e].double() @ x
            h = F.silu(gu[:I]) * gu[I:]
            out[t] += float(tw[t, k]) * (w2[e].double() @ h)
    return out


def _dense(hidden, w1, w2, tw, ti):
    E = w1.shape[0]
    I = w2.shape[2]
    dense = torch.zeros((hidden.shape[0], E), dtype=torch.float64)
    dense.scatter_add_(1, ti.long(), tw.double())
    x = hidden.double()
    out = 0
    for e in range(E):
        gu = x @ w1[e].double().t()
        y = (F.silu(gu[:, :I]) * gu[:, I:]) @ w2[e].double().t()
        out = out + dense[:, e:e + 1] * y
    return out


def test_moe_ref_matches_independent_paths():
    args = _inputs()
    got = moe_ref(*args).float()
    for other in (_per_slot(*args), _dense(*args)):
        want = other.float().to(torch.bfloat16).float()
        assert torch.allclose(got, want, atol=1e-2, rtol=1e-2)
        rel = (got - other.float()).norm() / other.float().norm()
        assert rel < 4e-3   # bf16 output rounding only


def test_moe_ref_invariants():
    hidden, w1, w2, tw, ti = _inputs(T=10, E=5, topk=2, seed=3)
    base = moe_ref(hidden, w1, w2, tw, ti)
    perm = torch.randperm(10, generator=torch.Generator().manual_seed(0))
    assert torch.equal(moe_ref(hidden[perm], w1, w2, tw[perm], ti[perm]), base[perm])       # token perm
    relabel = torch.tensor([3, 0, 4, 1, 2])
    inv = torch.argsort(relabel)
    assert torch.allclose(moe_ref(hidden, w1[relabel], w2[relabel], tw, inv[ti.long()].int()).float(),
                          base.float(), atol=1e-2, rtol=1e-2)                                 # expert relabel
    assert torch.allclose(moe_ref(hidden, w1, w2, tw.flip(1), ti.flip(1)).float(), base.float(),
                          atol=1e-2, rtol=1e-2)                                                # slot order


def test_moe_ref_dead_expert_and_invalid_ids():
    hidden, w1, w2, tw, ti = _inputs(T=8, E=4, topk=2, seed=4)
    w1z, w2z = w1.clone(), w2.clone()
    w1z[3] = float("nan")   # never selected -> never read
    w2z[3] = float("nan")
    ti2 = ti.clone()
    ti2[ti2 == 3] = 0
    assert torch.isfinite(moe_ref(hidden, w1z, w2z, tw, ti2).float()).all()
    ti3 = ti.clone()
    ti3[:, 1] = 99                               # out-of-range ids contribute nothing
    tw3 = tw.clone()
    tw3[:, 1] = 0
    assert torch.equal(moe_ref(hidden, w1, w2, tw, ti3), moe_ref(hidden, w1, w2, tw3, ti3))


def test_moe_ref_single_token_is_a_gemv():
    hidden, w1, w2, tw, ti = _inputs(T=1, E=3, topk=1, seed=5)
    tw = torch.ones_like(tw)
    e = int(ti[0, 0])
    I = w2.shape[2]
    gu = w1[e].float() @ hidden[0].float()
    want = (w2[e].float() @ (F.silu(gu[:I]) * gu[I:])).to(torch.bfloat16)
    assert torch.allclose(moe_ref(hidden, w1, w2, tw, ti)[0].float(), want.float(), atol=1e-2, rtol=1e-2)


def test_route_invariants():
    g = torch.Generator().manual_seed(0)
    logits = torch.randn((50, 8), generator=g)
    tw, ti = route(logits, 2)
    assert tw.dtype == torch.float32 and ti.dtype == torch.int32
    assert torch.allclose(tw.sum(-1), torch.ones(50))
    order = torch.argsort(logits, dim=-1, descending=True)[:, :2]
    assert torch.equal(ti.long(), order)
    p = torch.softmax(logits, -1)
    ratio = p.gather(1, order)[:, 0] / p.gather(1, order)[:, 1]
    assert torch.allclose(tw[:, 0] / tw[:, 1], ratio, rtol=1e-5)


def test_trace32_router_never_picks_dead_expert():
    assert TRACE32[-1] == 0 and len(TRACE32) == 32
    assert jagged_counts(40)[-1] == 0 and all(c > 0 for c in jagged_counts(40)[:-1])
    bias = trace32_bias(32)
    assert torch.isinf(bias[-1]) and bias[-1] < 0
    g = torch.Generator().manual_seed(1)
    _, ti = route(torch.randn((500, 32), generator=g) + bias, 8)
    assert not (ti == 31).any()
    counts = torch.bincount(ti.flatten().long(), minlength=32)
    assert counts[0] > counts[1] * 5      # jagged: expert 0 (16053) dominates expert 1 (105)


def test_workload_router_bias_matches_oracle_trace():
    """The bench workloads' router bias (host side) equals the oracle's trace bias."""
    from kore_amd import workloads as W

    for E in (1, 4, 8, 31, 32, 33, 64, 256):
        assert torch.equal(W.jagged_bias(E), trace32_bias(E)), E


def _align_bruteforce(ids, E, block):
    T, topk = ids.shape
    S = T * topk
    buckets = [[] for _ in range(E)]
    for s in range(S):
        e = int(ids.reshape(-1)[s])
        if 0 <= e < E:
            buckets[e].append(s)
    offsets, slots, owners = [0], [], []
    for e in range(E):
        run = buckets[e] + [S] * ((-len(buckets[e])) % block)
        slots += run
        owners += [e] * (len(run) // block)
        offsets.append(offsets[-1] + len(run))
    return np.array(offsets), np.array(slots, dtype=np.int64), np.array(owners, dtype=np.int64)


@pytest.mark.parametrize("T,topk,E,block", [(64, 2, 8, 32), (37, 3, 5, 16), (1, 1, 4, 64), (200, 8, 32, 64)])
def test_moe_align_ref(T, topk, E, block):
    g = torch.Generator().manual_seed(T)
    ids = torch.randint(-1, E + 1, (T, topk), generator=g).numpy()
    off, srt, blk = moe_align_ref(ids, E, block)
    b_off, b_srt, b_blk = _align_bruteforce(ids, E, block)
    assert np.array_equal(off, b_off) and np.array_equal(srt, b_srt) and np.array_equal(blk, b_blk)
    assert (np.diff(off) % block == 0).all()
    valid = ((ids >= 0) & (ids < E)).sum()
    assert (srt < T * topk).sum() == valid                      # every routed slot exactly once
    real = srt[srt < T * topk]
    assert len(np.unique(real)) == len(real)
    counts = np.bincount(ids[(ids >= 0) & (ids < E)], minlength=E)
    assert np.array_equal(off[1:], np.cumsum((counts + block - 1) // block * block))  # moe_ext align_offsets


# ---------------------------------------------------------------------------
# top-1 grouped GEMM, permute / unpermute, expert offsets
# ---------------------------------------------------------------------------
from oracle.moe import expert_offsets_ref, grouped_gemm_ref, moe_align_ref, permute_ref, unpermute_ref  # noqa: E402


def test_grouped_gemm_oracle_two_paths():
    """Per-token matvec (gather) path and the dense one-hot path both equal the oracle;
    a dead expert and an out-of-range id are handled."""
    g = torch.Generator().manual_seed(4)
    M, E, N, K = 40, 5, 24, 32
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = torch.randn(E, N, K, generator=g).to(torch.bfloat16)
    ids = torch.randint(0, E - 1, (M,), generator=g, dtype=torch.int32)  # expert E-1 dead
    ids[3] = E + 2  # matches no expert: zero row
    out = grouped_gemm_ref(x, w, ids)
    per_tok = torch.stack([x[m].double() @ w[ids[m]].double().t() if 0 <= ids[m] < E else torch.zeros(N).double()
                           for m in range(M)])
    assert torch.allclose(out.float(), per_tok.float(), atol=1e-2, rtol=1e-2)
    onehot = torch.zeros(M, E, dtype=torch.float64)
    valid = (ids >= 0) & (ids < E)
    onehot[valid.nonzero()[:, 0], ids[valid].long()] = 1.0
    dense = torch.einsum("me,enk,mk->mn", onehot, w.double(), x.double())
    assert torch.allclose(out.float(), dense.float(), atol=1e-2, rtol=1e-2)
    assert torch.all(out[3] == 0)


def test_grouped_gemm_fp8_oracle_pinned():
    """Per-token dequantised matvecs (exact in float64 for e4m3 products at this K) and,
    with every token on one expert, the dense a8w8 oracle on that expert's weight; a
    dropped scale or a wrong expert index fails one of them."""
    from oracle.quant import matmul_a8w8_ref, quant_rowwise_fp8

    g = torch.Generator().manual_seed(6)
    M, E, N, K = 36, 4, 16, 64
    xq, xs = quant_rowwise_fp8(torch.randn(M, K, generator=g))
    wq = torch.empty(E, N, K, dtype=torch.float8_e4m3fn)
    ws = torch.empty(E, N, 1)
    for e in range(E):
        wq[e], ws[e] = quant_rowwise_fp8(torch.randn(N, K, generator=g) * (e + 1))
    ids = torch.randint(0, E, (M,), generator=g, dtype=torch.int32)
    ids[5] = -1
    out = grouped_gemm_fp8_ref(xq, wq, xs, ws, ids)
    for m in range(M):
        e = int(ids[m])
        if e < 0:
            assert torch.all(out[m] == 0)
            continue
        r = (xq[m].double() * xs[m].double()) @ (wq[e].double() * ws[e].double()).t()
        assert torch.allclose(out[m].float(), r.float(), atol=1e-6, rtol=8e-3), m
    one = torch.full((M,), 2, dtype=torch.int32)
    dense = matmul_a8w8_ref(xq, wq[2], xs, ws[2].reshape(1, N))
    assert torch.equal(grouped_gemm_fp8_ref(xq, wq, xs, ws, one), dense)


def test_permute_unpermute_roundtrip_and_offsets():
    g = torch.Generator().manual_seed(5)
    M, E = 50, 6
    ids = torch.randint(0, E, (M,), generator=g, dtype=torch.int32)
    sort_idx = torch.argsort(ids, stable=True).to(torch.int32)
    h = torch.randn(M, 8, generator=g).to(torch.bfloat16)
    p = permute_ref(h, sort_idx)
    assert torch.all(ids[sort_idx.long()][1:] >= ids[sort_idx.long()][:-1])  # expert-sorted
    assert torch.equal(unpermute_ref(p, sort_idx), h)
    # offsets (block 1) are the bincount prefix sum; align offsets match the align oracle
    off = expert_offsets_ref(ids, E)
    assert off[0] == 0 and off[-1] == M and torch.equal(off[1:] - off[:-1], torch.bincount(ids.long(), minlength=E).int())
    for block in (1, 4, 64):
        a_off, _, _ = moe_align_ref(ids.reshape(M, 1).numpy(), E, block)
        assert np.array_equal(expert_offsets_ref(ids, E, block).numpy(), a_off)
