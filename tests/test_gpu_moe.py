"""GPU parity: MoE sort/align (bit-exact) and the fused top-k SiLU MoE (vs oracle)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import kore_amd
from kore_amd import workloads as W
from oracle.moe import moe_align_ref, moe_ref, trace32_bias
from tests.fourprong import ADV_FILLS, bit_equal, pair_only, verdict  # noqa: F401

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,topk,E,block", [(64, 2, 8, 32), (4096, 2, 8, 256), (256, 8, 32, 64),
                                            (1, 1, 4, 16), (333, 3, 70, 64), (2000, 8, 256, 128),
                                            (16384, 8, 128, 64), (2000, 4, 1024, 32), (1000, 1, 3, 1)])
def test_moe_align_bit_exact(gpu, T, topk, E, block):
    """One workgroup per 256 slots (two sub-chunks per workgroup at 131072 slots),
    up to 1024 experts, block 1 (the expert-offsets case): bit-exact against the
    brute-force oracle, invalid ids dropped."""
    g = torch.Generator().manual_seed(T + E)
    ids = torch.randint(0, E, (T, topk), generator=g, dtype=torch.int32)
    if T > 4:
        ids[::5, 0] = E - 1          # a heavy expert
        ids[1::7, -1] = -1           # invalid ids are dropped
        ids[2::11, 0] = E + 3
    off, srt, blk = kore_amd.moe_align(ids.to(gpu), E, block)
    r_off, r_srt, r_blk = moe_align_ref(ids.numpy(), E, block)
    assert np.array_equal(off.cpu().numpy(), r_off)
    n = int(r_off[-1])
    assert np.array_equal(srt.cpu().numpy()[:n], r_srt)
    assert (srt.cpu().numpy()[n:] == T * topk).all()
    assert np.array_equal(blk.cpu().numpy()[: n // block], r_blk)
    assert (blk.cpu().numpy()[n // block:] == -1).all()


@pytest.mark.parametrize("T,E,topk,D,I", [(32, 8, 2, 256, 256), (128, 8, 2, 1024, 1408),
                                          (256, 32, 8, 1024, 768), (64, 32, 8, 1024, 768)])
@pytest.mark.parametrize("seed", range(2))
def test_fused_moe_task_shapes(gpu, T, E, topk, D, I, seed):
    """fused_moe_silu_bf16 task shapes (task.yaml:12-18) with its jagged _TRACE32 router
    bias and dead last expert, weights ~ N(0,1)*0.05 (reference.py:69-78)."""
    hidden, w1, w2, tw, ti = W.moe_inputs(T, E, topk, D, I, seed=seed, wscale=0.05,
                                          router_bias=trace32_bias(E))
    assert not (ti == E - 1).any()
    out = kore_amd.fused_moe(*[t.to(gpu) for t in (hidden, w1, w2, tw, ti)])
    ref = moe_ref(hidden, w1, w2, tw, ti)
    verdict(out, ref, "fused_moe", "bf16", f"T{T} E{E} k{topk} D{D} I{I}")
    # The intermediate h travels to the down projection as two bf16 planes (hi = bf16(h),
    # lo = bf16(h - hi)), so the gate is the north-star 1e-2 allclose bound + SNR.
    verdict(out, ref, "north_star", "bf16", f"T{T} E{E} (1e-2)")


@pytest.mark.parametrize("T,E,topk,D,I", [(640, 4, 2, 512, 384), (700, 4, 3, 384, 256), (520, 2, 1, 256, 640)])
def test_fused_moe_prefill_tiles(gpu, T, E, topk, D, I):
    """Slot counts above 128 per expert select the 256-row prefill tiles (buffer-load
    pipeline for gate_up; two-plane down on 128x256 tiles when D % 256 == 0, else the
    128x128 register-staged tiles); ragged per-expert counts leave padding rows."""
    hidden, w1, w2, tw, ti = W.moe_inputs(T, E, topk, D, I, seed=T, wscale=0.05)
    out = kore_amd.fused_moe(*[t.to(gpu) for t in (hidden, w1, w2, tw, ti)])
    ref = moe_ref(hidden, w1, w2, tw, ti)
    verdict(out, ref, "fused_moe", "bf16", f"prefill tiles T{T} E{E} k{topk} D{D} I{I}")
    verdict(out, ref, "north_star", "bf16", f"prefill tiles T{T} (1e-2)")


@pytest.mark.parametrize("D", [512, 384])
def test_fused_moe_prefill_skewed(gpu, D):
    """256-row prefill tiles under skewed routing: one expert takes about two thirds of
    the 6000 slots (15 blocks, so its rows are split over several column-sweeping
    groups), experts 2, 4 and 7 receive nothing (empty experts between busy ones), the
    rest a few blocks each; D = 512 runs the two-plane down on 128x256 tiles, D = 384
    the 128x128 register-staged tiles."""
    T, E, topk, I = 3000, 8, 2, 384
    counts = torch.tensor([16053.0, 105.0, 0.0, 2724.0, 0.0, 88.0, 4102.0, 0.0])
    bias = torch.log(counts + 1e-6)
    bias[counts == 0] = float("-inf")
    hidden, w1, w2, tw, ti = W.moe_inputs(T, E, topk, D, I, seed=7, wscale=0.05, router_bias=bias)
    used = torch.bincount(ti.flatten(), minlength=E)
    assert used[2] == 0 and used[4] == 0 and used[7] == 0 and used[0] > 6 * 256
    out = kore_amd.fused_moe(*[t.to(gpu) for t in (hidden, w1, w2, tw, ti)])
    ref = moe_ref(hidden, w1, w2, tw, ti)
    verdict(out, ref, "fused_moe", "bf16", f"prefill skewed T{T} D{D}")
    verdict(out, ref, "north_star", "bf16", f"prefill skewed T{T} D{D} (1e-2)")


@pytest.mark.parametrize("T,E,topk,D,I", [(300, 4, 1, 256, 384), (500, 8, 2, 512, 256), (200, 4, 2, 384, 640),
                                          (1024, 32, 2, 768, 512)])
def test_fused_moe_128row_blocks(gpu, T, E, topk, D, I):
    """Slot counts of 17-128 per expert select 128-row blocks on the skinny ring engine
    (each expert's weights streamed once per block, two workgroups per CU for gate_up, the
    XCD-grouped grid for down).  Ragged counts leave padding rows, which the buffer range
    check zero-fills and the epilogues never store; K = 256 is the shortest ring."""
    hidden, w1, w2, tw, ti = W.moe_inputs(T, E, topk, D, I, seed=T + 1, wscale=0.05)
    out = kore_amd.fused_moe(*[t.to(gpu) for t in (hidden, w1, w2, tw, ti)])
    ref = moe_ref(hidden, w1, w2, tw, ti)
    verdict(out, ref, "fused_moe", "bf16", f"128-row blocks T{T} E{E} k{topk} D{D} I{I}")
    verdict(out, ref, "north_star", "bf16", f"128-row blocks T{T} (1e-2)")


def test_fused_moe_decode_config(gpu):
    """BASELINE config 5 decode variant: T=64, E=8, top-2, D=4096, I=14336, weights
    N(0,1)*0.02, plain softmax/top-2/renorm router."""
    args = W.moe_inputs(64, 8, 2, 4096, 14336, seed=0, device=gpu)
    out = kore_amd.fused_moe(*args)
    ref = moe_ref(*[t.cpu() for t in args])
    verdict(out, ref, "fused_moe", "bf16", "decode T=64")
    verdict(out, ref, "north_star", "bf16", "decode T=64 (1e-2)")


def test_fused_moe_prefill_config_sampled(gpu):
    """BASELINE config 5 prefill: T=4096 on the GPU; the oracle checks 256 sampled tokens
    (tokens are independent; 512 expert slots cover all 8 experts), plus determinism of
    the whole output."""
    T, E, topk, D, I = 4096, 8, 2, 4096, 14336
    dev = gpu
    hidden, w1, w2, tw, ti = W.moe_inputs(T, E, topk, D, I, seed=1, device=dev)
    out = kore_amd.fused_moe(hidden, w1, w2, tw, ti)
    out2 = kore_amd.fused_moe(hidden, w1, w2, tw, ti)
    assert bit_equal(out, out2), "determinism"
    rows = torch.randperm(T, generator=torch.Generator().manual_seed(0))[:256].to(dev)
    assert len(torch.unique(ti[rows])) == E
    ref = moe_ref(hidden[rows].cpu(), w1.cpu(), w2.cpu(), tw[rows].cpu(), ti[rows].cpu())
    verdict(out[rows], ref, "fused_moe", "bf16", "prefill T=4096 (256 sampled tokens)")
    verdict(out[rows], ref, "north_star", "bf16", "prefill T=4096 (1e-2)")


def test_fused_moe_prefill_config_full(gpu):
    """BASELINE config 5 prefill, every token: the CPU oracle over the whole T=4096
    output (about 2.9 TFLOP of fp32 CPU work, a few seconds on the host's cores)."""
    T, E, topk, D, I = 4096, 8, 2, 4096, 14336
    hidden, w1, w2, tw, ti = W.moe_inputs(T, E, topk, D, I, seed=1, device=gpu)
    out = kore_amd.fused_moe(hidden, w1, w2, tw, ti)
    ref = moe_ref(*[t.cpu() for t in (hidden, w1, w2, tw, ti)])
    assert ref.device.type == "cpu"
    verdict(out, ref, "fused_moe", "bf16", "prefill T=4096 (all tokens, CPU oracle)")
    verdict(out, ref, "north_star", "bf16", "prefill T=4096 (all tokens, 1e-2)")


@pytest.mark.parametrize("T,E,topk,D,I", [(64, 8, 2, 256, 384), (300, 4, 1, 256, 384), (640, 4, 2, 512, 384),
                                          (700, 4, 3, 384, 256)])
def test_fused_moe_generic_tile_paths(gpu, T, E, topk, D, I):
    """The register-staged tile paths that operands beyond the 32-bit buffer range take
    (forced with the kore_moe_test_force_generic hook): 32-row tiles over 32- and
    128-row aligned blocks (block_expert indexed through the aligned block size) and
    the 256 / 128-row prefill tiles (D % 256 == 0 and not), against the oracle."""
    from kore_amd import _lib

    lib = _lib.load()
    hidden, w1, w2, tw, ti = W.moe_inputs(T, E, topk, D, I, seed=T + 3, wscale=0.05)
    args = [t.to(gpu) for t in (hidden, w1, w2, tw, ti)]
    prev = lib.kore_moe_test_force_generic(1)
    try:
        out = kore_amd.fused_moe(*args)
    finally:
        lib.kore_moe_test_force_generic(prev)
    ref = moe_ref(hidden, w1, w2, tw, ti)
    verdict(out, ref, "fused_moe", "bf16", f"generic tiles T{T} E{E} k{topk} D{D} I{I}")
    verdict(out, ref, "north_star", "bf16", f"generic tiles T{T} (1e-2)")


@pytest.mark.parametrize("T,E,topk,D,I", [(64, 8, 2, 256, 384), (600, 4, 2, 256, 256)])
def test_fused_moe_adversarial(gpu, T, E, topk, D, I):
    """The generic adversarial fills (kore/tasks/_genops.py:855-879) on the activations
    and both weight tensors, the router's weights and ids kept: constant operands
    (h = silu(g) * u at 1e16 scale for the 'large' fill, silu of large negative gates
    at -0), alternating signs and small values; 32-row decode blocks and 256-row
    prefill tiles."""
    hidden, w1, w2, tw, ti = W.moe_inputs(T, E, topk, D, I, seed=T + 5, wscale=0.05)
    for name, fill in ADV_FILLS.items():
        h, a1, a2 = fill(hidden), fill(w1), fill(w2)
        out = kore_amd.fused_moe(h.to(gpu), a1.to(gpu), a2.to(gpu), tw.to(gpu), ti.to(gpu))
        ref = moe_ref(h, a1, a2, tw, ti)
        verdict(out, ref, "fused_moe", "bf16", f"adversarial {name} T{T} E{E} k{topk} D{D} I{I}")


def test_fused_moe_invariants(gpu):
    """Token-permutation equivariance and top-k slot-order invariance."""
    hidden, w1, w2, tw, ti = W.moe_inputs(96, 8, 2, 512, 384, seed=5, wscale=0.05)
    args = [t.to(gpu) for t in (hidden, w1, w2, tw, ti)]
    base = kore_amd.fused_moe(*args)
    perm = torch.randperm(96, generator=torch.Generator().manual_seed(2)).to(gpu)
    permuted = kore_amd.fused_moe(args[0][perm], args[1], args[2], args[3][perm], args[4][perm])
    pair_only(permuted.cpu(), base[perm].cpu(), "bf16", "token permutation", "metamorphic")
    swapped = kore_amd.fused_moe(args[0], args[1], args[2], args[3].flip(1).contiguous(),
                                 args[4].flip(1).contiguous())
    pair_only(swapped.cpu(), base.cpu(), "bf16", "slot order", "metamorphic")
