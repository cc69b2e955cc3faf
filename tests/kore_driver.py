"""Run a KORE candidate ``kernel.py`` under the task drivers' verifier protocol.

Test infrastructure: the verdict comes from the CPU oracle (``oracle/``), so this
module lives with the tests.  It restates the protocol of the reference's task
drivers so a shim under ``kore_amd/candidates`` is exercised exactly as ``KoreEnv``
exercises a candidate:

* the candidate module is loaded by path with ``importlib`` (``candidate_kernel``)
  and cached for the process, so module state persists from the timed loop into the
  post-timing re-check (``kore/tasks/gemm_bf16/driver.py:27-41``);
* correctness runs at least five reseeded trials and prints the worst SNR, the AND of
  ``allclose`` and the largest ``max_diff`` (``SNR: x dB`` / ``allclose: b`` /
  ``max_diff: x``; an exception prints ``CANDIDATE_ERROR``), as
  ``gemm_bf16/driver.py:101-124`` and ``_genops.py:947-988`` do;
* ``--bench-mode`` times one implementation: warm-up, a 256 MiB ``zero_()`` cache flush
  enqueued before each timed call's start event, ``wall_ms:`` per call and
  ``median_ms:`` (``gemm_bf16/driver.py:62-98``);
* ``--bench-both [--shapes a;b] --repeat R`` times candidate and reference back to back
  with randomised warm-up/iteration windows and prints ``SHAPE_BEGIN <spec>`` then
  ``CAND_median_ms:`` / ``REF_median_ms:`` per run, followed by the post-timing
  correctness re-check (``_genops.py:1010-1095``).

The reference implementation timed against the candidate is the vendor path on the
GPU (torch: hipBLASLt GEMMs), as in the reference drivers' ``--impl reference``;
AITER, which the reference uses for some tasks, is not installed here.
:func:`parse` applies ``KoreEnv``'s own output regexes (``kore/env/kore_env.py:67-72``,
last match wins).

    python -m tests.kore_driver gemm_bf16 --candidate kore_amd/candidates/gemm_bf16/kernel.py
    python -m tests.kore_driver gemm_bf16 --bench-both --shapes "M=1024,N=1024,K=1024;M=4096,N=4096,K=4096"
"""

from __future__ import annotations

import argparse
import importlib.util
import os
import random
import re
import sys
from dataclasses import dataclass
from pathlib import Path
from typing import Callable

import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from kore_amd import workloads as W  # noqa: E402
from oracle import gemm as og  # noqa: E402
from oracle import moe as om  # noqa: E402
from oracle import quant as oq  # noqa: E402
from oracle.compare import compare_outputs  # noqa: E402

CANDIDATES = ROOT / "kore_amd" / "candidates"


def parse_shape(spec: str, default: dict) -> dict:
    """``"M=1,N=2,K=3"`` -> dict; ``"default"`` -> the task's primary shape
    (the reference's ``parse_shape``, e.g. ``gemm_backward_bf16/reference.py:29-36``)."""
    if not spec or spec == "default":
        return dict(default)
    out = {}
    for kv in spec.split(","):
        k, v = kv.split("=")
        out[k.strip()] = int(v)
    return out


@dataclass
class Task:
    """One driver: entry name, primary shape, seeded inputs, oracle, reference impl."""
    entry: str
    default: dict
    inputs: Callable[[dict, int, str], tuple]          # (shape, seed, device) -> args
    oracle: Callable[[tuple], object]                   # CPU args -> expected (tensor or tuple)
    reference: Callable[[tuple], object]                # device args -> vendor-path output
    atol: float
    rtol: float
    snr: float


def _dense_inputs(shape, seed, device, dtype=torch.bfloat16):
    # gemm_bf16/reference.py:28-36: a ~ N(0,1)/sqrt(K), b[K,N] ~ N(0,1)
    g = torch.Generator().manual_seed(seed)
    M, N, K = shape["M"], shape["N"], shape["K"]
    a = (torch.randn((M, K), generator=g) / K ** 0.5).to(dtype)
    b = torch.randn((K, N), generator=g).to(dtype)
    return a.to(device), b.to(device)


def _fusion_task(op: str, dtype: torch.dtype) -> Task:
    import kore_amd

    has_bias, act = kore_amd.GEMM_FUSION_OPS[op]

    def inputs(shape, seed, device):
        a, b, bias = W.fused_inputs(shape["M"], shape["N"], shape["K"], seed=seed, dtype=dtype)
        args = (a, b, bias) if has_bias else (a, b)
        return tuple(t.to(device) for t in args)

    def oracle(args):
        return og.gemm_fusion_ref(args[0], args[1], args[2] if has_bias else None, act)

    def reference(args):
        y = torch.matmul(args[0], args[1])
        if has_bias:
            y = y + args[2]
        return og.act_fp32(act, y.float()).to(dtype) if act != "none" else y

    tol = dict(atol=1e-2, rtol=1e-2, snr=40.0 if dtype == torch.float32 else 30.0)
    return Task(op, {"M": 512, "N": 4096, "K": 4096}, inputs, oracle, reference, **tol)


def _tasks() -> dict[str, Task]:
    import kore_amd

    t = {
        "gemm_bf16": Task("gemm", {"M": 4096, "N": 4096, "K": 4096}, _dense_inputs,
                          lambda a: og.matmul_ref(a[0], a[1]), lambda a: torch.matmul(a[0], a[1]),
                          atol=1e-2, rtol=1e-2, snr=30.0),
        "genv_batched_gemm_bf16": Task(
            "batched_gemm", {"B": 8, "M": 512, "N": 512, "K": 512},
            lambda s, seed, dev: tuple(
                (torch.randn(sh, generator=torch.Generator().manual_seed(seed + i)) / s["K"] ** 0.5)
                .bfloat16().to(dev) for i, sh in enumerate([(s["B"], s["M"], s["K"]), (s["B"], s["N"], s["K"])])),
            lambda a: og.batched_gemm_ref(a[0], a[1]),
            lambda a: torch.bmm(a[0], a[1].transpose(1, 2).contiguous()),
            atol=1e-2, rtol=1e-2, snr=30.0),
        "gemm_fp8_a8w8_blockscale": Task(
            "gemm", {"M": 4096, "N": 4096, "K": 4096},
            lambda s, seed, dev: tuple(x.to(dev) for x in W.fp8_inputs(s["M"], s["N"], s["K"], seed=seed, scale=0.2)),
            lambda a: oq.matmul_blockscale_ref(*a),
            lambda a: _dequant_matmul(*a),
            atol=5e-1, rtol=5e-2, snr=25.0),
        # gemm_fp8_a8w8_pertoken / gemm_int8_a8w8 (task.yaml: primary 4096^3, snr 25):
        # dynamic per-token x scales [M,1], per-channel w scales [1,N]; the vendor path is
        # hipBLASLt's row-scaled fp8 GEMM / the int8 GEMM with the scales applied after it
        # (the tasks' own baseline, AITER gemm_a8w8, is absent here)
        "gemm_fp8_a8w8_pertoken": Task(
            "gemm", {"M": 4096, "N": 4096, "K": 4096},
            lambda s, seed, dev: tuple(x.to(dev) for x in W.a8w8_inputs(s["M"], s["N"], s["K"], "fp8", "pertoken",
                                                                         seed=seed)),
            lambda a: oq.matmul_a8w8_ref(*a),
            lambda a: torch._scaled_mm(a[0], a[1].t(), scale_a=a[2], scale_b=a[3], out_dtype=torch.bfloat16),
            atol=5e-1, rtol=5e-2, snr=25.0),
        "gemm_int8_a8w8": Task(
            "gemm", {"M": 4096, "N": 4096, "K": 4096},
            lambda s, seed, dev: tuple(x.to(dev) for x in W.a8w8_inputs(s["M"], s["N"], s["K"], "int8", "pertoken",
                                                                         seed=seed)),
            lambda a: oq.matmul_a8w8_ref(*a),
            lambda a: (torch._int_mm(a[0], a[1].t()).float() * a[2] * a[3]).bfloat16(),
            atol=5e-1, rtol=5e-2, snr=25.0),
        "fused_moe_silu_bf16": Task(
            "fused_moe", {"M": 256, "E": 32, "topk": 8, "D": 1024, "I": 768},
            lambda s, seed, dev: tuple(x.to(dev) for x in W.moe_inputs(s["M"], s["E"], s["topk"], s["D"], s["I"],
                                                                        seed=seed, wscale=0.05)),
            lambda a: om.moe_ref(*a),
            lambda a: _moe_torch(*a),  # a torch per-expert loop on the GPU (AITER absent)
            atol=3e-2, rtol=3e-2, snr=25.0),
        "gemm_backward_bf16": Task(
            "gemm_backward", {"M": 8192, "N": 4096, "K": 4096},
            lambda s, seed, dev: tuple(x.to(dev) for x in W.backward_inputs(s["M"], s["N"], s["K"], seed=seed)),
            lambda a: og.gemm_backward_ref(*a),
            lambda a: (torch.matmul(a[2], a[1]), torch.matmul(a[2].t(), a[0])),
            atol=2e-1, rtol=2e-2, snr=25.0),
    }
    for op in kore_amd.GEMM_FUSION_OPS:
        for dt, name in ((torch.bfloat16, "bf16"), (torch.float16, "fp16"), (torch.float32, "fp32")):
            t[f"gen_{op}_{name}"] = _fusion_task(op, dt)
    return t


def _moe_torch(hidden, w1, w2, topk_weight, topk_ids):
    """Vendor-path bar for the MoE task: per expert, two hipBLASLt GEMMs in the input
    dtype with SiLU-and-mul in fp32 between them, weighted scatter-add into the output."""
    I = w2.shape[2]
    out = torch.zeros(hidden.shape, dtype=torch.float32, device=hidden.device)
    ids = topk_ids.long()
    for e in range(w1.shape[0]):
        mask = ids == e
        idx = mask.any(dim=1).nonzero(as_tuple=True)[0]
        if idx.numel() == 0:
            continue
        gu = torch.matmul(hidden[idx], w1[e].t()).float()
        h = (torch.nn.functional.silu(gu[:, :I]) * gu[:, I:]).to(hidden.dtype)
        y = torch.matmul(h, w2[e].t()).float()
        out.index_add_(0, idx, y * (topk_weight.float() * mask.float()).sum(dim=1)[idx, None])
    return out.to(hidden.dtype)


def _dequant_matmul(xq, wq, xs, ws):
    """Vendor-path bar for the block-scaled task: dequantise on the GPU, one matmul."""
    K = xq.shape[1]
    xd = xq.float() * xs.repeat_interleave(128, dim=1)[:, :K]
    wd = wq.float() * ws.repeat_interleave(128, dim=0).repeat_interleave(128, dim=1)[: wq.shape[0], :K]
    return torch.matmul(xd, wd.t()).to(torch.bfloat16)


_MODULES: dict[str, object] = {}


def load_candidate(path: str, entry: str):
    """Load ``kernel.py`` by path (module name ``candidate_kernel``), cached per path."""
    mod = _MODULES.get(path)
    if mod is None:
        spec = importlib.util.spec_from_file_location("candidate_kernel", path)
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        _MODULES[path] = mod
    return getattr(mod, entry)


def _as_tuple(x):
    return tuple(x) if isinstance(x, (tuple, list)) else (x,)


def run_correctness(task: Task, cand_path: str, shape: dict, trials: int = 5, device: str = "cuda") -> int:
    """Worst-trial verdict over >= 5 seeds (the drivers' KernelBench-style multi-trial)."""
    fn = load_candidate(cand_path, task.entry)
    worst, maxd, ok = 999.0, 0.0, True
    for seed in range(max(5, trials)):
        args = task.inputs(shape, seed, device)
        ref = _as_tuple(task.oracle(tuple(a.cpu() for a in args)))
        try:
            out = _as_tuple(fn(*args))
            torch.cuda.synchronize()
        except Exception as e:  # the drivers report and fail the candidate
            print("SNR: -999.00 dB")
            print("allclose: False")
            print("max_diff: inf")
            print(f"CANDIDATE_ERROR: {type(e).__name__}: {e}")
            return 0
        if len(out) != len(ref):
            worst, ok = -999.0, False
            continue
        for o, r in zip(out, ref):
            s, md, close = compare_outputs(o, r, atol=task.atol, rtol=task.rtol)
            worst = min(worst, s)
            maxd = max(maxd, md)
            ok = ok and close
    print(f"SNR: {worst:.2f} dB")
    print(f"allclose: {ok}")
    print(f"max_diff: {maxd:.6f}")
    return 0


_FLUSH = None


def _flush() -> None:
    global _FLUSH
    if _FLUSH is None:
        _FLUSH = torch.empty(256 * 1024 * 1024, dtype=torch.int8, device="cuda")
    _FLUSH.zero_()


def _time(fn, warmup: int, iters: int, cold: bool = True, verbose: bool = True) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    st = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    en = [torch.cuda.Event(enable_timing=True) for _ in range(iters)]
    for i in range(iters):
        if cold:
            _flush()
        st[i].record()
        fn()
        en[i].record()
    torch.cuda.synchronize()
    times = sorted(s.elapsed_time(e) for s, e in zip(st, en))
    if verbose:
        for t in times:
            print(f"wall_ms: {t:.4f}")
    return times[len(times) // 2]


def _bench_fn(task: Task, cand_path: str, shape: dict, impl: str):
    args = task.inputs(shape, 0, "cuda")
    if impl == "reference":
        return lambda: task.reference(args)
    fn = load_candidate(cand_path, task.entry)
    return lambda: fn(*args)


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("task")
    p.add_argument("--candidate", default=None, help="kernel.py (default: kore_amd/candidates/<task>/kernel.py)")
    p.add_argument("--shape", default="default")
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--iters", type=int, default=30)
    p.add_argument("--bench-mode", action="store_true")
    p.add_argument("--bench-both", action="store_true")
    p.add_argument("--shapes", default=None)
    p.add_argument("--repeat", type=int, default=1)
    p.add_argument("--impl", default="candidate", choices=["candidate", "reference"])
    a = p.parse_args(argv)
    tasks = _tasks()
    if a.task not in tasks:
        raise SystemExit(f"unknown task {a.task!r}; known: {', '.join(sorted(tasks))}")
    task = tasks[a.task]
    cand = a.candidate or str(CANDIDATES / a.task / "kernel.py")
    cold = os.environ.get("KORE_BENCH_COLD", "1") != "0"
    shape = parse_shape(a.shape, task.default)
    if a.bench_both:
        specs = [s for s in (a.shapes or a.shape).split(";") if s]
        for spec in specs:
            sh = parse_shape(spec, task.default)
            cf, rf = _bench_fn(task, cand, sh, "candidate"), _bench_fn(task, cand, sh, "reference")
            if a.shapes:
                print(f"SHAPE_BEGIN {spec}")
            for _ in range(max(1, a.repeat)):
                w = random.randint(max(4, a.warmup - 3), a.warmup + 4)
                it = random.randint(max(8, a.iters - 5), a.iters + 6)
                print(f"CAND_median_ms: {_time(cf, w, it, cold, verbose=False):.4f}")
                print(f"REF_median_ms: {_time(rf, w, it, cold, verbose=False):.4f}")
        return run_correctness(task, cand, parse_shape(specs[0], task.default))
    if a.bench_mode:
        med = _time(_bench_fn(task, cand, shape, a.impl), a.warmup, a.iters, cold)
        print(f"median_ms: {med:.4f}")
        if a.impl == "candidate":  # post-timing re-check on the cached module
            return run_correctness(task, cand, shape)
        return 0
    return run_correctness(task, cand, shape)


# KoreEnv's parse (kore/env/kore_env.py:67-72): the last match of each line wins.
_SNR = re.compile(r"SNR:\s*([-\d.eE]+)")
_ALLCLOSE = re.compile(r"allclose:\s*(True|False)", re.IGNORECASE)
_MEDIAN = re.compile(r"(?<![A-Z_])median_ms:\s*([-\d.eE]+)")
_CAND_MED = re.compile(r"CAND_median_ms:\s*([-\d.eE]+)")
_REF_MED = re.compile(r"REF_median_ms:\s*([-\d.eE]+)")


def parse(out: str, snr_gate: float) -> dict:
    """Verdict of one driver run: SNR, allclose, pass, and the timing samples, per
    ``SHAPE_BEGIN`` block when present."""
    def last(rx):
        m = list(rx.finditer(out))
        return m[-1].group(1) if m else None

    snr = last(_SNR)
    ac = last(_ALLCLOSE)
    med = last(_MEDIAN)
    res = {
        "snr_db": float(snr) if snr is not None else None,
        "allclose": None if ac is None else ac.lower() == "true",
        "median_ms": float(med) if med is not None else None,
        "candidate_error": "CANDIDATE_ERROR" in out,
    }
    res["passed"] = bool(res["allclose"]) and res["snr_db"] is not None and res["snr_db"] >= snr_gate \
        and not res["candidate_error"]
    blocks = out.split("SHAPE_BEGIN")
    shapes = {}
    for b in blocks[1:]:
        spec = b.strip().split("\n", 1)[0].strip()
        shapes[spec] = ([float(m.group(1)) for m in _CAND_MED.finditer(b)],
                        [float(m.group(1)) for m in _REF_MED.finditer(b)])
    if not shapes and _CAND_MED.search(out):
        shapes["default"] = ([float(m.group(1)) for m in _CAND_MED.finditer(out)],
                             [float(m.group(1)) for m in _REF_MED.finditer(out)])
    res["shapes"] = shapes
    return res


if __name__ == "__main__":
    sys.exit(main())
