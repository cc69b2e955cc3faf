"""Benchmark of the GEMM-family hot path on one MI355X.

``python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME,...] [--no-cpu]``

A "step" is one call of an operator on one batch of synthetic, seeded inputs that
are resident in HBM before timing starts.  The headline (``value``) is the fp8
a8w8 block-scaled GEMM at M=2048, N=7168, K=4096 -- the first configuration named
by the metric; every other BASELINE configuration (bf16 GEMM 4096^3 and 1024^3,
fp16 GEMM+bias+{GELU,ReLU,SiLU} 4096^3, batched GEMM, the fp8 M sweep, MoE decode
T=64 and prefill T=4096) is reported under ``configs`` with the same fields.

Per configuration: W warm-up steps, then K steps back to back between
``torch.cuda.synchronize()`` calls.  ``ms_per_step`` is host wall time / K;
``kernel_ms`` is the HIP-event time over the same K steps / K, with both events
recorded on the stream the kernels are launched on (torch's current stream).
``graph_ms`` is the same K steps captured once in a HIP graph and replayed, timed
with events around the replays / K: back-to-back device time without host launch
gaps, which for microsecond kernels (fp8 M=16) is otherwise dominated by the Python
call.  Per-configuration ``tflops``/``tb_per_s``/``frac_of_bound`` use the lower of
``kernel_ms`` and ``graph_ms`` (graph replay adds a few microseconds of per-node
overhead on long kernels); the headline ``value`` is wall time and its ``roofline``
uses ``kernel_ms``.  ``cold_ms`` follows the reference drivers' protocol: median of events
around one step preceded by a 512 MiB cache flush (``kore/tasks/_genops.py:787-813`` flushes
256 MiB; MI355X has 256 MiB of Infinity Cache).  Roofline fractions use the
algorithmic FLOPs/bytes of ``kore_amd.roofline`` and MI355X peaks (bf16 2.5 PF, fp8
5.0 PF, HBM 8 TB/s).  ``roofline.traffic`` is the HBM traffic per launch of the
headline kernel recorded by rocprofv3 FETCH_SIZE/WRITE_SIZE runs
(``profiles/hbm_traffic.md``, written by ``python -m kore_amd.profiling traffic``).

``cpu_baseline`` times the CPU oracle (the restated torch-fp32 reference) on a row
sample of the headline workload, on the host's cores; it is a reported baseline.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

HEADLINE = "fp8_blockscale_2048x7168x4096"


def _parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--only", default=None, help="comma-separated config names to run")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    p.add_argument("--cold-iters", type=int, default=10)
    p.add_argument("--no-graph", action="store_true", help="skip the graph-replay timing")
    return p.parse_args()


class Timer:
    def __init__(self, steps: int, warmup: int, cold_iters: int, graph: bool = True):
        self.steps, self.warmup, self.cold_iters, self.graph = steps, warmup, cold_iters, graph
        self._flush = None

    def graph_ms(self, fn, replays: int = 3):
        """Device time per step of K steps captured in one graph and replayed."""
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(self.steps):
                fn()
        g.replay()  # first replay uploads the graph
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(replays):
            g.replay()
        end.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / (replays * self.steps)
        del g
        return ms

    def run(self, fn, min_warm_s: float = 0.5):
        # W warm-up steps, and at least min_warm_s of them so the GPU clocks have
        # ramped before the first timed configuration
        t_w = time.perf_counter()
        n = 0
        while n < self.warmup or time.perf_counter() - t_w < min_warm_s:
            fn()
            n += 1
            if n % 8 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record()
        for _ in range(self.steps):
            fn()
        end.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / self.steps
        kern = start.elapsed_time(end) / self.steps
        cold = []
        if self.cold_iters:
            if self._flush is None:
                self._flush = torch.empty(512 * 1024 * 1024, dtype=torch.int8, device="cuda")
            for _ in range(self.cold_iters):
                self._flush.zero_()
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                fn()
                e.record()
                torch.cuda.synchronize()
                cold.append(s.elapsed_time(e))
        graph = self.graph_ms(fn) if self.graph else None
        return wall, kern, (statistics.median(cold) if cold else None), graph


def _entry(name, op, dims, dtype, wall, kern, cold, graph):
    from kore_amd import roofline as R

    rf = R.roofline(op, dims, dtype)
    # device time per step: the lower of the eager event time and the graph-replay
    # time (eager includes host launch gaps for microsecond kernels; graph replay adds
    # per-node overhead that shows on long kernels)
    t = (min(kern, graph) if graph is not None else kern) * 1e-3
    return {
        "name": name, "op": op, "dims": dims, "dtype": dtype,
        "ms_per_step": round(wall, 5), "kernel_ms": round(kern, 5),
        "graph_ms": round(graph, 5) if graph is not None else None,
        "cold_ms": round(cold, 5) if cold is not None else None,
        "tflops": round(rf.flops / t / 1e12, 2),
        "tb_per_s": round(rf.bytes / t / 1e12, 3),
        "bound": rf.bound,
        "frac_of_bound": round(rf.t_min_s / t, 4),
        "frac_mfma_peak": round(rf.flops / t / rf.peak_flops, 4),
        "frac_hbm_peak": round(rf.bytes / t / rf.peak_bw, 4),
    }


def cpu_baseline(seconds_budget: float = 20.0):
    """Time the CPU oracle (restated torch-fp32 reference) on a row sample of the
    headline fp8 workload: rows [0, m) of X against the full W [7168, 4096]."""
    from kore_amd import workloads as W
    from oracle.quant import matmul_blockscale_ref

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    m = 128
    xq, wq, xs, ws = W.fp8_inputs(2048, 7168, 4096, seed=0, device="cpu")
    xq, xs = xq[:m].contiguous(), xs[:m].contiguous()
    matmul_blockscale_ref(xq, wq, xs, ws)  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 and time.perf_counter() - t_start < seconds_budget:
        t0 = time.perf_counter()
        matmul_blockscale_ref(xq, wq, xs, ws)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {"value": round(2.0 * m * 7168 * 4096 / t / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle.quant.matmul_blockscale_ref on rows 0..{m} of the 2048x7168x4096 workload "
                      f"(fp32 dequant + torch CPU matmul on {threads} threads), median of {len(times)} runs, "
                      f"{t * 1e3:.1f} ms per run"}


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU; --gpus {args.gpus} is not supported "
              "(the GEMM family shards without communication; the sharding design is documented, "
              "not measured).", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    import kore_amd._lib as L
    from kore_amd.profiling import read_traffic
    from kore_amd.workloads import bench_workloads

    L.load()
    dev = torch.device("cuda:0")
    timer = Timer(args.steps, args.warmup, args.cold_iters, graph=not args.no_graph)
    work = bench_workloads()
    names = list(work)
    if args.only:
        names = [n for n in names if n in args.only.split(",")]
    results = {}
    for name in names:
        fn, op, dims, dtype = work[name](dev)
        wall, kern, cold, graph = timer.run(fn)
        results[name] = _entry(name, op, dims, dtype, wall, kern, cold, graph)
        r = results[name]
        gtxt = f"graph {graph * 1e3:.1f} us, " if graph is not None else ""
        print(f"# {name}: {r['tflops']} TFLOP/s, {r['tb_per_s']} TB/s, kernel {kern * 1e3:.1f} us, "
              f"{gtxt}wall {wall * 1e3:.1f} us, frac_of_bound {r['frac_of_bound']}", file=sys.stderr, flush=True)
        del fn
        torch.cuda.empty_cache()
    head = results.get(HEADLINE) or next(iter(results.values()))
    flops = 2.0 * head["dims"]["M"] * head["dims"]["N"] * head["dims"]["K"] if "K" in head["dims"] else None
    # the headline roofline is priced on the eager timed region's event time per launch
    from kore_amd import roofline as R

    hrf = R.roofline(head["op"], head["dims"], head["dtype"])
    if head["bound"] == "mfma":
        achieved = round(hrf.flops / (head["kernel_ms"] * 1e-3) / 1e12, 2)
        peak, unit = (5000.0 if head["dtype"] == "fp8" else 2500.0), "TFLOP/s"
    else:
        achieved, peak, unit = round(hrf.bytes / (head["kernel_ms"] * 1e-3) / 1e9, 1), 8000.0, "GB/s"
    line = {
        "metric": "TFLOP/s + % MFMA peak, fp8 blockscale GEMM 2048x7168x4096 and bf16 GEMM 4096^3",
        "value": round(flops / (head["ms_per_step"] * 1e-3) / 1e12, 2) if flops else head["tflops"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic (seeded N(0,1) inputs; fp8: quantised 1x128 / 128x128 to OCP e4m3, fp32 scales)",
        "config": {"workload": head["name"], **head["dims"], "parallelism": "single-gpu"},
        "frac_mfma_peak": head["frac_mfma_peak"],
        "roofline": {"bound": head["bound"], "achieved": achieved, "peak": peak, "unit": unit,
                     "frac": round(achieved / peak, 4), "traffic": read_traffic(head["name"]),
                     "kernel": "gemm_fp8_pipe_kernel" if head["dtype"] == "fp8" else None,
                     "kernel_ms": head["kernel_ms"]},
        "configs": results,
    }
    if "bf16_gemm_4096" in results:
        r = results["bf16_gemm_4096"]
        line["bf16_gemm_4096"] = {"tflops": r["tflops"], "frac_mfma_peak": r["frac_mfma_peak"],
                                  "kernel_ms": r["kernel_ms"], "ms_per_step": r["ms_per_step"]}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
