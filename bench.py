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
uses ``kernel_ms``.  ``cold_ms`` follows the reference drivers' protocol
(``kore/tasks/_genops.py:787-813``): median of events around one step preceded by a
256 MiB ``zero_()`` flush, which leaves the 256 MiB Infinity Cache full of dirty lines;
``cold_frac_of_bound`` is the roofline fraction at that time.  Roofline fractions use the
algorithmic FLOPs/bytes of ``kore_amd.roofline`` and MI355X peaks (bf16 2.5 PF, fp8
5.0 PF, HBM 8 TB/s).  ``roofline.traffic`` is the HBM traffic per launch of the
headline kernel recorded by rocprofv3 FETCH_SIZE/WRITE_SIZE runs
(``profiles/hbm_traffic.md``, written by ``python -m kore_amd.profiling traffic``).

``cpu_baseline`` (per configuration, and for the headline at the top level) times the
CPU oracle -- the restated torch-fp32 reference, ``oracle/`` -- on a bounded sample of
the same seeded inputs (rows, batches or tokens, copied from the device), with
``torch.set_num_threads`` at the host's thread budget, and names the CPU model.  It is
a reported baseline, never a gate.
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
# the kernel the headline dispatches to on MI355X (256 CUs): 256x224 tiles, one per CU
HEADLINE_KERNEL = "gemm_fp8_wide_kernel"


def _parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--only", default=None, help="comma-separated config names to run")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baselines")
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
                self._flush = torch.empty(256 * 1024 * 1024, dtype=torch.int8, device="cuda")
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
    tc = cold * 1e-3 if cold is not None else None
    return {
        "name": name, "op": op, "dims": dims, "dtype": dtype,
        "ms_per_step": round(wall, 5), "kernel_ms": round(kern, 5),
        "graph_ms": round(graph, 5) if graph is not None else None,
        "cold_ms": round(cold, 5) if cold is not None else None,
        "tflops": round(rf.flops / t / 1e12, 2),
        "tb_per_s": round(rf.bytes / t / 1e12, 3),
        "bound": rf.bound,
        "frac_of_bound": round(rf.t_min_s / t, 4),
        "cold_frac_of_bound": round(rf.t_min_s / tc, 4) if tc else None,
        "frac_mfma_peak": round(rf.flops / t / rf.peak_flops, 4),
        "frac_hbm_peak": round(rf.bytes / t / rf.peak_bw, 4),
    }


def cpu_model() -> str:
    """The host CPU's model string, with its family / model / stepping numbers (a
    virtualised host may report only a generic name such as "AMD EPYC")."""
    try:
        info: dict[str, str] = {}
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if not ln.strip():
                    break  # the first processor's block is enough
                k, _, v = ln.partition(":")
                info[k.strip()] = v.strip()
        if "model name" in info:
            ids = [f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info]
            return f"{info['model name']} ({', '.join(ids)}; {os.cpu_count()} logical CPUs)" if ids else info["model name"]
    except OSError:
        pass
    import platform

    return platform.processor() or platform.machine()


def _cpu_threads() -> int:
    # the host's thread budget (OMP_NUM_THREADS where the job sets it, else every core)
    env = os.environ.get("OMP_NUM_THREADS", "")
    return int(env) if env.isdigit() and int(env) > 0 else (os.cpu_count() or 1)


def _cpu_sample(op, dims, dtype, args, target_flops=4e10):
    """(run, work, unit, what): the oracle on a bounded sample of the same inputs."""
    import oracle.gemm as og
    import oracle.moe as om
    import oracle.quant as oq

    cpu = lambda t: t.cpu() if isinstance(t, torch.Tensor) else t  # noqa: E731
    if op == "gemm":
        a, b, bias, act = args
        M, N, K = dims["M"], dims["N"], dims["K"]
        m = max(1, min(M, int(target_flops / (2.0 * N * K))))
        a_s, b_s, bias_s = cpu(a[:m]), cpu(b), cpu(bias)
        return (lambda: og.gemm_fusion_ref(a_s, b_s, bias_s, act)), 2.0 * m * N * K, "TFLOP/s", \
            f"oracle.gemm.gemm_fusion_ref on rows 0..{m} of A"
    if op == "batched_gemm":
        a, b = args
        per = 2.0 * dims["M"] * dims["N"] * dims["K"]
        nb = max(1, min(dims["B"], int(target_flops / per)))
        a_s, b_s = cpu(a[:nb]), cpu(b[:nb])
        return (lambda: og.batched_gemm_ref(a_s, b_s)), per * nb, "TFLOP/s", \
            f"oracle.gemm.batched_gemm_ref on batches 0..{nb}"
    if op == "gemm_backward":
        x, w, dy = args
        M, N, K = dims["M"], dims["N"], dims["K"]
        m = max(1, min(M, int(target_flops / (4.0 * N * K))))
        x_s, w_s, dy_s = cpu(x[:m]), cpu(w), cpu(dy[:m])
        return (lambda: og.gemm_backward_ref(x_s, w_s, dy_s)), 4.0 * m * N * K, "TFLOP/s", \
            f"oracle.gemm.gemm_backward_ref on rows 0..{m} of X and dY"
    if op in ("gemm_fp8", "gemm_a8w8"):
        xq, wq, xs, ws = args
        M, N, K = dims["M"], dims["N"], dims["K"]
        m = max(1, min(M, int(target_flops / (2.0 * N * K))))
        xq_s, wq_s, xs_s, ws_s = cpu(xq[:m]), cpu(wq), cpu(xs[:m]), cpu(ws)
        fn = oq.matmul_blockscale_ref if op == "gemm_fp8" else oq.matmul_a8w8_ref
        return (lambda: fn(xq_s, wq_s, xs_s, ws_s)), 2.0 * m * N * K, "TFLOP/s", \
            f"oracle.quant.{fn.__name__} on rows 0..{m} of X"
    if op == "fused_moe":
        # The oracle upcasts every expert's weights to fp32 on each call; at the BASELINE
        # shapes that copy (2.8 GB of bf16 weights) costs far more than the GEMMs of a
        # bounded token sample.  The weights are upcast once here, before timing (the
        # oracle's own .float() is then a no-op), so the timed runs are its GEMMs and
        # SiLU; the one-off upcast time is reported in the sample string.
        h, w1, w2, tw, ti = args
        per_tok = 6.0 * dims["topk"] * dims["D"] * dims["I"]
        t = max(1, min(dims["M"], int(target_flops / per_tok)))
        t0 = time.perf_counter()
        w1_s, w2_s = cpu(w1).float(), cpu(w2).float()
        up_s = time.perf_counter() - t0
        h_s, tw_s, ti_s = cpu(h[:t]), cpu(tw[:t]), cpu(ti[:t])
        return (lambda: om.moe_ref(h_s, w1_s, w2_s, tw_s, ti_s)), per_tok * t, "TFLOP/s", \
            (f"oracle.moe.moe_ref on tokens 0..{t}, weights upcast to fp32 once before timing "
             f"(that upcast, device copy included: {up_s:.2f} s, not in the rate)")
    if op == "moe_grouped_gemm":
        target_flops /= 4  # the oracle loops over the experts, upcasting each one's weights
        if dtype == "fp8":
            xq, wq, xs, ws, ids = args
            m = max(1, min(dims["M"], int(target_flops / (2.0 * dims["N"] * dims["K"]))))
            sl = (cpu(xq[:m]), cpu(wq), cpu(xs[:m]), cpu(ws), cpu(ids[:m]))
            return (lambda: om.grouped_gemm_fp8_ref(*sl)), 2.0 * m * dims["N"] * dims["K"], "TFLOP/s", \
                f"oracle.moe.grouped_gemm_fp8_ref on tokens 0..{m}"
        x, w, ids = args
        m = max(1, min(dims["M"], int(target_flops / (2.0 * dims["N"] * dims["K"]))))
        sl = (cpu(x[:m]), cpu(w), cpu(ids[:m]))
        return (lambda: om.grouped_gemm_ref(*sl)), 2.0 * m * dims["N"] * dims["K"], "TFLOP/s", \
            f"oracle.moe.grouped_gemm_ref on tokens 0..{m}"
    if op == "moe_permute":
        h, sidx = args
        h_s, sidx_s = cpu(h), cpu(sidx)
        return (lambda: om.permute_ref(h_s, sidx_s)), 2.0 * h.numel() * h.element_size(), "GB/s", \
            "oracle.moe.permute_ref on the whole input"
    return None


def cpu_baseline(op, dims, dtype, args, budget_s: float = 1.5):
    """Median of up to 3 oracle runs on the sample (after one untimed run), within a
    per-configuration time budget."""
    sample = _cpu_sample(op, dims, dtype, args)
    if sample is None:
        return None
    run, work, unit, what = sample
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    run()
    times, t_start = [], time.perf_counter()
    while len(times) < 3 and (not times or time.perf_counter() - t_start < budget_s):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    scale = 1e12 if unit == "TFLOP/s" else 1e9
    return {"value": round(work / t / scale, 4), "unit": unit, "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{what}, fp32 torch on {threads} threads, median of {len(times)} runs, "
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
        w = work[name](dev)
        wall, kern, cold, graph = timer.run(w.fn)
        results[name] = _entry(name, w.op, w.dims, w.dtype, wall, kern, cold, graph)
        r = results[name]
        gtxt = f"graph {graph * 1e3:.1f} us, " if graph is not None else ""
        print(f"# {name}: {r['tflops']} TFLOP/s, {r['tb_per_s']} TB/s, kernel {kern * 1e3:.1f} us, "
              f"{gtxt}wall {wall * 1e3:.1f} us, " + (f"cold {cold * 1e3:.1f} us, " if cold is not None else "") +
              f"frac_of_bound {r['frac_of_bound']} (cold {r['cold_frac_of_bound']})", file=sys.stderr, flush=True)
        if not args.no_cpu:
            r["cpu_baseline"] = cpu_baseline(w.op, w.dims, w.dtype, w.args)
        del w
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
                     "kernel": HEADLINE_KERNEL if head["name"] == HEADLINE else None,
                     "kernel_ms": head["kernel_ms"], "cold_ms": head["cold_ms"],
                     "cold_frac": head["cold_frac_of_bound"]},
        "configs": results,
    }
    if "bf16_gemm_4096" in results:
        r = results["bf16_gemm_4096"]
        line["bf16_gemm_4096"] = {"tflops": r["tflops"], "frac_mfma_peak": r["frac_mfma_peak"],
                                  "kernel_ms": r["kernel_ms"], "ms_per_step": r["ms_per_step"]}
    if head.get("cpu_baseline"):
        line["cpu_baseline"] = head["cpu_baseline"]
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
