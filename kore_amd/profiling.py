"""Workload runner and rocprofv3 summarisers for the GEMM-family kernels.

Run under the profiler (the program itself follows ``--``)::

    rocprofv3 --kernel-trace --stats --output-format csv -d <dir> -o run -- \\
        python3 -m kore_amd.profiling run <workload> [--iters K]   # prints "W warm-up + K timed calls"
    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir> -o run -- \\
        python3 -m kore_amd.profiling run <workload>
    rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir> -o run -- \\
        python3 -m kore_amd.profiling copy --mib 256

then, anywhere (no GPU needed), turn the CSV output into the text summaries kept
under ``profiles/``::

    python3 -m kore_amd.profiling stats <dir> --warmup-calls W --iters K --out profiles/<name>.md --cmd "<command>"
    python3 -m kore_amd.profiling traffic --workload <w> --kernel <substr> \\
        --fetch <dir> --write <dir> --copy-fetch <dir> --copy-write <dir> --copy-mib 256 \\
        --out profiles/hbm_traffic.md --cmd "<commands>"

HBM traffic calibration: FETCH_SIZE / WRITE_SIZE count L2-to-fabric traffic in KiB
per dispatch.  A plain device copy of a known size (``copy``) reads and writes
exactly that many bytes, so ``known / counted`` is the factor applied to the
kernel's counts.  ``bench.py`` reads the resulting ``traffic[...]`` lines.
"""

from __future__ import annotations

import argparse
import csv
import glob
import os
import statistics
import sys

PROFILES = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "profiles")
TRAFFIC_FILE = os.path.join(PROFILES, "hbm_traffic.md")


# --------------------------------------------------------------------------- #
# GPU side: the programs rocprofv3 runs
# --------------------------------------------------------------------------- #
def _run(workload: str, iters: int, warmup: int, min_warm_s: float = 0.5) -> None:
    """``warmup`` calls, and at least ``min_warm_s`` of them (the GPU clock ramps up
    over the first few hundred microseconds of load, as in ``bench.py``), then
    ``iters`` calls.  The printed counts let ``stats --warmup-calls W --iters K`` keep
    only the dispatches of the last K calls."""
    import time

    import torch

    from kore_amd import _lib
    from kore_amd.workloads import bench_workloads

    _lib.load()
    wl = bench_workloads()
    if workload not in wl:
        raise SystemExit(f"unknown workload {workload!r}; choose from {', '.join(wl)}")
    fn = wl[workload](torch.device("cuda:0")).fn
    t0, n = time.perf_counter(), 0
    while n < warmup or time.perf_counter() - t0 < min_warm_s:
        fn()
        n += 1
        if n % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    print(f"profiling.run {workload}: {n} warm-up + {iters} timed calls done", flush=True)


def _copy(mib: int, iters: int) -> None:
    import torch

    n = mib * 1024 * 1024
    x = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    y = torch.empty_like(x)
    for _ in range(iters):
        y.copy_(x)
    torch.cuda.synchronize()
    print(f"profiling.copy: {iters} copies of {mib} MiB done", flush=True)


# --------------------------------------------------------------------------- #
# CPU side: summaries
# --------------------------------------------------------------------------- #
def _one(pattern: str) -> str:
    hits = sorted(glob.glob(pattern, recursive=True))
    if not hits:
        raise SystemExit(f"no file matches {pattern}")
    return hits[0]


def _short(name: str) -> str:
    """Kernel name without the parameter list and anonymous-namespace noise."""
    n = name.replace("kore::(anonymous namespace)::", "").replace("kore::", "")
    if n.startswith("void "):
        n = n[5:]
    depth, out = 0, []
    for ch in n:
        if ch == "(" and depth == 0:
            break
        depth += ch == "<"
        depth -= ch == ">"
        out.append(ch)
    return "".join(out).strip()


def kernel_stats(directory: str) -> list[dict]:
    path = _one(os.path.join(directory, "**", "*kernel_stats.csv"))
    with open(path) as f:
        return list(csv.DictReader(f))


def timed_dispatches(directory: str, warmup_calls: int | None = None, iters: int | None = None):
    """``(name, duration_ns)`` of the traced dispatches in start order, restricted to the
    timed calls: with ``W`` warm-up and ``K`` timed calls, a kore kernel dispatched
    ``n`` times (n a multiple of W + K) keeps its last ``n K / (W + K)`` dispatches, and
    the window opens at the earliest start among those, so every other dispatch inside
    it (workspace fills, copies) is kept too."""
    path = _one(os.path.join(directory, "**", "*kernel_trace.csv"))
    with open(path) as f:
        rows = sorted(csv.DictReader(f), key=lambda r: int(r["Start_Timestamp"]))
    recs = [(r["Kernel_Name"], int(r["Start_Timestamp"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
            for r in rows]
    if not warmup_calls or not iters:
        return [(n, d) for n, _, d in recs]
    total = warmup_calls + iters
    starts: dict[str, list[int]] = {}
    for n, t, _ in recs:
        if "kore" in n:
            starts.setdefault(n, []).append(t)
    opens = []
    for n, ts in starts.items():
        if len(ts) % total:
            raise SystemExit(f"{_short(n)}: {len(ts)} dispatches is not a multiple of {total} calls")
        opens.append(ts[len(ts) - len(ts) // total * iters])
    if not opens:
        raise SystemExit(f"no kore kernels in {path}")
    t_open = min(opens)
    return [(n, d) for n, t, d in recs if t >= t_open]


def write_stats(directory: str, out: str, cmd: str, title: str, warmup_calls: int | None = None,
                iters: int | None = None) -> None:
    recs = timed_dispatches(directory, warmup_calls, iters)
    per: dict[str, list[int]] = {}
    for n, d in recs:
        per.setdefault(n, []).append(d)
    total_ns = sum(d for _, d in recs)
    scope = (f"Dispatches of the last {iters} of {warmup_calls + iters} calls ({warmup_calls} warm-up calls, at "
             "least 0.5 s of them, so the clock has ramped)." if warmup_calls and iters else "All traced dispatches.")
    lines = [f"# {title}", "", "Command (from the repository root, on one MI355X):", "", "```", cmd, "```", "",
             scope, "",
             "| kernel | calls | average (us) | median (us) | min (us) | max (us) | share |",
             "|---|---|---|---|---|---|---|"]
    other_calls, other_ns = 0, 0
    for n, ds in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        if "kore" not in n:  # torch kernels: input generation, workspace fills, copies
            other_calls += len(ds)
            other_ns += sum(ds)
            continue
        lines.append(f"| `{_short(n)}` | {len(ds)} | {statistics.mean(ds) / 1e3:.1f} | "
                     f"{statistics.median(ds) / 1e3:.1f} | {min(ds) / 1e3:.1f} | {max(ds) / 1e3:.1f} | "
                     f"{100.0 * sum(ds) / total_ns:.1f}% |")
    if other_calls:
        lines.append(f"| other (torch kernels: fills, copies) | {other_calls} | {other_ns / other_calls / 1e3:.1f} | "
                     f"| | | {100.0 * other_ns / total_ns:.1f}% |")
    os.makedirs(os.path.dirname(os.path.abspath(out)), exist_ok=True)
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(f"wrote {out}")


def counter_values(directory: str, counter: str, kernel_substr: str) -> list[float]:
    """Per-dispatch values of one counter for the kernels whose name contains
    ``kernel_substr`` (dimension instances summed)."""
    path = _one(os.path.join(directory, "**", "*counter_collection.csv"))
    per = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter or kernel_substr.lower() not in r["Kernel_Name"].lower():
                continue
            per[r["Dispatch_Id"]] = per.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    if not per:
        raise SystemExit(f"{counter} for {kernel_substr!r} not found in {path}")
    return [per[k] for k in sorted(per, key=int)]


def write_traffic(a) -> None:
    fetch = statistics.median(counter_values(a.fetch, "FETCH_SIZE", a.kernel))
    write = statistics.median(counter_values(a.write, "WRITE_SIZE", a.kernel))
    known_kib = a.copy_mib * 1024.0
    cf = statistics.median(counter_values(a.copy_fetch, "FETCH_SIZE", a.copy_kernel))
    cw = statistics.median(counter_values(a.copy_write, "WRITE_SIZE", a.copy_kernel))
    f_fetch, f_write = known_kib / cf, known_kib / cw
    traffic = (fetch * f_fetch + write * f_write) * 1024.0
    entry = (f"traffic[{a.workload}] = {traffic:.0f}  # bytes per launch of {a.kernel}: "
             f"FETCH_SIZE {fetch:.0f} KiB x {f_fetch:.4f} + WRITE_SIZE {write:.0f} KiB x {f_write:.4f}")
    body = []
    if os.path.exists(a.out):
        # keep every other workload's section
        skip = False
        with open(a.out) as f:
            for ln in f:
                ln = ln.rstrip("\n")
                if ln.startswith("## "):
                    skip = ln == f"## {a.workload}"
                if not skip:
                    body.append(ln)
        while body and not body[-1]:
            body.pop()
    if not body:
        body = ["# HBM traffic per launch (rocprofv3 FETCH_SIZE / WRITE_SIZE)", "",
                "FETCH_SIZE and WRITE_SIZE count L2-to-fabric traffic in KiB per dispatch.  Each is",
                "scaled by known/counted for a plain device copy of a known size (same counters,",
                "same session), so the figures are bytes that left or entered the L2s.", ""]
    body += ["", f"## {a.workload}", "", "Commands:", "", "```", a.cmd, "```", "",
             f"copy calibration: {a.copy_mib} MiB copy counted FETCH {cf:.0f} KiB, WRITE {cw:.0f} KiB "
             f"(known {known_kib:.0f} KiB)", "", entry]
    with open(a.out, "w") as f:
        f.write("\n".join(body) + "\n")
    print(entry)


PMC_FILE = os.path.join(PROFILES, "pmc_counters.md")
PMC_COUNTERS = ("MfmaUtil", "LdsBankConflict", "LdsUtil", "VALUBusy")


def _replace_section(path: str, header: list[str], key: str, section: list[str]) -> None:
    """Rewrite ``path`` keeping every ``## <other>`` section and replacing ``## key``."""
    body = []
    if os.path.exists(path):
        skip = False
        with open(path) as f:
            for ln in f:
                ln = ln.rstrip("\n")
                if ln.startswith("## "):
                    skip = ln == f"## {key}"
                if not skip:
                    body.append(ln)
        while body and not body[-1]:
            body.pop()
    if not body:
        body = list(header)
    body += ["", f"## {key}", ""] + section
    with open(path, "w") as f:
        f.write("\n".join(body) + "\n")


def write_pmc(a) -> None:
    """Per-kernel medians of the derived counters of one ``--pmc`` run."""
    path = _one(os.path.join(a.dir, "**", "*counter_collection.csv"))
    vals: dict[str, dict[str, dict[str, float]]] = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if "kore" not in r["Kernel_Name"]:
                continue
            k = _short(r["Kernel_Name"])
            vals.setdefault(k, {}).setdefault(r["Counter_Name"], {})
            d = vals[k][r["Counter_Name"]]
            d[r["Dispatch_Id"]] = d.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
    if not vals:
        raise SystemExit(f"no kore kernels in {path}")
    names = [c for c in PMC_COUNTERS if any(c in v for v in vals.values())]
    unit = {"MfmaUtil": "MFMA busy (% of SIMD-cycles)", "LdsBankConflict": "LDS bank conflicts (cycles per access cycle)",
            "LdsUtil": "LDS active (% of CU-cycles)", "VALUBusy": "VALU busy (% of CU-cycles)"}
    section = ["Command (from the repository root, on one MI355X):", "", "```", a.cmd, "```", "",
               "| kernel | " + " | ".join(unit.get(n, n) for n in names) + " |",
               "|---|" + "---|" * len(names)]
    for k, cs in vals.items():
        cells = []
        for n in names:
            v = statistics.median(cs[n].values()) if n in cs else float("nan")
            cells.append(f"{v:.3f}" if n == "LdsBankConflict" else f"{v:.1f}")
        section.append(f"| `{k}` | " + " | ".join(cells) + " |")
    if a.note:
        section += ["", a.note]
    header = ["# rocprofv3 derived counters per kernel", "",
              "MfmaUtil = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs); LdsBankConflict =",
              "SQ_LDS_BANK_CONFLICT / (SQ_LDS_IDX_ACTIVE - SQ_LDS_BANK_CONFLICT); LdsUtil and VALUBusy are",
              "SQ_LDS_IDX_ACTIVE and SQ_ACTIVE_INST_VALU over GRBM_GUI_ACTIVE x CUs (rocprofv3's own",
              "definitions).  Medians over the profiled dispatches of each kernel.  Busy fractions count",
              "every CU of the GPU, so a grid that occupies 224 of the 256 CUs reads at most 87.5%."]
    _replace_section(a.out, header, a.workload, section)
    print("\n".join(section[-len(vals):]))


# The verifier's "grounding" counter set in its single-pass groups
# (kore/verifier/pmc.py:91-127 for the set, GROUNDING_PASSES for the passes; every
# group fits one rocprofv3 hardware pass on gfx950).
GROUNDING_PASSES = [
    ["SQ_WAVES", "SQ_BUSY_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU", "SQ_INSTS_VMEM", "SQ_INSTS_SALU",
     "SQ_WAIT_INST_ANY", "SQ_WAIT_INST_LDS", "GRBM_GUI_ACTIVE", "GRBM_COUNT"],
    ["SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_VALU_MFMA_MOPS_F16", "SQ_INSTS_VALU_MFMA_MOPS_F32", "SQ_INSTS_LDS",
     "SQ_ACTIVE_INST_VMEM"],
    ["TCC_HIT_sum", "TCC_MISS_sum", "TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum"],
    ["TCC_EA0_WRREQ_sum", "TCC_EA0_WRREQ_64B_sum"],
    ["SQ_INSTS_VALU_MFMA_MOPS_F8", "SQ_INSTS_VALU_MFMA_MOPS_F6F4", "SQ_INSTS_VALU_MFMA_MOPS_XF32"],
]
GROUNDING_FILE = os.path.join(PROFILES, "grounding_counters.md")


def grounding_counters(dirs: list[str], kernel_substr: str) -> dict[str, float]:
    """Median per dispatch of every counter found in the pass directories, for the
    kernels whose name contains ``kernel_substr`` (dimension instances summed)."""
    out: dict[str, float] = {}
    for d in dirs:
        paths = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
        if not paths:
            continue  # a pass that did not run (e.g. counters absent on the device)
        per: dict[str, dict[str, float]] = {}
        with open(paths[0]) as f:
            for r in csv.DictReader(f):
                if kernel_substr.lower() not in r["Kernel_Name"].lower():
                    continue
                c = per.setdefault(r["Counter_Name"], {})
                c[r["Dispatch_Id"]] = c.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
        for name, vals in per.items():
            out[name] = statistics.median(vals.values())
    return out


def grounding_derived(c: dict[str, float], xcds: int = 8, simds: int = 1024) -> dict[str, float]:
    """Derived quantities of the grounding set.

    The verifier's own formulas (kore/verifier/pmc.py): ``l2_hit_rate`` = HIT / (HIT +
    MISS); HBM bytes with the exact 32B/64B split; ``mfma_busy_fraction`` =
    min(1, SQ_VALU_MFMA_BUSY_CYCLES / GRBM_GUI_ACTIVE) and ``mfma_ops`` = the sum of
    the MFMA counters (pmc.py:479-495).  On MI355X SQ_VALU_MFMA_BUSY_CYCLES sums busy
    cycles over all 1024 SIMDs and GRBM_GUI_ACTIVE sums the 8 XCDs' active cycles, so
    the verifier's fraction saturates at 1; ``mfma_busy_pct`` normalises per SIMD-cycle
    (busy / (GRBM_GUI_ACTIVE / 8 x 1024)).  ``mfma_flops`` = 512 x the MOPS counters.
    """
    d: dict[str, float] = {}
    busy, active = c.get("SQ_VALU_MFMA_BUSY_CYCLES"), c.get("GRBM_GUI_ACTIVE")
    if busy is not None and active:
        d["mfma_busy_fraction"] = max(0.0, min(1.0, busy / active))
        d["mfma_busy_pct"] = 100.0 * busy / (active / xcds * simds)
    if "TCC_HIT_sum" in c and "TCC_MISS_sum" in c and c["TCC_HIT_sum"] + c["TCC_MISS_sum"] > 0:
        d["l2_hit_rate"] = c["TCC_HIT_sum"] / (c["TCC_HIT_sum"] + c["TCC_MISS_sum"])
    if "TCC_EA0_RDREQ_sum" in c:
        rd = c["TCC_EA0_RDREQ_sum"]
        rd32 = min(c.get("TCC_EA0_RDREQ_32B_sum", 0.0), rd)
        d["hbm_read_bytes"] = 32.0 * rd32 + 64.0 * (rd - rd32)
    if "TCC_EA0_WRREQ_sum" in c:
        wr = c["TCC_EA0_WRREQ_sum"]
        wr64 = min(c.get("TCC_EA0_WRREQ_64B_sum", 0.0), wr)
        d["hbm_write_bytes"] = 64.0 * wr64 + 32.0 * (wr - wr64)
    mf = [k for k in c if "MFMA" in k.upper()]
    if mf:
        d["mfma_ops"] = sum(c[k] for k in mf)
    mops = sum(c[k] for k in c if k.startswith("SQ_INSTS_VALU_MFMA_MOPS_"))
    if mops:
        d["mfma_flops"] = 512.0 * mops
    return d


def copy_fetch_factor(path: str = TRAFFIC_FILE) -> float | None:
    """known / counted read bytes of the plain device copy recorded in ``path`` (the
    ``copy calibration`` line written by ``traffic``), or None."""
    if not os.path.exists(path):
        return None
    factor = None
    with open(path) as f:
        for ln in f:
            if ln.startswith("copy calibration:"):
                # "... counted FETCH <f> KiB, WRITE <w> KiB (known <k> KiB)"
                parts = ln.replace(",", " ").replace("(", " ").split()
                fetch = float(parts[parts.index("FETCH") + 1])
                known = float(parts[parts.index("known") + 1])
                factor = known / fetch
    return factor


def write_grounding(a) -> None:
    c = grounding_counters(a.dirs, a.kernel)
    if not c:
        raise SystemExit(f"no counters for {a.kernel!r} in {a.dirs}")
    d = grounding_derived(c)
    f = copy_fetch_factor()
    if f is not None and "hbm_read_bytes" in d:
        # the EA0 read requests cover a fixed share of the reads on this device; the copy
        # calibration of profiles/hbm_traffic.md measures it (same counter basis as FETCH_SIZE)
        d["hbm_read_bytes_ea0"] = d["hbm_read_bytes"]
        d["hbm_read_bytes"] = d["hbm_read_bytes_ea0"] * f
        d["copy_fetch_factor"] = f
    section = ["Commands (from the repository root, on one MI355X), one per pass:", "", "```", a.cmd, "```", "",
               f"Kernel: `{a.kernel}`; medians per dispatch.", "", "| counter | value |", "|---|---|"]
    section += [f"| `{k}` | {v:.6g} |" for k, v in sorted(c.items())]
    section += ["", "| derived | value |", "|---|---|"]
    section += [f"| {k} | {v:.6g} |" for k, v in d.items()]
    if a.note:
        section += ["", a.note]
    header = ["# rocprofv3 grounding counters (the KORE verifier's set)", "",
              "The counter set and its five single-pass groups are the reference verifier's",
              "`grounding` set (`kore/verifier/pmc.py:91-127`).  Derived with the verifier's formulas:",
              "`l2_hit_rate` = HIT / (HIT + MISS); HBM bytes from the EA request counts with the",
              "32B/64B split (read = 32 x RDREQ_32B + 64 x (RDREQ - RDREQ_32B), write = 64 x WRREQ_64B",
              "+ 32 x (WRREQ - WRREQ_64B)); `mfma_busy_fraction` = min(1, MFMA_BUSY / GRBM_GUI_ACTIVE);",
              "`mfma_ops` = sum of the MFMA counters.  On MI355X MFMA_BUSY sums all 1024 SIMDs and",
              "GRBM_GUI_ACTIVE sums the 8 XCDs, so that fraction saturates; `mfma_busy_pct` =",
              "MFMA_BUSY / (GRBM_GUI_ACTIVE / 8 x 1024) is per SIMD-cycle.  `mfma_flops` = 512 x MOPS.",
              "The EA0 read requests count half of a plain device copy's reads on MI355X (the copy",
              "calibration in `hbm_traffic.md`, where FETCH_SIZE has the same basis), so",
              "`hbm_read_bytes` = `hbm_read_bytes_ea0` x `copy_fetch_factor`; writes need no factor.",
              "These are the same bytes as `hbm_traffic.md`'s FETCH figures."]
    _replace_section(a.out, header, a.workload, section)
    print("\n".join(section))


def read_traffic(workload: str, path: str = TRAFFIC_FILE):
    """Bytes per launch recorded for ``workload`` in the traffic summary, or None."""
    try:
        with open(path) as f:
            for ln in f:
                if ln.startswith(f"traffic[{workload}]"):
                    return float(ln.split("=", 1)[1].split("#", 1)[0])
    except OSError:
        return None
    return None


def _vendor_configs(dev):
    """``name -> (what, build)`` of the vendor library's call on every compute-bound bench
    configuration (the reference times such a ``baseline_fn`` beside each task,
    ``kore/tasks/_genops.py:453-464``, ``kore/tasks/aiter_ref.py:227-256``).  ``build()``
    draws the bench's own seeded inputs and returns a list of ``(label, fn)`` variants:
    every vendor route torch offers for the op (a fused hipBLASLt epilogue where one
    exists, else the GEMM plus torch's elementwise kernel); the bar is the fastest."""
    import torch
    import torch.nn.functional as F

    from kore_amd import workloads as W

    f8 = torch.float8_e4m3fn

    def fp8(M):
        def build():
            xq, wq, xs, ws = W.fp8_inputs(M, 7168, 4096, seed=0, device=dev)
            one = torch.ones((), device=dev)
            sa, sb = xs[:, :1].contiguous(), ws.new_ones((1, 7168))
            v = [("_scaled_mm per-tensor (unit scales; less work than block scales)",
                  lambda: torch._scaled_mm(xq, wq.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16)),
                 ("_scaled_mm row-wise scales",
                  lambda: torch._scaled_mm(xq, wq.t(), scale_a=sa, scale_b=sb, out_dtype=torch.bfloat16))]
            # 1x128 activation / 128x128 weight block scales, where the vendor path has them
            xsb, wsb = xs.contiguous(), ws.t().contiguous()
            v.append(("_scaled_mm 1x128 / 128x128 block scales",
                      lambda: torch._scaled_mm(xq, wq.t(), scale_a=xsb, scale_b=wsb, out_dtype=torch.bfloat16)))
            return v
        return build

    def dense(n, kn=False):
        def build():
            if kn:
                g = W._gen(dev, 0)
                a = (torch.randn((n, n), generator=g, device=dev) / n ** 0.5).to(torch.bfloat16)
                b = torch.randn((n, n), generator=g, device=dev).to(torch.bfloat16)
            else:
                a, b = W.dense_inputs(n, n, n, seed=0, device=dev)
            return [("torch.matmul", lambda: torch.matmul(a, b))]
        return build

    def fused(act, M=4096, N=4096, K=4096, kn=False, dtype=torch.float16):
        def build():
            if kn:
                g = W._gen(dev, 0)
                a = (torch.randn((M, K), generator=g, device=dev) / K ** 0.5).to(dtype)
                b = (torch.randn((K, N), generator=g, device=dev) / K ** 0.5).to(dtype)
                bias = torch.randn((N,), generator=g, device=dev).to(dtype)
            else:
                a, b, bias = W.fused_inputs(M, N, K, seed=0, device=dev, dtype=dtype)
            ew = {"gelu": lambda y: F.gelu(y, approximate="tanh"), "relu": F.relu, "silu": F.silu}[act]
            v = [("addmm + torch elementwise", lambda: ew(torch.addmm(bias, a, b)))]
            if act in ("gelu", "relu"):
                v.append(("_addmm_activation (hipBLASLt epilogue)",
                          lambda: torch._addmm_activation(bias, a, b, use_gelu=act == "gelu")))
            return v
        return build

    def batched():
        a, bt = W.batched_inputs(64, 1024, 1024, 128, seed=0, device=dev)
        bkn = bt.transpose(1, 2).contiguous()  # [B,K,N] contiguous: no transposed right operand
        return [("torch.bmm", lambda: torch.bmm(a, bkn))]

    def backward():
        x, w, dy = W.backward_inputs(8192, 4096, 4096, seed=0, device=dev)
        dyt = dy.t().contiguous()
        return [("two matmuls (dY^T materialised outside the timed call)",
                 lambda: (torch.matmul(dy, w), torch.matmul(dyt, x))),
                ("two matmuls, dY^T as a view", lambda: (torch.matmul(dy, w), torch.matmul(dy.t(), x)))]

    def fp32_bias():
        g = W._gen(dev, 0)
        a = torch.randn((512, 4096), generator=g, device=dev) / 64.0
        b = torch.randn((4096, 4096), generator=g, device=dev) / 64.0
        bias = torch.randn((4096,), generator=g, device=dev)
        return [("addmm", lambda: torch.addmm(bias, a, b))]

    def a8w8(M, kind):
        def build():
            xq, wq, xs, ws = W.a8w8_inputs(M, 4096, 4096, kind, "pertoken", seed=0, device=dev)
            if kind == "fp8":
                wsr = ws.reshape(1, -1).contiguous()
                return [("_scaled_mm row-wise scales",
                         lambda: torch._scaled_mm(xq, wq.t(), scale_a=xs, scale_b=wsr, out_dtype=torch.bfloat16))]
            wsr = ws.reshape(1, -1)
            return [("torch._int_mm + scales", lambda: (torch._int_mm(xq, wq.t()).float() * xs * wsr).bfloat16())]
        return build

    return {
        "fp8_blockscale_2048x7168x4096": fp8(2048),
        "bf16_gemm_4096": dense(4096),
        "bf16_gemm_1024": dense(1024),
        "bf16_gemm_4096_kn": dense(4096, kn=True),
        "fp16_gemm_bias_gelu_4096": fused("gelu"),
        "fp16_gemm_bias_relu_4096": fused("relu"),
        "fp16_gemm_bias_silu_4096": fused("silu"),
        "bf16_batched_64x1024x1024x128": batched,
        "bf16_gemm_backward_8192x4096x4096": backward,
        "fp16_gemm_bias_gelu_512x4096x4096_kn": fused("gelu", 512, 4096, 4096, kn=True),
        "bf16_gemm_bias_gelu_512x4096x4095_kn": fused("gelu", 512, 4096, 4095, kn=True, dtype=torch.bfloat16),
        "fp32_gemm_bias_512x4096x4096": fp32_bias,
        "fp8_blockscale_512x7168x4096": fp8(512),
        "fp8_blockscale_128x7168x4096": fp8(128),
        "fp8_blockscale_16x7168x4096": fp8(16),
        "fp8_a8w8_pertoken_4096": a8w8(4096, "fp8"),
        "int8_a8w8_4096": a8w8(4096, "int8"),
        "fp8_a8w8_pertoken_16x4096x4096": a8w8(16, "fp8"),
    }


def _vendor(iters: int, out: str | None = None, cmd: str = "", only: str | None = None,
            min_warm_s: float = 0.3) -> None:
    """Time the vendor library on every compute-bound bench configuration, the way
    ``bench.py`` times this build: at least ``min_warm_s`` of warm-up calls, ``iters``
    calls between events (eager), the same calls captured in a graph and replayed, and
    the reference drivers' cold protocol (a 256 MiB ``zero_()`` before each call, median
    of 10).  A variant the vendor path rejects is recorded as unsupported.  Timing only:
    the vendor library is run, never read."""
    import statistics
    import time

    import torch

    dev = torch.device("cuda")
    flush = torch.empty(256 << 20, dtype=torch.int8, device=dev)
    rows = []
    for name, build in _vendor_configs(dev).items():
        if only and name not in only.split(","):
            continue
        variants = build()
        for label, fn in variants:
            try:
                fn()
                torch.cuda.synchronize()
            except Exception as e:  # noqa: BLE001 -- an unsupported vendor route is a result
                rows.append((name, label, None, None, None, f"unsupported: {type(e).__name__}: {str(e)[:80]}"))
                print(f"profiling.vendor {name} / {label}: unsupported ({type(e).__name__})", flush=True)
                continue
            t0, n = time.perf_counter(), 0
            while time.perf_counter() - t0 < min_warm_s:
                fn()
                n += 1
                if n % 32 == 0:
                    torch.cuda.synchronize()
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(iters):
                fn()
            e.record()
            torch.cuda.synchronize()
            eager = s.elapsed_time(e) / iters * 1e3
            graph = None
            try:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    for _ in range(iters):
                        fn()
                g.replay()
                torch.cuda.synchronize()
                s.record()
                for _ in range(3):
                    g.replay()
                e.record()
                torch.cuda.synchronize()
                graph = s.elapsed_time(e) / (3 * iters) * 1e3
                del g
            except Exception:  # noqa: BLE001 -- a route that cannot be captured keeps its eager time
                graph = None
            cold = []
            for _ in range(10):
                flush.zero_()
                s.record()
                fn()
                e.record()
                torch.cuda.synchronize()
                cold.append(s.elapsed_time(e) * 1e3)
            rows.append((name, label, eager, graph, statistics.median(cold), ""))
            print(f"profiling.vendor {name} / {label}: eager {eager:.1f} us, graph "
                  f"{'-' if graph is None else f'{graph:.1f}'} us, cold {statistics.median(cold):.1f} us", flush=True)
        del variants
        torch.cuda.empty_cache()
    if out:
        lines = ["# Vendor bars on the same box (hipBLASLt / torch; timed, never read)", "",
                 "Command (from the repository root, on one MI355X):", "", "```", cmd, "```", "",
                 f"Per variant: {iters} calls between HIP events after at least {min_warm_s} s of warm-up "
                 "(eager), the same calls captured in a graph and replayed (graph), and the reference "
                 "drivers' cold protocol (256 MiB `zero_()` before each call, median of 10).  "
                 "`warm` = the lower of eager and graph, as bench.py reports this build.  The bar of a "
                 "configuration is its fastest supported variant.", "",
                 "| configuration | vendor variant | eager (us) | graph (us) | warm (us) | cold (us) | note |",
                 "|---|---|---|---|---|---|---|"]
        f = lambda v: "-" if v is None else f"{v:.1f}"  # noqa: E731
        for name, label, eager, graph, cold, note in rows:
            warm = None if eager is None else (min(eager, graph) if graph is not None else eager)
            lines.append(f"| {name} | {label} | {f(eager)} | {f(graph)} | {f(warm)} | {f(cold)} | {note} |")
        with open(out, "w") as fh:
            fh.write("\n".join(lines) + "\n")
        print(f"wrote {out}")


def write_vendor(trace_dir: str, out: str, cmd: str, iters: int) -> None:
    """Average duration of the last ``iters`` dispatches of every vendor GEMM kernel
    (names containing ``Cijk``) in a rocprofv3 kernel trace."""
    paths = glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not paths:
        raise SystemExit(f"no kernel_trace.csv under {trace_dir}")
    per: dict[str, list[tuple[int, int]]] = {}
    with open(paths[0]) as f:
        for r in csv.DictReader(f):
            if "Cijk" in r["Kernel_Name"]:
                per.setdefault(r["Kernel_Name"], []).append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    lines = ["# hipBLASLt kernels on the same box (the vendor bar; timed, never read)", "",
             "Commands (from the repository root, on one MI355X):", "", "```", cmd, "```", "",
             f"Average over the last {iters} dispatches of each kernel, after at least 0.5 s of warm-up",
             "calls (back to back, warm cache).  This build on the same shapes: `bf16_gemm_4096.md`,",
             "`fp8_blockscale_2048x7168x4096.md` (block scales, more work than per-tensor),",
             "`fp32_gemm_bias_512x4096x4096.md`; cold task-driver medians in `driver_protocol.md`.", "",
             "| first dispatch order | average (us) | min (us) | kernel (name as printed, truncated) |",
             "|---|---|---|---|"]
    order = sorted(per, key=lambda k: per[k][0][0])
    for i, name in enumerate(order):
        d = sorted(per[name])[-iters:]
        durs = [(e - s_) / 1e3 for s_, e in d]
        lines.append(f"| {i + 1} | {statistics.mean(durs):.1f} | {min(durs):.1f} | `{name[:150]}` |")
    with open(out, "w") as f:
        f.write("\n".join(lines) + "\n")
    print(f"wrote {out}")


def main(argv=None) -> int:
    p = argparse.ArgumentParser(prog="python -m kore_amd.profiling")
    sub = p.add_subparsers(dest="action", required=True)
    r = sub.add_parser("run")
    r.add_argument("workload")
    r.add_argument("--iters", type=int, default=20)
    r.add_argument("--warmup", type=int, default=3)
    r.add_argument("--min-warm-s", type=float, default=0.5,
                   help="seconds of warm-up calls at least (0 for counter runs, which serialise dispatches)")
    c = sub.add_parser("copy")
    c.add_argument("--mib", type=int, default=256)
    c.add_argument("--iters", type=int, default=5)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--out", required=True)
    s.add_argument("--cmd", required=True)
    s.add_argument("--title", default="rocprofv3 kernel-trace summary")
    s.add_argument("--warmup-calls", type=int, default=None, help="warm-up calls printed by `run`")
    s.add_argument("--iters", type=int, default=None, help="timed calls of `run`")
    t = sub.add_parser("traffic")
    t.add_argument("--workload", required=True)
    t.add_argument("--kernel", required=True)
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--copy-fetch", required=True)
    t.add_argument("--copy-write", required=True)
    t.add_argument("--copy-mib", type=int, default=256)
    t.add_argument("--copy-kernel", default="copy")
    t.add_argument("--out", default=TRAFFIC_FILE)
    t.add_argument("--cmd", required=True)
    m = sub.add_parser("pmc")
    m.add_argument("dir")
    m.add_argument("--workload", required=True)
    m.add_argument("--out", default=PMC_FILE)
    m.add_argument("--cmd", required=True)
    m.add_argument("--note", default="")
    vd = sub.add_parser("vendor", help="time the vendor library on every compute-bound bench configuration")
    vd.add_argument("--iters", type=int, default=20)
    vd.add_argument("--out", default=None)
    vd.add_argument("--cmd", default="")
    vd.add_argument("--only", default=None)
    vs = sub.add_parser("vendor-stats")
    vs.add_argument("dir")
    vs.add_argument("--out", required=True)
    vs.add_argument("--cmd", required=True)
    vs.add_argument("--iters", type=int, default=20)
    sub.add_parser("grounding-passes", help="print the grounding counter groups, one pass per line")
    gr = sub.add_parser("grounding")
    gr.add_argument("dirs", nargs="+")
    gr.add_argument("--workload", required=True)
    gr.add_argument("--kernel", required=True)
    gr.add_argument("--out", default=GROUNDING_FILE)
    gr.add_argument("--cmd", required=True)
    gr.add_argument("--note", default="")
    a = p.parse_args(argv)
    if a.action == "run":
        _run(a.workload, a.iters, a.warmup, a.min_warm_s)
    elif a.action == "copy":
        _copy(a.mib, a.iters)
    elif a.action == "stats":
        write_stats(a.dir, a.out, a.cmd, a.title, a.warmup_calls, a.iters)
    elif a.action == "pmc":
        write_pmc(a)
    elif a.action == "vendor":
        _vendor(a.iters, a.out, a.cmd, a.only)
    elif a.action == "vendor-stats":
        write_vendor(a.dir, a.out, a.cmd, a.iters)
    elif a.action == "grounding-passes":
        print("\n".join(" ".join(g) for g in GROUNDING_PASSES))
    elif a.action == "grounding":
        write_grounding(a)
    else:
        write_traffic(a)
    return 0


if __name__ == "__main__":
    sys.exit(main())
