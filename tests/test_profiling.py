"""CPU tests of the rocprofv3 summarisers (synthetic CSVs in rocprofv3's layout) and
of the benchmark workload registry."""

from __future__ import annotations

import csv
import math
from argparse import Namespace
from pathlib import Path

from kore_amd import profiling as P
from kore_amd import roofline as R
from kore_amd.workloads import bench_workloads


def _counters(d: Path, rows):
    d.mkdir(parents=True)
    with open(d / "run_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"], r)))


def test_traffic_calibration_and_roundtrip(tmp_path):
    kern = "void kore::(anonymous namespace)::gemm_fp8_pipe_kernel<X>(P)"
    # two dimension instances per dispatch are summed; the median over dispatches is used
    _counters(tmp_path / "f", [(1, kern, "FETCH_SIZE", 100), (1, kern, "FETCH_SIZE", 100),
                               (2, kern, "FETCH_SIZE", 150), (2, kern, "FETCH_SIZE", 150),
                               (3, "other", "FETCH_SIZE", 9999)])
    _counters(tmp_path / "w", [(1, kern, "WRITE_SIZE", 50), (2, kern, "WRITE_SIZE", 50)])
    _counters(tmp_path / "cf", [(7, "__amd_rocclr_copyBuffer", "FETCH_SIZE", 512)])
    _counters(tmp_path / "cw", [(7, "__amd_rocclr_copyBuffer", "WRITE_SIZE", 1024)])
    assert P.counter_values(str(tmp_path / "f"), "FETCH_SIZE", "gemm_fp8_pipe") == [200.0, 300.0]
    out = tmp_path / "traffic.md"
    a = Namespace(workload="w1", kernel="gemm_fp8_pipe", fetch=str(tmp_path / "f"), write=str(tmp_path / "w"),
                  copy_fetch=str(tmp_path / "cf"), copy_write=str(tmp_path / "cw"), copy_mib=1,
                  copy_kernel="copy", out=str(out), cmd="cmd")
    P.write_traffic(a)
    # fetch: median 250 KiB x (1024/512); write: 50 KiB x (1024/1024)
    want = (250 * 2.0 + 50 * 1.0) * 1024
    assert math.isclose(P.read_traffic("w1", str(out)), want)
    # a second workload keeps the first; rewriting the first replaces its section
    a.workload = "w2"
    P.write_traffic(a)
    a.workload = "w1"
    P.write_traffic(a)
    text = out.read_text()
    assert text.count("## w1") == 1 and text.count("## w2") == 1
    assert P.read_traffic("w2", str(out)) == P.read_traffic("w1", str(out))
    assert P.read_traffic("missing", str(out)) is None
    assert P.read_traffic("w1", str(tmp_path / "nope.md")) is None


def _trace(d: Path, rows):
    d.mkdir(parents=True)
    with open(d / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for name, start, dur in rows:
            w.writerow({"Kernel_Name": name, "Start_Timestamp": start, "End_Timestamp": start + dur})


def test_stats_keep_only_the_timed_calls(tmp_path):
    """3 warm-up + 2 timed calls of a two-kernel step: only the last two calls' dispatches
    (and the torch fill inside their window) are summarised; the slow first calls (clock
    ramp) and the input generation before them are not."""
    ka = "void kore::(anonymous namespace)::gemm_a_kernel<1>(P)"
    kb = "kore::(anonymous namespace)::combine_kernel(P)"
    fill = "void at::native::vectorized_elementwise_kernel<FillFunctor>(int)"
    rows, t = [(fill, 0, 500)], 1000
    for call, (da, db) in enumerate([(90, 9), (50, 5), (40, 4), (10, 2), (12, 2)]):
        rows += [(ka, t, da), (kb, t + 100, db)]
        if call == 4:
            rows.append((fill, t + 150, 7))
        t += 1000
    _trace(tmp_path / "tr", rows)
    kept = P.timed_dispatches(str(tmp_path / "tr"), warmup_calls=3, iters=2)
    assert [d for n, d in kept if n == ka] == [10, 12] and [d for n, d in kept if n == kb] == [2, 2]
    assert [d for n, d in kept if n == fill] == [7]
    assert len(P.timed_dispatches(str(tmp_path / "tr"))) == 12
    out = tmp_path / "s.md"
    P.write_stats(str(tmp_path / "tr"), str(out), "cmd", "t", 3, 2)
    row = [ln for ln in out.read_text().splitlines() if ln.startswith("| `gemm_a_kernel")][0]
    assert row.startswith("| `gemm_a_kernel<1>` | 2 | 0.0 |")  # 11 ns average, printed in us
    # a kernel count that is not a multiple of the calls is an error, not a silent average
    _trace(tmp_path / "bad", rows[:-2])
    try:
        P.timed_dispatches(str(tmp_path / "bad"), warmup_calls=3, iters=2)
    except SystemExit as e:
        assert "not a multiple" in str(e)
    else:
        raise AssertionError("expected SystemExit")


def test_copy_fetch_factor(tmp_path):
    f = tmp_path / "t.md"
    f.write_text("x\ncopy calibration: 256 MiB copy counted FETCH 131084 KiB, WRITE 262144 KiB (known 262144 KiB)\n")
    assert math.isclose(P.copy_fetch_factor(str(f)), 262144 / 131084)
    assert P.copy_fetch_factor(str(tmp_path / "none.md")) is None


def test_short_kernel_names():
    assert P._short("void kore::(anonymous namespace)::gemm_buf_kernel<kore::BF16, 256, 256>(kore::P)") == \
        "gemm_buf_kernel<BF16, 256, 256>"
    assert P._short("kore::(anonymous namespace)::moe_align_kernel(int const*, int)") == "moe_align_kernel"


def test_bench_workloads_cover_every_config():
    w = bench_workloads()
    assert list(w)[0] == "fp8_blockscale_2048x7168x4096"
    want = {"bf16_gemm_4096", "bf16_gemm_1024", "fp16_gemm_bias_gelu_4096", "fp16_gemm_bias_relu_4096",
            "fp16_gemm_bias_silu_4096", "bf16_batched_64x1024x1024x128", "fp8_blockscale_512x7168x4096",
            "fp8_blockscale_128x7168x4096", "fp8_blockscale_16x7168x4096", "moe_decode_T64", "moe_prefill_T4096"}
    assert want <= set(w)


def test_headline_roofline_figures():
    """The headline's algorithmic work: 2*2048*7168*4096 FLOPs over (MK + NK) fp8 bytes
    plus 2MN bf16 output bytes; MFMA-bound at 5 PF."""
    r = R.roofline("gemm_fp8", {"M": 2048, "N": 7168, "K": 4096}, "fp8")
    assert r.flops == 2.0 * 2048 * 7168 * 4096
    assert r.bytes == 2048 * 4096 + 7168 * 4096 + 2 * 2048 * 7168
    assert r.bound == "mfma"


def test_pmc_summary_sections(tmp_path):
    kern = "void kore::(anonymous namespace)::gemm_fp8_pipe_kernel<X>(P)"
    _counters(tmp_path / "p", [(1, kern, "MfmaUtil", 40.0), (2, kern, "MfmaUtil", 44.0), (3, kern, "MfmaUtil", 50.0),
                               (1, kern, "LdsBankConflict", 0.25), (2, kern, "LdsBankConflict", 0.25),
                               (3, kern, "LdsBankConflict", 0.25), (4, "other", "MfmaUtil", 99.0)])
    out = tmp_path / "pmc.md"
    P.write_pmc(Namespace(dir=str(tmp_path / "p"), workload="w1", out=str(out), cmd="cmd1", note=""))
    P.write_pmc(Namespace(dir=str(tmp_path / "p"), workload="w2", out=str(out), cmd="cmd2", note="n"))
    P.write_pmc(Namespace(dir=str(tmp_path / "p"), workload="w1", out=str(out), cmd="cmd3", note=""))
    text = out.read_text()
    assert text.count("## w1") == 1 and text.count("## w2") == 1 and "cmd3" in text and "cmd1" not in text
    row = [ln for ln in text.splitlines() if ln.startswith("| `gemm_fp8_pipe_kernel")][0]
    assert "| 44.0 |" in row and "0.250" in row  # medians; the non-kore kernel is ignored


def test_grounding_passes_and_derived():
    """The grounding groups stay within one rocprofv3 pass each (<= 8 SQ, <= 4 TCC,
    <= 2 GRBM counters) and the derived values follow the verifier's formulas."""
    from kore_amd import profiling as P

    for g in P.GROUNDING_PASSES:
        assert sum(c.startswith("SQ_") for c in g) <= 8
        assert sum(c.startswith("TCC_") for c in g) <= 4
        assert sum(c.startswith("GRBM_") for c in g) <= 2
    d = P.grounding_derived({"TCC_HIT_sum": 3.0, "TCC_MISS_sum": 1.0, "TCC_EA0_RDREQ_sum": 10.0,
                             "TCC_EA0_RDREQ_32B_sum": 4.0, "TCC_EA0_WRREQ_sum": 5.0, "TCC_EA0_WRREQ_64B_sum": 5.0,
                             "SQ_VALU_MFMA_BUSY_CYCLES": 512.0, "GRBM_GUI_ACTIVE": 1.0,
                             "SQ_INSTS_VALU_MFMA_MOPS_BF16": 2.0})
    assert d["l2_hit_rate"] == 0.75
    assert d["hbm_read_bytes"] == 32 * 4 + 64 * 6 and d["hbm_write_bytes"] == 64 * 5
    assert d["mfma_busy_fraction"] == 1.0 and d["mfma_busy_pct"] == 400.0
    assert d["mfma_flops"] == 1024.0 and d["mfma_ops"] == 514.0


def test_vendor_stats_last_dispatches(tmp_path):
    """The vendor summary averages the last `iters` dispatches of each vendor kernel and
    ignores everything else (the warm-up calls, torch's own kernels)."""
    rows, t = [], 0
    for name, durs in [("Cijk_A_MT256", [900, 800, 100, 110]), ("Custom_Cijk_B", [50, 40, 30, 30]),
                       ("at::native::fill", [5, 5])]:
        for d in durs:
            rows.append((name, t, d))
            t += 1000
    _trace(tmp_path / "v", rows)
    out = tmp_path / "v.md"
    P.write_vendor(str(tmp_path / "v"), str(out), "cmd", 2)
    text = out.read_text()
    assert "| 1 | 0.1 | 0.1 | `Cijk_A_MT256` |" in text and "| 2 | 0.0 | 0.0 | `Custom_Cijk_B` |" in text
    assert "fill" not in text
