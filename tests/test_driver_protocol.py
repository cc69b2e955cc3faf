"""The verifier-protocol runner (tests/kore_driver.py): shape specs, task table and
the KoreEnv-style parse of driver output, on the CPU."""

from __future__ import annotations

import pytest

from tests import kore_driver as kd


def test_parse_shape():
    assert kd.parse_shape("M=1,N=2,K=3", {"M": 9}) == {"M": 1, "N": 2, "K": 3}
    assert kd.parse_shape("default", {"M": 9}) == {"M": 9}


def test_parse_last_match_and_gate():
    out = "SNR: 10.00 dB\nallclose: False\nSNR: 85.20 dB\nallclose: True\nmax_diff: 0.01\n"
    v = kd.parse(out, 30.0)
    assert v["snr_db"] == 85.2 and v["allclose"] is True and v["passed"]
    assert not kd.parse(out, 90.0)["passed"]
    err = "SNR: -999.00 dB\nallclose: False\nmax_diff: inf\nCANDIDATE_ERROR: ValueError: x\n"
    v = kd.parse(err, 25.0)
    assert v["candidate_error"] and not v["passed"]


def test_parse_bench_both_blocks():
    out = ("SHAPE_BEGIN M=1,N=2,K=3\nCAND_median_ms: 0.5\nREF_median_ms: 1.0\nCAND_median_ms: 0.6\n"
           "REF_median_ms: 1.1\nSHAPE_BEGIN M=4,N=5,K=6\nCAND_median_ms: 2.0\nREF_median_ms: 3.0\n"
           "SNR: 60.0 dB\nallclose: True\n")
    v = kd.parse(out, 30.0)
    assert v["shapes"]["M=1,N=2,K=3"] == ([0.5, 0.6], [1.0, 1.1])
    assert v["shapes"]["M=4,N=5,K=6"] == ([2.0], [3.0])
    assert v["median_ms"] is None and v["passed"]


def test_task_table_matches_candidates():
    tasks = kd._tasks()
    for name, t in tasks.items():
        path = kd.CANDIDATES / name / "kernel.py"
        assert path.exists(), name
        assert f"def {t.entry}(" in path.read_text(), (name, t.entry)


@pytest.mark.parametrize("task", ["gemm_bf16", "gemm_backward_bf16", "gen_gemm_bias_gelu_fp16",
                                  "gemm_fp8_a8w8_pertoken", "gemm_int8_a8w8"])
def test_task_inputs_and_oracle_shapes(task):
    t = kd._tasks()[task]
    shape = {"M": 64, "N": 48, "K": 32}
    args = t.inputs(shape, 0, "cpu")
    ref = kd._as_tuple(t.oracle(args))
    assert all(r.shape[0] in (64, 48) for r in ref)
