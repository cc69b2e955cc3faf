"""The shims under kore_amd/candidates, run under the task drivers' protocol
(tests/kore_driver.py) on the GPU and judged by KoreEnv's parse: verdict lines from
five reseeded trials, the cold-cache timing lines, and the --bench-both per-shape
candidate/reference medians followed by the post-timing re-check."""

from __future__ import annotations

import contextlib
import io

import pytest

from tests import kore_driver as kd

pytestmark = pytest.mark.gpu


def _run(argv):
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        assert kd.main(argv) == 0
    return buf.getvalue()


@pytest.mark.parametrize("task,shape", [("gemm_bf16", "M=64,N=512,K=512"),
                                        ("gen_gemm_bias_gelu_fp16", "M=256,N=512,K=384"),
                                        ("gen_gemm_sigmoid_fp32", "M=64,N=256,K=256"),
                                        ("gemm_fp8_a8w8_blockscale", "M=128,N=256,K=256"),
                                        ("genv_batched_gemm_bf16", "B=4,M=256,N=256,K=128"),
                                        ("fused_moe_silu_bf16", "M=32,E=8,topk=2,D=256,I=256"),
                                        ("gemm_backward_bf16", "M=256,N=256,K=256"),
                                        ("gemm_fp8_a8w8_pertoken", "M=300,N=512,K=1024"),
                                        ("gemm_int8_a8w8", "M=300,N=512,K=1024")])
def test_driver_correctness(gpu, task, shape):
    out = _run([task, "--shape", shape])
    v = kd.parse(out, kd._tasks()[task].snr)
    assert v["passed"], out


def test_driver_bench_both_shapes(gpu):
    out = _run(["gemm_bf16", "--bench-both", "--shapes", "M=1024,N=1024,K=1024;M=2048,N=2048,K=2048",
                "--repeat", "2", "--warmup", "4", "--iters", "10"])
    v = kd.parse(out, 30.0)
    assert v["passed"], out
    for spec in ("M=1024,N=1024,K=1024", "M=2048,N=2048,K=2048"):
        cand, ref = v["shapes"][spec]
        assert len(cand) == 2 and len(ref) == 2 and min(cand) > 0 and min(ref) > 0


def test_driver_bench_mode(gpu):
    out = _run(["gemm_backward_bf16", "--shape", "M=1024,N=512,K=512", "--bench-mode", "--warmup", "3",
                "--iters", "9"])
    v = kd.parse(out, 25.0)
    assert v["passed"] and v["median_ms"] is not None and out.count("wall_ms:") == 9, out


@pytest.mark.parametrize("task,shape", [("fused_moe_silu_bf16", "M=64,E=8,topk=2,D=256,I=512"),
                                        ("gemm_fp8_a8w8_blockscale", "M=128,N=256,K=512"),
                                        ("gemm_backward_bf16", "M=256,N=128,K=256"),
                                        ("gemm_fp8_a8w8_pertoken", "M=256,N=512,K=512"),
                                        ("gemm_int8_a8w8", "M=256,N=512,K=512")])
def test_driver_reference_impls(gpu, task, shape):
    """The vendor-path implementations timed against the candidates compute the task:
    each agrees with the CPU oracle under the task's gate."""
    from oracle.compare import compare_outputs

    t = kd._tasks()[task]
    sh = kd.parse_shape(shape, t.default)
    args = t.inputs(sh, 3, "cuda")
    got = kd._as_tuple(t.reference(args))
    want = kd._as_tuple(t.oracle(tuple(x.cpu() for x in args)))
    for o, r in zip(got, want):
        snr, _, close = compare_outputs(o, r, atol=t.atol, rtol=t.rtol)
        assert close and snr >= t.snr, (task, snr)
    out = _run([task, "--bench-both", "--shape", shape, "--repeat", "1", "--warmup", "2", "--iters", "8"])
    assert kd.parse(out, t.snr)["passed"], out
