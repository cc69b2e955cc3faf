"""CPU tests of the host side: roofline formulas, comparator semantics, the C ABI
(library loads, exports every declared symbol, validates arguments without a GPU),
and the drop-in ``kernel.py`` candidates (signatures + the reference's static scanner
rules).
"""

from __future__ import annotations

import ast
import ctypes
import math
import re
from pathlib import Path

import pytest
import torch

from kore_amd import roofline as R
from oracle.compare import compare_outputs, compare_pair, snr_db, tolerance_for

ROOT = Path(__file__).resolve().parents[1]


# --------------------------------------------------------------------------- #
# roofline: known-answer vectors restated from the reference's tests
# (tests/test_rooflines.py:14-24, 81-85 and the MoE formula rooflines.py:235-245)
# --------------------------------------------------------------------------- #
def test_roofline_gemm_exact():
    f, q = R.flops_bytes("gemm", {"M": 512, "N": 1024, "K": 2048}, "bf16")
    assert f == 2.0 * 512 * 1024 * 2048
    assert q == (512 * 2048 + 2048 * 1024 + 512 * 1024) * 2


def test_roofline_fp8_bytes_mixed():
    f, q = R.flops_bytes("gemm_fp8", {"M": 256, "N": 256, "K": 256}, "fp8_e4m3fnuz")
    assert f == 2.0 * 256 ** 3
    assert q == (256 * 256 + 256 * 256) * 1 + 256 * 256 * 2


def test_roofline_batched_exact():
    f, q = R.flops_bytes("batched_gemm", {"B": 8, "M": 128, "N": 256, "K": 512}, "bf16")
    assert f == 2.0 * 8 * 128 * 256 * 512
    assert q == 8 * (128 * 512 + 512 * 256 + 128 * 256) * 2


def test_roofline_moe_and_bounds():
    f, q = R.flops_bytes("fused_moe", {"M": 64, "E": 8, "topk": 2, "D": 4096, "I": 14336}, "bf16")
    assert f == 64 * 2 * 6.0 * 4096 * 14336 and q == (8 * 3 * 4096 * 14336 + 2 * 64 * 4096) * 2
    assert R.roofline("fused_moe", {"M": 64, "E": 8, "topk": 2, "D": 4096, "I": 14336}, "bf16").bound == "hbm"
    r = R.roofline("gemm", {"M": 4096, "N": 4096, "K": 4096}, "bf16")
    assert r.bound == "mfma" and math.isclose(r.t_min_s, 2 * 4096 ** 3 / 2.5e15)
    r8 = R.roofline("gemm_fp8", {"M": 2048, "N": 7168, "K": 4096}, "fp8")
    assert math.isclose(r8.t_min_s, 2 * 2048 * 7168 * 4096 / 5e15)


def test_roofline_peak_override(monkeypatch):
    monkeypatch.setenv("KORE_PEAK_HBM_BW", "9.9e12")
    monkeypatch.setenv("KORE_PEAK_FP8", "6.0e15")
    p = R.resolve_peaks()
    assert p["hbm_bytes_per_s"] == 9.9e12 and p["fp8_flops_per_s"] == 6.0e15


# --------------------------------------------------------------------------- #
# comparator semantics (kore/tasks/_genops.py:906-945, kore/verify/equivalence.py:197-253)
# --------------------------------------------------------------------------- #
def test_snr_and_allclose_rules():
    r = torch.tensor([1.0, 2.0, 3.0])
    assert snr_db(r, r) == 999.0
    assert snr_db(r, torch.zeros(3)) == -999.0
    assert compare_outputs(r, r) == (999.0, 0.0, True)
    inf = torch.tensor([1.0, float("inf"), float("nan")])
    assert compare_outputs(inf, inf.clone())[2]                       # matched structure
    assert not compare_outputs(torch.tensor([1.0, -float("inf"), float("nan")]), inf)[2]   # inf sign
    assert not compare_outputs(torch.tensor([1.0, 5.0, float("nan")]), inf)[2]             # position
    s, d, ok = compare_outputs(torch.tensor([1.0, 2.0, 3.02]), r)
    assert ok and abs(d - 0.02) < 1e-6 and 40 < s < 60


def test_four_prong_pair_rule():
    tol = tolerance_for("bf16")
    assert (tol.rtol, tol.atol, tol.snr_db_min) == (3e-2, 1e-2, 30.0)
    e = torch.ones(100)
    assert compare_pair(e, e, tol).ok and compare_pair(e, e, tol).snr_db == math.inf
    bad = e.clone()
    bad[3] = 1.1
    res = compare_pair(bad, e, tol)
    assert not res.ok and "rel-err" in res.reason
    nanc = e.clone()
    nanc[0] = float("nan")
    assert not compare_pair(nanc, e, tol).ok
    assert tolerance_for("fp32").rtol == 3e-3


# --------------------------------------------------------------------------- #
# C ABI: the shared library loads and exports every symbol the header declares
# --------------------------------------------------------------------------- #
HEADER = ROOT / "include" / "kore_amd.h"
LIB = ROOT / "kore_amd" / "libkore_amd.so"


def _declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(kore_\w+)\s*\(", text)))


def test_header_declarations_are_complete():
    names = _declared_functions()
    assert {"kore_gemm", "kore_batched_gemm", "kore_gemm_a8w8_blockscale", "kore_moe_align",
            "kore_fused_moe", "kore_last_error"} <= set(names)


@pytest.fixture(scope="module")
def lib():
    assert LIB.exists(), "libkore_amd.so is not built (python kore_amd/build.py)"
    from kore_amd import _lib

    return _lib.load()


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    from kore_amd import _lib

    assert set(_declared_functions()) == set(_lib.SIGNATURES)
    assert lib.kore_abi_version() == 200


def test_capi_validation_without_gpu(lib):
    """Argument checks run before any HIP call, so they are testable on the CPU."""
    fake = ctypes.c_void_p(256)
    assert lib.kore_gemm(0, 0, fake, 8, 1, fake, 1, 8, None, fake, 8, 0, 8, 8, None, 0, None) == 1   # M = 0
    assert b"M, N, batch >= 1" in lib.kore_last_error()
    assert lib.kore_gemm(0, 9, fake, 8, 1, fake, 1, 8, None, fake, 8, 8, 8, 8, None, 0, None) == 1   # bad act
    assert lib.kore_gemm(7, 0, fake, 8, 1, fake, 1, 8, None, fake, 8, 8, 8, 8, None, 0, None) == 1   # bad dtype
    assert lib.kore_gemm(0, 0, fake, 8, 1, fake, 1, 8, None, None, 8, 8, 8, 8, None, 0, None) == 1   # null C
    assert lib.kore_gemm_workspace_bytes(0, 0, fake, 8, 1, fake, 1, 8, None, fake, 8, 0, 8, 8) == 0
    assert lib.kore_gemm_a8w8_blockscale(fake, 4095, fake, 4095, fake, 32, 1, fake, 32, 1, fake, 128,
                                         16, 128, 4095, None) == 1
    assert b"multiples of 128" in lib.kore_last_error()
    assert lib.kore_moe_align(None, 4, 2, 8, 32, None, None, None, 64, None) == 1
    assert lib.kore_fused_moe(fake, 64, fake, fake, fake, fake, fake, 4, 64, 100, 8, 2, fake, 1 << 30, None) == 2
    assert lib.kore_moe_align_capacity(64, 2, 8, 32) == 384   # align_up(128 + 8*31, 32)
    assert lib.kore_moe_align_capacity(0, 2, 8, 32) == 256
    ws_small = lib.kore_fused_moe_workspace_bytes(64, 2, 8, 4096, 14336)
    ws_big = lib.kore_fused_moe_workspace_bytes(4096, 2, 8, 4096, 14336)
    assert 0 < ws_small < ws_big
    assert lib.kore_fused_moe(fake, 4096, fake, fake, fake, fake, fake, 64, 4096, 14336, 8, 2, fake,
                              ws_small - 1, None) == 4   # workspace too small


def test_gemm_workspace_queries_without_gpu(lib):
    """The workspace a call needs is planned on the host by the same dispatch that
    launches it: zero for the in-place engines (fp32 K tails included), the packed
    operands for a K tail on a grid too small for the bf16 K-tail mode or a transposed
    operand, the split-K partials for a decode-sized M.  A workspace smaller
    than the query fails with KORE_EWORKSPACE before anything is launched."""
    fake = ctypes.c_void_p(256)
    # 4096^3, A and B = W.t() K-contiguous: the engines read both in place
    assert lib.kore_gemm_workspace_bytes(0, 0, fake, 4096, 1, fake, 1, 4096, None, fake, 4096,
                                         4096, 4096, 4096) == 0
    # 512x1024x4095 with the task's [K, N] B: A packed to [512, 4096] bf16, B read in place
    packed = lib.kore_gemm_workspace_bytes(0, 0, fake, 4095, 1, fake, 1024, 1, None, fake, 1024, 512, 1024, 4095)
    assert 512 * 4096 * 2 <= packed <= 512 * 4096 * 2 + 1024
    # the same with B = W.t() (rows of 4095 elements, unaligned): B is packed too
    both = lib.kore_gemm_workspace_bytes(0, 0, fake, 4095, 1, fake, 1, 4095, None, fake, 1024, 512, 1024, 4095)
    assert both >= packed + 1024 * 4096 * 2
    # 1x2048x4096: split K, fp32 partials of the [1, 2048] output per slice
    split = lib.kore_gemm_workspace_bytes(0, 0, fake, 4096, 1, fake, 2048, 1, None, fake, 2048, 1, 2048, 4096)
    assert split > 0 and (split - 256) % (2048 * 4) == 0
    rc = lib.kore_gemm(0, 0, fake, 4095, 1, fake, 1024, 1, None, fake, 1024, 512, 1024, 4095, None, 0, None)
    assert rc == 4 and b"workspace bytes" in lib.kore_last_error()
    # the query leaves room for a 256-byte alignment step; an aligned workspace one byte
    # short of the packed operands is rejected
    rc = lib.kore_gemm(0, 0, fake, 4095, 1, fake, 1024, 1, None, fake, 1024, 512, 1024, 4095, fake, packed - 257, None)
    assert rc == 4
    # fp32 K tail with K-contiguous A: the ring kernel's K-tail mode reads it in place
    assert lib.kore_gemm_workspace_bytes(2, 0, fake, 4095, 1, fake, 1024, 1, None, fake, 1024, 512, 1024, 4095) == 0
    # fp32 with an M-contiguous A (a transposed view) and a K tail: A packed to [M, Kp] fp32
    f32 = lib.kore_gemm_workspace_bytes(2, 0, fake, 1, 512, fake, 1024, 1, None, fake, 1024, 512, 1024, 4095)
    assert f32 >= 512 * 4096 * 4
    # batched with B[i] = [N, K] K-contiguous: in place
    assert lib.kore_batched_gemm_workspace_bytes(0, fake, 1024 * 128, 128, 1, fake, 1024 * 128, 128, 1, fake,
                                                 1024 * 1024, 1024, 64, 1024, 1024, 128) == 0
    # backward: dY^T is read in place as a transposed view; at the task's primary shape
    # both GEMMs run on the in-place buffer engine (no scratch), while a small dW grid
    # packs dY^T [N, M] into the workspace
    assert lib.kore_gemm_backward_workspace_bytes(0, fake, 4096, fake, 4096, fake, 4096, fake, 4096, fake, 4096,
                                                  8192, 4096, 4096) == 0
    bwd = lib.kore_gemm_backward_workspace_bytes(0, fake, 1024, fake, 1024, fake, 1024, fake, 1024, fake, 1024,
                                                 1024, 1024, 1024)
    assert 1024 * 1024 * 2 <= bwd <= 4 * 1024 * 1024 * 2 + 4096
    assert lib.kore_gemm_backward_workspace_bytes(0, fake, 4096, fake, 4096, fake, 4096, fake, 4096, fake, 4096,
                                                  0, 4096, 4096) == 0


# --------------------------------------------------------------------------- #
# drop-in candidates: signatures and the reference's static scanner rules
# (kore/reward/reward.py:70-179, restated)
# --------------------------------------------------------------------------- #
CAND = ROOT / "kore_amd" / "candidates"
SCAN_RULES = [
    r"\b(?:import|from)\s+aiter\b", r"\baiter\.",
    r"\bimport\s+rocblas\b|\bhipblaslt\b|\brocblas\b|\bmiopen\b|\brocsolver\b|\bhipblas\b",
    r"torch\.(matmul|mm|bmm|addmm|baddbmm|einsum|softmax|rms_norm|layer_norm|scaled_dot_product_attention)\s*\(",
    r"torch\.(tensordot|chain_matmul|mv|inner|vdot|dot|kron)\s*\(",
    r"[\w\)\]][^\S\n]*@=", r"torch\.nn\.functional\.\w+\s*\(",
    r"\bF\.(scaled_dot_product_attention|linear|softmax|rms_norm|layer_norm|gelu|silu|conv\w*)\s*\(",
    r"\b(?!tl\.)(?!triton\.)[A-Za-z_]\w*\.(?:matmul|addmm|baddbmm|einsum|scaled_dot_product_attention|softmax|"
    r"log_softmax|gelu|silu|elu|sigmoid|layer_norm|rms_norm|group_norm|batch_norm|linear|conv\w*)\s*\(",
    r"\b(?!tl\.)(?!triton\.)[A-Za-z_]\w*\.(?:bmm|mm)\s*\(",
    r"\bfrom\s+torch(?:\.\w+)*\s+import\b", r"\bimport\s+torch(?:\.\w+)*\s+as\s+\w+",
    r"getattr\s*\(\s*(?:torch|np|numpy|F|nn|aiter|__builtins__|builtins)\b",
    r"\batexit\b|signal\.signal|\bfaulthandler\b|sys\.excepthook|def\s+__del__\b",
    r"\.(flash_attn\w*|fused_moe|paged_attention)\s*\(",
    r"\b(?:import\s+reference|from\s+reference\s+import)\b",
    r"\b(?:reference|ref_program|ref_impl|matmul_ref|\w+_oracle|oracle)\s*\(",
    r"\b(?:import\s+kore\b|from\s+kore\b|kore\.tasks)", r"\b(?:import|from)\s+(?:driver|reference)\b",
    r"\b(?:ref_fn|baseline_fn|matmul_ref)\s*\(", r"\bimportlib\b|__import__\s*\(|\bexec\s*\(|\beval\s*\(",
    r"\bctypes\b|\bcffi\b|\bCDLL\b|dlopen|LoadLibrary", r"(?:SNR|allclose|median_ms|wall_ms)\s*:",
    r"\bsys\.argv\b|\bargparse\b|\bgetopt\b", r"\btime\.sleep\s*\(|\basyncio\.sleep\s*\(",
    r"\bsubprocess\b|\bmultiprocessing\b|\bthreading\b|os\.system|os\.popen|os\.fork",
    r"[\w\)\]][^\S\n]*@[^\S\n]*[\w\(]", r"\bsys\.modules\b", r"\bos\.environ\b|\bos\.getenv\b|\bgetenv\s*\(",
]


def _strip(src: str) -> str:
    src = re.sub(r'("""|\'\'\')(?:.|\n)*?\1', "", src)
    return "\n".join(line.split("#", 1)[0] for line in src.splitlines())


EXPECTED_ENTRIES = {
    "gemm_bf16": ("gemm", 2), "genv_batched_gemm_bf16": ("batched_gemm", 2),
    "moe_batched_gemm_bf16": ("batched_gemm", 2), "gemm_fp8_a8w8_blockscale": ("gemm", 4),
    "genv_gemm_a8w8_blockscale_fp8": ("gemm_a8w8_blockscale", 4),
    "fused_moe_silu_bf16": ("fused_moe", 5),
    # a8w8 with per-row/per-column scales: gemm_fp8_a8w8/driver.py:40 takes ``gemm_fp8``;
    # the _quant_common tasks take ENTRY = "gemm"; vendor_ops.py:742 ``gemm_a8w8``
    "gemm_fp8_a8w8": ("gemm_fp8", 4), "gemm_fp8_a8w8_pertoken": ("gemm", 4),
    "gemm_fp8_a8w8_pertensor": ("gemm", 4), "gemm_int8_a8w8": ("gemm", 4),
    "genv_gemm_a8w8_fp8": ("gemm_a8w8", 4), "genv_gemm_a8w8_int8": ("gemm_a8w8", 4),
    # MoE dispatch stages exposed as tasks (moe_grouped_gemm_bf16/reference.py:25,
    # moe_permute_bf16/reference.py:25; breadth entries are the op names, moe_ext.py:853)
    "moe_grouped_gemm_bf16": ("grouped_gemm", 3), "genb_moe_grouped_gemm_bf16": ("moe_grouped_gemm", 3),
    "moe_grouped_gemm_fp8": ("grouped_gemm_fp8", 5), "genb_moe_grouped_gemm_fp8_fp8": ("moe_grouped_gemm_fp8", 5),
    "moe_permute_bf16": ("moe_permute", 2), "genb_moe_permute_bf16": ("moe_permute", 2),
    "genb_moe_permute_fp16": ("moe_permute", 2), "genb_moe_unpermute_bf16": ("moe_unpermute", 2),
    "genb_moe_unpermute_fp16": ("moe_unpermute", 2),
    "genb_moe_align_block_offsets_bf16": ("moe_align_block_offsets", 3),
    "genb_moe_align_block_offsets_fp16": ("moe_align_block_offsets", 3),
    "genb_moe_expert_offsets_bf16": ("moe_expert_offsets", 2), "genb_moe_expert_offsets_fp16": ("moe_expert_offsets", 2),
    # gemm_backward_bf16/reference.py:22 ENTRY, candidate_grads calls fn(x, w, dy)
    "gemm_backward_bf16": ("gemm_backward", 3),
}


@pytest.mark.parametrize("task", sorted(p.name for p in CAND.iterdir() if p.is_dir() and not p.name.startswith("_")))
def test_candidate_passes_scanner_and_signature(task):
    src = (CAND / task / "kernel.py").read_text()
    code = _strip(src)
    for pat in SCAN_RULES:
        assert not re.search(pat, code), f"{task}: scanner rule {pat!r} fires"
    assert not re.search(r"except\s*[\w. ,()]*:\s*(?:\n\s*)*(?:return|pass|out\s*=)", code)
    tree = ast.parse(src)
    funcs = {n.name: len(n.args.args) for n in tree.body if isinstance(n, ast.FunctionDef)}
    if task in EXPECTED_ENTRIES:
        name, arity = EXPECTED_ENTRIES[task]
    else:  # gen_<op>_<dtype>
        name = task[len("gen_"):].rsplit("_", 1)[0]
        arity = 3 if "bias" in name else 2
    assert funcs.get(name) == arity, (task, funcs)


def test_every_fusion_op_has_candidates():
    import kore_amd

    for op in kore_amd.GEMM_FUSION_OPS:
        for dt in ("bf16", "fp16", "fp32"):
            assert (CAND / f"gen_{op}_{dt}" / "kernel.py").exists()


def test_host_extension_registers_every_operator():
    """The product's host layer is the C++ extension kore_amd._C (over the C ABI): every
    operator is bound on the module and registered as torch.ops.korehip.<op>, with the
    schema the drivers' callables need."""
    import kore_amd
    from kore_amd import _C

    ops = ["gemm", "gemm_fused", "batched_gemm", "gemm_backward", "gemm_a8w8_blockscale", "gemm_a8w8",
           "moe_align", "fused_moe", "grouped_gemm", "grouped_gemm_fp8", "gather_rows", "scatter_rows"]
    for op in ops:
        assert callable(getattr(_C, op)), op
        assert hasattr(torch.ops.korehip, op), op
    assert str(torch.ops.korehip.gemm_fused.default._schema) == \
        "korehip::gemm_fused(Tensor a, Tensor b, Tensor? bias, int act) -> Tensor"
    assert "libkore_amd.so" in open("/proc/self/maps").read()
    assert kore_amd.ops._C is _C


def test_ops_fail_loudly_without_device_tensors():
    import kore_amd

    a = torch.zeros((4, 8), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HIP device"):
        kore_amd.gemm(a, a.t())
    with pytest.raises(ValueError, match="HIP device"):
        torch.ops.korehip.gemm_a8w8_blockscale(a, a, a, a)


def test_registered_grouped_ops_check_shapes_before_the_device():
    """torch.ops.korehip.* can be called without the Python layer: the C++ operators
    check dims, K, dtypes, the number of expert ids, the scale shapes and the rows a
    scatter reads before anything reaches the device.  CPU tensors with a consistent
    shape get as far as the device check."""
    import kore_amd  # noqa: F401  (loads the extension and registers the operators)

    ops = torch.ops.korehip
    bf = torch.bfloat16
    f8 = torch.float8_e4m3fn
    x, w = torch.zeros((8, 64), dtype=bf), torch.zeros((2, 128, 64), dtype=bf)
    ids = torch.zeros(8, dtype=torch.int32)
    with pytest.raises(ValueError, match="one id per row"):
        ops.grouped_gemm(x, w, ids[:5])                       # short expert_ids
    with pytest.raises(ValueError, match="int32"):
        ops.grouped_gemm(x, w, ids.to(torch.int64))
    with pytest.raises(ValueError, match="w\\[E,N,K\\]"):
        ops.grouped_gemm(x, torch.zeros((2, 128, 32), dtype=bf), ids)   # K mismatch
    with pytest.raises(NotImplementedError, match="bf16"):
        ops.grouped_gemm(x.float(), w.float(), ids)
    with pytest.raises(ValueError, match="HIP device"):
        ops.grouped_gemm(x, w, ids)                           # consistent: the device check

    xq, wq = torch.zeros((8, 128), dtype=f8), torch.zeros((2, 128, 128), dtype=f8)
    xs, wsc = torch.ones((8, 1)), torch.ones((2, 128, 1))
    with pytest.raises(ValueError, match="one id per row"):
        ops.grouped_gemm_fp8(xq, wq, xs, wsc, ids[:3])
    with pytest.raises(ValueError, match="x_scale"):
        ops.grouped_gemm_fp8(xq, wq, torch.ones((4, 1)), wsc, ids)       # short x_scale
    with pytest.raises(ValueError, match="x_scale"):
        ops.grouped_gemm_fp8(xq, wq, torch.ones((8, 2)), wsc, ids)       # not a column
    with pytest.raises(ValueError, match="w_scale"):
        ops.grouped_gemm_fp8(xq, wq, xs, torch.ones((2, 64)), ids)
    with pytest.raises(ValueError, match="HIP device"):
        ops.grouped_gemm_fp8(xq, wq, torch.ones((16, 1))[::2], wsc, ids)  # strided x_scale is accepted

    src = torch.zeros((4, 16), dtype=bf)
    with pytest.raises(ValueError, match="one src row per index"):
        ops.scatter_rows(src, torch.arange(6, dtype=torch.int32))
    with pytest.raises(ValueError, match="int32"):
        ops.gather_rows(src, torch.arange(2))
    with pytest.raises(ValueError, match="HIP device"):
        ops.scatter_rows(src, torch.arange(4, dtype=torch.int32))


def test_fake_kernels_trace_every_operator():
    """Every korehip operator has a shape-only kernel, so FakeTensor tracing (the first
    stage of torch.compile) runs without touching data pointers."""
    import kore_amd  # noqa: F401
    from torch.fx.experimental.proxy_tensor import make_fx

    ops = torch.ops.korehip
    bf, f8 = torch.bfloat16, torch.float8_e4m3fn

    def fn(a, b, bias, xq, wq, xs, wsb, ids2, hidden, w1, w2, tw, ti, gx, gw, gid, xsr, wsr, gq, gwq, gws):
        return (ops.gemm(a, b), ops.gemm_fused(a, b, bias, 2), ops.batched_gemm(a[None], b.t()[None]),
                ops.gemm_backward(a, b.t(), ops.gemm(a, b)), ops.gemm_a8w8_blockscale(xq, wq, xs, wsb),
                ops.gemm_a8w8(xq, wq, xsr, wsr), ops.moe_align(ids2, 8, 32),
                ops.fused_moe(hidden, w1, w2, tw, ti), ops.grouped_gemm(gx, gw, gid),
                ops.grouped_gemm_fp8(gq, gwq, xsr, gws, gid), ops.gather_rows(a, gid),
                ops.scatter_rows(a, gid))

    args = (torch.zeros(64, 128, dtype=bf), torch.zeros(128, 256, dtype=bf), torch.zeros(256, dtype=bf),
            torch.zeros(64, 256, dtype=f8), torch.zeros(384, 256, dtype=f8), torch.ones(64, 2),
            torch.ones(3, 2), torch.zeros(64, 2, dtype=torch.int32), torch.zeros(64, 128, dtype=bf),
            torch.zeros(8, 512, 128, dtype=bf), torch.zeros(8, 128, 256, dtype=bf), torch.ones(64, 2),
            torch.zeros(64, 2, dtype=torch.int32), torch.zeros(64, 128, dtype=bf),
            torch.zeros(4, 256, 128, dtype=bf), torch.zeros(64, dtype=torch.int32), torch.ones(64, 1),
            torch.ones(1, 384), torch.zeros(64, 256, dtype=f8), torch.zeros(4, 384, 256, dtype=f8),
            torch.ones(4, 384, 1))
    g = make_fx(fn, tracing_mode="fake")(*args)
    outs = [n for n in g.graph.nodes if n.op == "call_function" and "korehip" in str(n.target)]
    assert len(outs) == 13
    shapes = {str(n.target): n.meta["val"] for n in outs}
    assert tuple(shapes["korehip.gemm_fused.default"].shape) == (64, 256)
    assert shapes["korehip.gemm_a8w8_blockscale.default"].dtype == bf
    assert [tuple(t.shape) for t in shapes["korehip.moe_align.default"]] == [(9,), (384,), (12,)]
    assert tuple(shapes["korehip.grouped_gemm_fp8.default"].shape) == (64, 384)
    assert tuple(shapes["korehip.scatter_rows.default"].shape) == (64, 128)
