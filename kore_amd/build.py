"""Build libkore_amd.so (gfx950) in-tree with hipcc.

Every source under ``kore_amd/csrc`` is compiled to an object for gfx950 (in
parallel), then linked into ``kore_amd/libkore_amd.so``.  Objects go to
``kore_amd/_build``.  Run ``python -m kore_amd.build`` or call :func:`build`.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libkore_amd.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # packed fp32 VALU ops are kept out of every kernel on this hardware
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{PKG.parent / 'include'}",
]


# Per-source extra flags.  The fp8 block-scaled kernel promotes each MFMA partial
# with VALU FMAs; MFMA results must then live in VGPRs (VALU cannot read AGPRs), so
# that file selects the VGPR form of the MFMA instructions.
EXTRA_FLAGS = {
    "gemm_fp8_blockscale.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def _sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path, verbose: bool) -> tuple[Path, float]:
    obj = BUILD / (src.stem + ".o")
    flags = COMMON_FLAGS + EXTRA_FLAGS.get(src.name, [])
    cmd = [HIPCC, *flags, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd = [HIPCC, *flags, "-x", "hip", "-c", str(src), "-o", str(obj)]
    t0 = time.time()
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed for {src.name}")
    if verbose:
        noisy = [ln for ln in (res.stdout + res.stderr).splitlines()
                 if "packed-fp32-ops" not in ln and ln.strip()]
        if noisy:
            sys.stderr.write("\n".join(noisy) + "\n")
    return obj, time.time() - t0


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc source for gfx950 and link libkore_amd.so; returns its path."""
    if not Path(HIPCC).exists() and shutil.which(HIPCC) is None:
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD.mkdir(exist_ok=True)
    srcs = _sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    objs = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for obj, dt in ex.map(lambda s: _compile(s, verbose), srcs):
            objs.append(obj)
            if verbose:
                print(f"  compiled {obj.name} in {dt:.1f}s")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("link of libkore_amd.so failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    t = time.time()
    path = build(verbose=True)
    print(f"built {path} in {time.time() - t:.1f}s")
