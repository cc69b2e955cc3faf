"""Build libkore_amd.so (gfx950) and the kore_amd._C host extension in-tree.

Every source under ``kore_amd/csrc`` is compiled to an object for gfx950 (in
parallel), then linked into ``kore_amd/libkore_amd.so``.  Objects go to
``kore_amd/_build``.  ``kore_amd/ext/kore_ops.cpp`` (the PyTorch-ROCm operators over
the C ABI) is then compiled against torch into ``kore_amd/_C.so``, linked to
``libkore_amd.so`` through an ``$ORIGIN`` runpath.  Run ``python kore_amd/build.py``
or call :func:`build`.
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
EXT_SRC = PKG / "ext" / "kore_ops.cpp"
EXT = PKG / "_C.so"
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
    build_ext(verbose)
    return LIB


def build_ext(verbose: bool = False) -> Path:
    """Compile the torch host extension kore_amd/_C.so against the built library."""
    import sysconfig

    import torch

    tdir = Path(torch.__file__).resolve().parent
    cxx = os.environ.get("CXX", "g++")
    abi = int(torch.compiled_with_cxx11_abi())
    tmp = EXT.with_suffix(".so.tmp")
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wno-unused-function",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_EXTENSION_NAME=_C",
           "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           f"-I{tdir / 'include'}", f"-I{tdir / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
           "-I/opt/rocm/include", f"-I{sysconfig.get_paths()['include']}", f"-I{PKG.parent / 'include'}",
           str(EXT_SRC), f"-L{tdir / 'lib'}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
           f"-L{PKG}", "-l:libkore_amd.so", "-Wl,-rpath,$ORIGIN", "-o", str(tmp)]
    t0 = time.time()
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("build of kore_amd/_C.so failed")
    os.replace(tmp, EXT)
    if verbose:
        print(f"  compiled _C.so in {time.time() - t0:.1f}s")
    return EXT


if __name__ == "__main__":
    t = time.time()
    path = build(verbose=True)
    print(f"built {path} in {time.time() - t:.1f}s")
